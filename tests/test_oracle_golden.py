"""Pins the CPU oracle (oracle/anneal_oracle.c) before it is trusted as the parity reference.

Each oracle function is checked against what the reference's own tests hold (known answers, tie tables,
codec bit patterns) and, where those leave it open, against mathematics that a plausible mistake
(dropped term, wrong sign, transposed operand, wrong tie rule) would break: finite differences of an
independent f64 forward, textbook closed forms, brute force.

Pin map (oracle function -> checks):
  ora_f32_to_f16 / ora_f16_to_f32  -> conversion_test.go:8-116 table; numpy IEEE RTNE on 2^20 finite patterns
  ora_matmul                       -> webgpu_test.go:224-253 [58,64,139,154]; numpy f64
  ora_linear_mse                   -> webgpu_test.go:278-325 loss 2.8625; :445-446 analytic gx, gW; FD
  ora_exp2_sum_grad                -> webgpu_test.go:327-368 ln2*2^x
  ora_maxpool2d                    -> maxpool_test.go:43-129 cases vs brute force (bit-exact);
                                      maxpool_test.go:217-307 tie tables (0.5/0.5, 1/3); FD
  ora_softmax_ce                   -> textbook softmax - onehot; f64 logsumexp loss; tie rows
  ora_mlp_ce_step                  -> FD of an independent f64 forward; SGD update identity
  ora_convnet_step                 -> FD of an independent f64 forward (conv, pool, fc, CE)
  ora_mlp3_f16_step                -> FD of an f64 forward without f16 rounding (tol 2e-2); f16 rounding points
  ora_chain_step                   -> FD of an f64 forward; closed form dg = r * sum(S)
"""
import numpy as np
import pytest

import oracle_lib as O

RNG = np.random.default_rng(1234)


# ── codec ────────────────────────────────────────────────────────────────────

# (f32 bits, f16 bits) from backend/webgpu/conversion_test.go:13-38
CODEC_TABLE = [
    (0x00000000, 0x0000), (0x80000000, 0x8000), (0x3F800000, 0x3C00), (0xBF800000, 0xBC00),
    (0x477FE000, 0x7BFF), (0x38800000, 0x0400), (0x3F801000, 0x3C00), (0x3F802000, 0x3C01),
    (0x3F803000, 0x3C02), (0x3F805000, 0x3C02), (0x33800000, 0x0001), (0x33000000, 0x0000),
    (0x477FF000, 0x7C00), (0x501502F9, 0x7C00), (0x7F800000, 0x7C00), (0x7FC00000, 0x7E00),
    (0x7F800001, 0x7C01),
]


def bits_to_f32(b):
    return float(np.array([b], np.uint32).view(np.float32)[0])


def codec_bits(fn, fbits):
    """Calls an array codec on raw f32 bits (a Python float would quiet a signaling NaN)."""
    src = np.array([fbits], np.uint32).view(np.float32)
    dst = np.zeros(1, np.uint16)
    fn(src.ctypes.data, dst.ctypes.data, 1)
    return int(dst[0])


@pytest.mark.parametrize("fbits,hbits", CODEC_TABLE)
def test_codec_table(fbits, hbits):
    lib = O.load()
    assert codec_bits(lambda s, d, n: lib.ora_f32_to_f16_array(O.C.c_void_p(s), O.C.c_void_p(d), n), fbits) == hbits


def test_codec_widen_table():
    lib = O.load()
    for h, want in [(0x3C00, 0x3F800000), (0x0001, 0x33800000)]:
        got = np.array([lib.ora_f16_to_f32(h)], np.float32).view(np.uint32)[0]
        assert got == want
    assert np.isnan(lib.ora_f16_to_f32(0x7C01))


def test_codec_matches_ieee_rtne_on_random_patterns():
    lib = O.load()
    bits = RNG.integers(0, 2**32, size=1 << 16, dtype=np.uint64).astype(np.uint32)
    f = bits.view(np.float32)
    f = f[np.isfinite(f)]
    want = f.astype(np.float16).view(np.uint16)
    h = np.zeros(f.size, np.uint16)
    lib.ora_f32_to_f16_array(O.fp(np.ascontiguousarray(f)), h.ctypes.data_as(O.C.POINTER(O.C.c_uint16)), f.size)
    np.testing.assert_array_equal(h, want)
    back = np.zeros(f.size, np.float32)
    lib.ora_f16_to_f32_array(h.ctypes.data_as(O.C.POINTER(O.C.c_uint16)), O.fp(back), f.size)
    np.testing.assert_array_equal(back, want.view(np.float16).astype(np.float32))


def test_product_codec_matches_oracle_table():
    """The library's host codec (used for every f16 upload) follows the same table."""
    from anneal_amd import _lib as L
    lib = L.load()
    for fbits, hbits in CODEC_TABLE:
        if (fbits & 0x7F800000) == 0x7F800000 and (fbits & 0x7FFFFF):
            continue  # NaN payloads: covered through the upload path on the GPU
        assert lib.ah_f32_to_f16(bits_to_f32(fbits)) == hbits


# ── primitive known answers ──────────────────────────────────────────────────

def test_matmul_known_answer():
    C = O.matmul(np.array([[1, 2, 3], [4, 5, 6]]), np.array([[7, 8], [9, 10], [11, 12]]))
    np.testing.assert_array_equal(C, [[58, 64], [139, 154]])


def test_matmul_vs_numpy():
    A, B = RNG.standard_normal((17, 33)), RNG.standard_normal((33, 9))
    C = O.matmul(A, B)
    assert O.relerr(C, A.astype(np.float32).astype(np.float64) @ B.astype(np.float32).astype(np.float64)) < 1e-6


MSE_X = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
MSE_W = np.array([[0.1, 0.2], [0.3, 0.4], [0.5, 0.6]], np.float32)
MSE_T = np.array([[1, 2], [3, 4]], np.float32)


def test_mse_forward_known_answer():
    loss, _, _ = O.linear_mse(MSE_X, MSE_W, MSE_T)
    assert abs(loss - 2.8625) < 1e-5


def test_mse_backward_known_answer_and_fd():
    _, gx, gW = O.linear_mse(MSE_X, MSE_W, MSE_T)
    np.testing.assert_allclose(gx.ravel(), [0.14, 0.34, 0.54, 0.335, 0.765, 1.195], atol=1e-5)
    np.testing.assert_allclose(gW.ravel(), [4.4, 5.2, 5.95, 6.8, 7.5, 8.4], atol=1e-5)
    f = lambda x, W: np.mean((x.astype(np.float64) @ W.astype(np.float64) - MSE_T) ** 2)  # noqa: E731
    eps = 1e-3
    for arr, g in ((MSE_X, gx), (MSE_W, gW)):
        fd = np.zeros(arr.size)
        for i in range(arr.size):
            p, m = arr.astype(np.float64).ravel().copy(), arr.astype(np.float64).ravel().copy()
            p[i] += eps
            m[i] -= eps
            if arr is MSE_X:
                fd[i] = (f(p.reshape(arr.shape), MSE_W) - f(m.reshape(arr.shape), MSE_W)) / (2 * eps)
            else:
                fd[i] = (f(MSE_X, p.reshape(arr.shape)) - f(MSE_X, m.reshape(arr.shape))) / (2 * eps)
        np.testing.assert_allclose(g.ravel(), fd, atol=1e-2)


def test_exp2_sum_gradient_known_answer():
    _, g = O.exp2_sum_grad(np.array([0, 1, 2, 3], np.float32))
    np.testing.assert_allclose(g, np.log(2) * np.array([1, 2, 4, 8]), rtol=1e-6)


# ── max-pool ─────────────────────────────────────────────────────────────────

def brute_pool(x, kH, kW, sH, sW):
    N, C, H, W = x.shape
    oH, oW = (H - kH) // sH + 1, (W - kW) // sW + 1
    out = np.zeros((N, C, oH, oW), np.float32)
    for i in range(oH):
        for j in range(oW):
            out[:, :, i, j] = x[:, :, i * sH:i * sH + kH, j * sW:j * sW + kW].max(axis=(2, 3))
    return out


# cases of maxpool_test.go:53-61
POOL_CASES = [(1, 1, 4, 4, 2, 2, 2, 2, False), (1, 1, 4, 4, 2, 2, 1, 1, False), (1, 1, 8, 8, 2, 2, 2, 2, False),
              (1, 1, 8, 8, 4, 4, 4, 4, False), (1, 1, 8, 6, 3, 2, 2, 1, False), (1, 1, 4, 4, 2, 2, 2, 2, True),
              (2, 3, 8, 8, 2, 2, 2, 2, False)]


@pytest.mark.parametrize("case", POOL_CASES)
def test_maxpool_forward_bit_exact(case):
    N, C, H, W, kH, kW, sH, sW, neg = case
    data = np.arange(1, N * C * H * W + 1, dtype=np.float32)
    data = (-data if neg else data).reshape(N, C, H, W)
    out, _ = O.maxpool2d(data, kH, kW, sH, sW, grad=False)
    np.testing.assert_array_equal(out, brute_pool(data, kH, kW, sH, sW))


def test_maxpool_two_way_tie():
    _, g = O.maxpool2d(np.array([3, 3, 1, 2], np.float32).reshape(1, 1, 2, 2), 2, 2, 2, 2)
    np.testing.assert_array_equal(g.ravel(), [0.5, 0.5, 0.0, 0.0])


def test_maxpool_three_way_tie():
    _, g = O.maxpool2d(np.array([5, 5, 5, 0, 0, 0, 0, 0, 0], np.float32).reshape(1, 1, 1, 9), 1, 9, 1, 9)
    np.testing.assert_allclose(g.ravel()[:3], np.float32(1.0) * np.float32(1.0 / 3.0), rtol=0)
    np.testing.assert_array_equal(g.ravel()[3:], 0.0)


@pytest.mark.parametrize("case", [POOL_CASES[0], POOL_CASES[1], POOL_CASES[4], POOL_CASES[6]])
def test_maxpool_backward_fd(case):
    """maxpool_test.go:131-215: FD of L = sum(out^2) on tie-free data."""
    N, C, H, W, kH, kW, sH, sW, _ = case
    x = RNG.permutation(N * C * H * W).astype(np.float32).reshape(N, C, H, W) * 0.1
    out, _ = O.maxpool2d(x, kH, kW, sH, sW, grad=False)
    _, g = O.maxpool2d(x, kH, kW, sH, sW, adj=2 * out)
    eps = 1e-3
    xd = x.astype(np.float64)
    for idx in RNG.choice(x.size, size=min(x.size, 24), replace=False):
        p, m = xd.ravel().copy(), xd.ravel().copy()
        p[idx] += eps
        m[idx] -= eps
        lp = (brute_pool(p.reshape(x.shape), kH, kW, sH, sW).astype(np.float64) ** 2).sum()
        lm = (brute_pool(m.reshape(x.shape), kH, kW, sH, sW).astype(np.float64) ** 2).sum()
        assert abs((lp - lm) / (2 * eps) - g.ravel()[idx]) < 5e-3 * max(1.0, abs(g.ravel()[idx]))


# ── softmax cross-entropy ────────────────────────────────────────────────────

def textbook_ce(z, lab):
    z = z.astype(np.float64)
    m = z.max(1, keepdims=True)
    lse = np.log(np.exp(z - m).sum(1, keepdims=True)) + m
    p = np.exp(z - lse)
    oh = np.eye(z.shape[1])[lab]
    return -(z - lse)[np.arange(len(lab)), lab].mean(), (p - oh) / len(lab)


@pytest.mark.parametrize("B,C", [(64, 10), (7, 512), (1, 3)])
def test_softmax_ce_vs_textbook(B, C):
    z = RNG.standard_normal((B, C)).astype(np.float32) * 3
    lab = RNG.integers(0, C, B).astype(np.int32)
    loss, dz = O.softmax_ce(z, lab)
    wl, wdz = textbook_ce(z, lab)
    assert abs(loss - wl) < 1e-5 * max(1, abs(wl))
    assert O.relerr(dz, wdz) < 1e-5


def test_softmax_ce_ties_at_max():
    z = np.array([[2.0, 2.0, 1.0, 2.0], [0.0, 0.0, 0.0, 0.0]], np.float32)
    lab = np.array([1, 3], np.int32)
    loss, dz = O.softmax_ce(z, lab)
    wl, wdz = textbook_ce(z, lab)
    assert abs(loss - wl) < 1e-6
    assert O.relerr(dz, wdz) < 1e-6


# ── config steps: finite differences of independent f64 forwards ─────────────

def fd_check(lossfn, params: dict, grads: dict, names, n_probe=12, eps=1e-4, tol=5e-3):
    for name in names:
        base = params[name].astype(np.float64)
        g = grads["d" + name].ravel()
        scale = max(np.max(np.abs(g)), 1e-8)
        for idx in RNG.choice(base.size, size=min(base.size, n_probe), replace=False):
            p, m = base.ravel().copy(), base.ravel().copy()
            p[idx] += eps
            m[idx] -= eps
            lp = lossfn({**params, name: p.reshape(base.shape)})
            lm = lossfn({**params, name: m.reshape(base.shape)})
            fd = (lp - lm) / (2 * eps)
            assert abs(fd - g[idx]) <= tol * scale, f"{name}[{idx}]: fd {fd} vs oracle {g[idx]}"


def test_mlp_ce_step_fd_and_sgd():
    from anneal_amd.data import mlp_ce_inputs
    p = mlp_ce_inputs(8, 12, 16, 5, seed=3)
    p["b1"] = RNG.standard_normal(16).astype(np.float32) * 0.1
    p["b2"] = RNG.standard_normal(5).astype(np.float32) * 0.1
    loss, g, new = O.mlp_ce_step(p, lr=0.01)
    lf = lambda q: O.mlp_ce_loss_f64(q["x"], q["labels"], q["W1"], q["b1"], q["W2"], q["b2"])  # noqa: E731
    assert abs(loss - lf(p)) < 1e-5
    fd_check(lf, p, g, ["W1", "b1", "W2", "b2"])
    for k in ("W1", "b1", "W2", "b2"):
        np.testing.assert_array_equal(new[k], (p[k] - np.float32(0.01) * g["d" + k]).astype(np.float32))


def test_convnet_step_fd():
    from anneal_amd.data import convnet_inputs
    p = convnet_inputs(N=2, Hin=8, C1=2, C2=3, NC=4, seed=5)
    for k in ("cb1", "cb2", "fb"):
        p[k] = RNG.standard_normal(p[k].shape).astype(np.float32) * 0.1
    loss, g, _ = O.convnet_step(p, lr=0.01)
    lf = lambda q: O.convnet_loss_f64(q["x"], q["labels"], q["cw1"], q["cb1"], q["cw2"], q["cb2"], q["fw"], q["fb"])  # noqa: E731
    assert abs(loss - lf(p)) < 1e-5
    fd_check(lf, p, g, ["cw1", "cb1", "cw2", "cb2", "fw", "fb"], eps=1e-5)


def test_mlp3_f16_step_fd():
    from anneal_amd.data import f16_quantize, mlp3_inputs
    p = mlp3_inputs(B=16, D0=8, D1=16, D2=12, D3=6, seed=7)
    p["x"], p["t"] = f16_quantize(p["x"]), f16_quantize(p["t"])
    q = {k: (f16_quantize(v) if k[0] in "Wb" else v) for k, v in p.items()}
    loss, g, _ = O.mlp3_step(p, lr=1e-3)
    lf = lambda r: O.mlp3_loss_f64(r["x"], r["t"], r["W1"], r["b1"], r["W2"], r["b2"], r["W3"], r["b3"])  # noqa: E731
    assert abs(loss - lf(q)) < 2e-2 * lf(q)
    fd_check(lf, q, g, ["W1", "b1", "W2", "b2", "W3", "b3"], eps=1e-3, tol=2e-2)


def test_mlp3_loss_narrows_to_f16():
    """The f16 Sum narrows its f32 accumulator (codegen/lower.go:712): a sum above 65504 becomes +Inf."""
    from anneal_amd.data import mlp3_inputs
    p = mlp3_inputs(B=64, D0=8, D1=8, D2=8, D3=1100, seed=9)
    p["t"] = np.full_like(p["t"], 8.0)
    loss, g, _ = O.mlp3_step(p, lr=1e-3)
    assert np.isinf(loss)
    assert np.all(np.isfinite(g["dW3"]))


def test_chain_step_fd_and_closed_form():
    X = RNG.standard_normal((16, 8)).astype(np.float32)
    g = (1 + 0.02 * RNG.standard_normal(8)).astype(np.float32)
    loss, dX, dg = O.chain_step(X, g)
    assert abs(loss - O.chain_loss_f64(X, g)) < 1e-5 * abs(loss)
    Y = X.T.astype(np.float64)
    S = np.exp(Y - Y.max(1, keepdims=True))
    S /= S.sum(1, keepdims=True)
    r = 1 / np.sqrt((S * S).mean(1) + 1e-6)
    assert O.relerr(dg, r * S.sum(1)) < 1e-5
    fd_check(lambda q: O.chain_loss_f64(q["X"], q["g"]), {"X": X, "g": g}, {"dX": dX, "dg": dg}, ["X", "g"],
             n_probe=24, eps=1e-4, tol=1e-3)


def test_chain_step_tie_rows():
    """Rows with a repeated maximum still differentiate to the textbook gradient (tie split of a zero sum)."""
    X = RNG.standard_normal((12, 4)).astype(np.float32)
    X[3, :] = 5.0
    X[7, :] = 5.0
    g = np.ones(4, np.float32)
    _, dX, _ = O.chain_step(X, g)
    fd_check(lambda q: O.chain_loss_f64(q["X"], q["g"]), {"X": X, "g": g}, {"dX": dX, "dg": np.zeros(4)}, ["X"],
             n_probe=24, eps=1e-5, tol=2e-3)


def test_oracle_np_matches_c_oracle():
    """The blocked numpy restatement used for full-size config-3 parity equals the C oracle at small
    sizes (only f32 summation order differs)."""
    from anneal_amd import data
    from oracle_np import mlp3_step_np
    p = data.mlp3_inputs(96, 64, 128, 96, 32, seed=5)
    p["b1"] = (0.1 * RNG.standard_normal(128)).astype(np.float32)
    q = dict(p)
    q["x"], q["t"] = data.f16_quantize(p["x"]), data.f16_quantize(p["t"])
    wl, g, new = O.mlp3_step(q, 1e-3)
    nl, ng, nnew = mlp3_step_np(q, 1e-3)
    assert abs(nl - wl) <= 1e-3 * abs(wl)
    for k in g:
        assert O.relerr(ng[k], g[k]) < 2e-3, k
    for k in new:
        assert np.max(np.abs(nnew[k] - new[k])) <= 1e-6 * max(1.0, np.max(np.abs(new[k]))), k


def test_chain_closed_form_f64_matches_oracle():
    """The f64 closed form used to judge column-max elements at full size agrees with the oracle on
    every other element (and the tie-free mathematics: d loss / d X sums to zero per column)."""
    from oracle_np import chain_dX_f64
    X = RNG.standard_normal((512, 96)).astype(np.float32)
    g = (1 + 0.02 * RNG.standard_normal(96)).astype(np.float32)
    _, wdX, _ = O.chain_step(X, g)
    ex = chain_dX_f64(X, g)
    mask = np.zeros(X.shape, bool)
    mask[X.argmax(0), np.arange(96)] = True
    assert np.max(np.abs(wdX - ex)[~mask]) / np.max(np.abs(ex)) < 1e-5
    assert np.max(np.abs(ex.sum(0))) < 1e-12 * X.shape[0]


@pytest.mark.parametrize("B,D,H,Cn", [(64, 784, 128, 10), (256, 512, 2048, 512)])
def test_mlp_ce_f64_closed_form_matches_c_oracle(B, D, H, Cn):
    """The float64 closed form used for config 4 at N = 4096 agrees with the C oracle where the oracle is
    fast (its f32 rounding is the only difference)."""
    from anneal_amd import data
    from oracle_np import mlp_ce_step_f64
    p = data.mlp_ce_inputs(B, D, H, Cn, seed=11, x_lo=-1.0, x_hi=1.0)
    wl, g, new = O.mlp_ce_step(p, 0.01)
    fl, fg, fnew = mlp_ce_step_f64(p, 0.01)
    assert abs(fl - wl) <= 1e-5 * max(1.0, abs(wl))
    for k in g:
        assert O.relerr(g[k], fg[k]) < 1e-5, k


def test_mlp_ce_grads_given_hidden_reduces_to_closed_form():
    """With the exact hidden layer relu(Z1) (dead units tagged -0.0), the conditioned backward equals the
    float64 closed form; flipping one live unit's tag to dead removes exactly that unit's row of dZ1
    from dW1 and db1 for that sample."""
    from anneal_amd import data
    from oracle_np import mlp_ce_grads_given_hidden_f64, mlp_ce_step_f64
    p = data.mlp_ce_inputs(96, 64, 48, 10, seed=5, x_lo=-1.0, x_hi=1.0)
    Z1 = np.asarray(p["x"], np.float64) @ np.asarray(p["W1"], np.float64).T + np.asarray(p["b1"], np.float64)
    H1 = np.where(Z1 < 0, np.float32(-0.0), Z1.astype(np.float32)).astype(np.float32)
    fl, fg, _ = mlp_ce_step_f64(p, 0.01)
    gl, gg = mlp_ce_grads_given_hidden_f64(p, H1)
    assert abs(gl - fl) < 1e-6
    for k in fg:
        assert O.relerr(gg[k], fg[k]) < 1e-6, k
    n, j = np.argwhere(Z1 > 0.1)[0]
    H2 = H1.copy()
    H2[n, j] = np.float32(-0.0)          # the mask now drops (n, j); the forward sees 0 there
    _, g2 = mlp_ce_grads_given_hidden_f64(p, H2)
    H3 = H1.copy()
    H3[n, j] = np.float32(0.0)           # same forward value, unit alive
    _, g3 = mlp_ce_grads_given_hidden_f64(p, H3)
    # the two differ only in the (n, j) term of dZ1: dW1[j] by dZ1[n, j] * x[n], db1[j] by dZ1[n, j]
    dz1 = g3["db1"][j] - g2["db1"][j]
    assert dz1 != 0
    np.testing.assert_allclose(g3["dW1"][j] - g2["dW1"][j], dz1 * np.asarray(p["x"], np.float64)[n], rtol=1e-9, atol=1e-15)
    rows = np.arange(48) != j
    np.testing.assert_array_equal(g3["dW1"][rows], g2["dW1"][rows])
