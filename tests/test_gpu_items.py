"""The hot path through the drop-in boundary: "tmpl:" items run by ah_run / ah_run_symbolic, and plans
replayed as HIP graphs (tensor.JIT), on the GPU.

- Kernel level: MaxPool2D forward and backward (reduce-path tie split, overlapping first-tie rule, gaps
  between windows) and the fused pool+ReLU backward, bit for bit against ora_maxpool2d on tie-heavy
  inputs (tensor/nn/maxpool_test.go:217-307, tensor/gradient_ruleset.go:307-320); softmax-CE rows with
  tied maxima: an exactly equal share per tied position, values within 2 ulp of ora_softmax_ce.
- Config level: one training step of each BASELINE config as an ExecItem list vs the oracle
  (backend/webgpu/executor.go:26-237, schedule/exec.go:6-32), and plans replayed as graphs vs eager runs.
- Run contract: buffers start at zero (a missing or short leaf input leaves zeros).
"""
import numpy as np
import pytest

import oracle_lib as O
import wgsl_lower as WL
from anneal_amd import _lib as L
from anneal_amd import data, items
from anneal_amd.executor import Buffer, ExecItem, Executor, Plan

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _pool_items(N, C, H, W, kh, kw, sh, sw):
    oH, oW = (H - kh) // sh + 1, (W - kw) // sw + 1
    prm = f"N={N};C={C};H={H};W={W};kh={kh};kw={kw};sh={sh};sw={sw}"
    x, adj = Buffer(1, N * C * H * W, [N, C, H, W]), Buffer(2, N * C * oH * oW, [N, C, oH, oW])
    fwd = ExecItem(f"tmpl:maxpool2d;{prm}", [Buffer(10, N * C * oH * oW, [N, C, oH, oW]), x])
    bwd = ExecItem(f"tmpl:maxpool2d_bwd;{prm}", [Buffer(11, N * C * H * W, [N, C, H, W]), x, adj])
    return [fwd, bwd]


POOL_CASES = [
    # (x values or generator, window, stride): the reference's own tie tables, then tie-heavy windows
    (np.array([3, 3, 1, 2], np.float32).reshape(1, 1, 2, 2), (2, 2), (2, 2)),           # 2-way tie: 0.5/0.5
    (np.array([5, 5, 5, 0, 0, 0, 0, 0, 0], np.float32).reshape(1, 1, 1, 9), (1, 9), (1, 9)),  # 3-way: 1/3
    ("ties", (2, 2), (2, 2)),          # config-2 pooling with 1-, 2-, 3- and 4-way ties (ReLU zeros)
    ("ties", (3, 3), (3, 3)),          # 9-element windows: 1/3, 1/5, 1/7, 1/9 shares
    ("ties", (2, 2), (3, 3)),          # gaps between windows get zero gradient
    ("ties", (3, 3), (2, 2)),          # overlapping windows: the binary Maximum chain, first tie wins
]


@pytest.mark.parametrize("case", range(len(POOL_CASES)))
def test_maxpool_fwd_bwd_bit_exact(dev, case):
    xv, (kh, kw), (sh, sw) = POOL_CASES[case]
    rng = np.random.default_rng(100 + case)
    if isinstance(xv, str):
        x = np.maximum(rng.integers(-3, 3, (3, 5, 14, 14)).astype(np.float32), 0)   # mostly tied zeros
        x[0, 0] = 0.0                                                                 # an all-equal plane
    else:
        x = xv
    N, C, H, W = x.shape
    oH, oW = (H - kh) // sh + 1, (W - kw) // sw + 1
    adj = rng.standard_normal((N, C, oH, oW)).astype(np.float32)
    if not isinstance(xv, str):
        adj[:] = 1.0                                   # the reference's Sum loss: adjoint 1 per window
    want_out, want_gx = O.maxpool2d(x, kh, kw, sh, sw, adj=adj)
    out = Executor(dev).run(_pool_items(N, C, H, W, kh, kw, sh, sw), {1: x.ravel(), 2: adj.ravel()})
    np.testing.assert_array_equal(bits(out[10]), bits(want_out.ravel()))
    np.testing.assert_array_equal(bits(out[11]), bits(want_gx.ravel()))
    if case == 0:
        np.testing.assert_array_equal(out[11], [0.5, 0.5, 0, 0])
    if case == 1:
        np.testing.assert_array_equal(out[11][:3], np.float32(1.0) * (np.float32(1.0) / np.float32(3.0)))


def test_pool_relu_bwd_bit_exact(dev):
    """The fused 2x2 pool backward + ReLU mask of config 2 (tagged activations) vs the oracle's pool
    backward followed by the ReLU rule Where(z == relu(z), adj, 0), on windows with every tie count."""
    rng = np.random.default_rng(7)
    N, C, H = 4, 8, 28
    z = rng.integers(-2, 3, (N, C, H, H)).astype(np.float32) * 0.5     # many equal values, negatives, zeros
    h_ref = np.maximum(z, 0)
    h_tag = np.where(z < 0, np.float32(-0.0), z + np.float32(0.0)).astype(np.float32)   # relu_tag
    p, _ = O.maxpool2d(h_ref, 2, 2, 2, 2, grad=False)
    dp = rng.standard_normal(p.shape).astype(np.float32)
    _, gh = O.maxpool2d(h_ref, 2, 2, 2, 2, adj=dp)
    want = np.where(z == h_ref, gh, np.float32(0))
    item = ExecItem(f"tmpl:pool_relu_bwd;N={N};C={C};H={H}",
                    [Buffer(10, z.size, list(z.shape)), Buffer(1, dp.size, list(dp.shape)),
                     Buffer(2, z.size, list(z.shape)), Buffer(3, p.size, list(p.shape))])
    got = Executor(dev).run([item], {1: dp.ravel(), 2: h_tag.ravel(), 3: p.ravel()})[10]
    np.testing.assert_array_equal(bits(got), bits(want.ravel()))


def test_softmax_ce_tie_rows(dev):
    """Rows whose maximum is tied and whose other logits underflow exp2 to exactly 0 (so every exp2/log2
    is exact in any f32 implementation). The tie split itself is exact: every tied position of a row
    gets bit-identical gradients (the label aside), so each receives the same 1/tie share of the max
    path. The share is formed from a row sum the kernel takes in wave order, where the reference's
    serial loop adds in column order; that moves the last bit, so values are held to 2 ulp of the oracle
    (softmax-CE is a reduction: the 1e-5 relative bar applies)."""
    C = 16
    z = np.full((6, C), -200.0, np.float32)
    z[0, [1, 5]] = 3.0                 # 2-way tie, label elsewhere
    z[1, [0, 2, 9, 11]] = 1.0          # 4-way tie
    z[2, :] = 0.5                      # all 16 tied
    z[3, [0, 2, 4, 6, 8, 10, 12, 14]] = -1.0   # 8-way tie
    z[4, [3, 12]] = 2.0                # 2-way tie, label on a tied position
    z[5, :] = -3.0                     # all tied, negative
    lab = np.array([3, 0, 7, 4, 12, 15], np.int32)
    wl, wdz = O.softmax_ce(z, lab)
    B = z.shape[0]
    item = ExecItem(f"tmpl:softmax_ce;B={B};C={C}", [Buffer(10, B * C, [B, C]), Buffer(1, B * C, [B, C]),
                                                      Buffer(2, B, [B], L.AH_I32), Buffer(11, B, [B])])
    loss_item = ExecItem(f"tmpl:reduce;op=sum;axis=1;M=1;N={B};scale={items.f32_key(-1.0 / B)}",
                         [Buffer(12, 1, [1]), Buffer(11, B, [B])])
    out = Executor(dev).run([item, loss_item], {1: z.ravel(), 2: lab.view(np.float32)})
    dz = out[10].reshape(B, C)
    for r in range(B):
        tied = [c for c in range(C) if z[r, c] == z[r].max() and c != lab[r]]
        assert len(set(bits(dz[r, tied]).tolist())) == 1, r
        assert dz[r, lab[r]] != 0 and np.all(dz[r][(z[r] < z[r].max()) & (np.arange(C) != lab[r])] == 0), r
    ulps = np.abs(bits(dz).astype(np.int64) - bits(wdz).astype(np.int64))
    ulps[np.sign(dz) != np.sign(wdz)] = 1 << 30
    print("softmax-CE tie rows: max ulp distance to the oracle", int(ulps.max()), "elements off:", int((ulps > 0).sum()))
    assert ulps.max() <= 2
    assert abs(out[12][0] - wl) <= 1e-6 * abs(wl)


def test_reduce_template_vs_numpy(dev):
    rng = np.random.default_rng(3)
    M, N = 300, 70
    G = rng.standard_normal((M, N)).astype(np.float32)
    ex = Executor(dev)
    for op, axis in (("sum", 0), ("sum", 1), ("max", 0), ("max", 1), ("sumsq", 0), ("sumsq", 1)):
        n_out = N if axis == 0 else M
        it = ExecItem(f"tmpl:reduce;op={op};axis={axis};M={M};N={N};scale=0.5",
                      [Buffer(10, n_out, [n_out]), Buffer(1, M * N, [M, N])])
        got = ex.run([it], {1: G.ravel()})[10]
        g64 = G.astype(np.float64)
        want = {"sum": 0.5 * g64.sum(axis), "max": g64.max(axis), "sumsq": 0.5 * (g64 * g64).sum(axis)}[op]
        if op == "max":
            np.testing.assert_array_equal(got, want.astype(np.float32))
        else:
            assert O.relerr(got, want) < 1e-5, (op, axis)


def test_run_zeroes_missing_and_short_inputs(dev):
    """Fresh-buffer semantics: a leaf with no input, and the tail of a short input, read as zeros; a
    second run on the same device sees no leftovers."""
    src = r'''
extern "C" __global__ void kernel(float *data0, const float *data1, const float *data2) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < 256) data0[i] = data1[i] * 2.0f + data2[i];
}'''
    it = ExecItem(src, [Buffer(10, 256, [256]), Buffer(1, 256, [256]), Buffer(2, 256, [256])],
                  local_size=(64, 1, 1), workgroup_count=(4, 1, 1))
    ex = Executor(dev)
    full = np.arange(256, dtype=np.float32)
    ex.run([it], {1: full, 2: full})                       # leaves non-zero data behind, if any survived
    got = ex.run([it], {1: full[:100]})                    # short input, no input for uop 2
    want = np.zeros(256, np.float32)
    want[:100] = full[:100] * 2
    np.testing.assert_array_equal(got[10], want)


def check_grads(got, want, tol, keys):
    for k in keys:
        assert O.relerr(np.ravel(got[k]), np.ravel(want[k])) < tol, k


def test_config1_step_as_items_vs_oracle(dev):
    p = data.mlp_ce_inputs(64, 784, 128, 10)
    its, lv, outs = items.mlp_ce(64, 784, 128, 10)
    res = Executor(dev).run(its, items.inputs(lv, p))
    assert set(res) == set(outs.values())
    got = {k: res[u] for k, u in outs.items()}
    wl, g, _ = O.mlp_ce_step(p, 0.01)
    assert abs(got["loss"][0] - wl) <= 1e-4 * max(1, abs(wl))
    check_grads(got, g, 1e-4, ("dW1", "db1", "dW2", "db2"))


def test_config1_sgd_items_update_parameters(dev):
    p = data.mlp_ce_inputs(64, 784, 128, 10)
    its, lv, outs = items.mlp_ce(64, 784, 128, 10, sgd_lr=0.01)
    res = Executor(dev).run(its, items.inputs(lv, p))
    assert set(res) == set(outs.values())
    _, _, new = O.mlp_ce_step(p, 0.01)
    for k in ("W1", "b1", "W2", "b2"):
        step = np.max(np.abs(new[k] - p[k]))
        assert np.max(np.abs(res[outs[k]] - new[k].ravel())) <= 1e-4 * step + 4e-7 * np.max(np.abs(new[k])), k


def test_config2_step_as_items_vs_oracle(dev):
    p = data.convnet_inputs()
    its, lv, outs = items.convnet(32)
    res = Executor(dev).run(its, items.inputs(lv, p))
    assert set(res) == set(outs.values())
    got = {k: res[u] for k, u in outs.items()}
    wl, g, _ = O.convnet_step(p, 0.01)
    assert abs(got["loss"][0] - wl) <= 1e-4 * max(1, abs(wl))
    check_grads(got, g, 1e-4, ("dfb", "dfw", "dcw2", "dcb2", "dcw1", "dcb1"))


def test_config3_small_step_as_items_vs_oracle(dev):
    B, D0, D1, D2, D3 = 256, 128, 256, 256, 128
    p = data.mlp3_inputs(B, D0, D1, D2, D3)
    its, lv, outs = items.mlp3_f16(B, D0, D1, D2, D3)
    res = Executor(dev).run(its, items.inputs(lv, p))      # f16 leaves upload through the codec
    got = {k: res[u] for k, u in outs.items()}
    q = dict(p)
    q["x"], q["t"] = data.f16_quantize(p["x"]), data.f16_quantize(p["t"])
    wl, g, _ = O.mlp3_step(q, 1e-3)
    assert abs(got["loss"][0] - wl) < 2e-2 * abs(wl)
    check_grads(got, g, 2e-2, ("dW1", "db1", "dW2", "db2", "dW3", "db3"))


def test_config5_chain_item_vs_oracle(dev):
    R, Cc = 1024, 512
    p = data.chain_inputs(R, Cc)
    its, lv, outs = items.chain(R, Cc)
    res = Executor(dev).run(its, items.inputs(lv, p))
    wl, wdX, wdg = O.chain_step(p["X"], p["g"])
    assert O.relerr(res[outs["dX"]].reshape(R, Cc), wdX) < 1e-4
    assert O.relerr(res[outs["dg"]], wdg) < 1e-5
    assert abs(res[outs["loss"]][0] - wl) < 1e-5 * abs(wl)


def test_config2_plan_graph_replays_match_eager(dev):
    """A static plan captured once and replayed on new inputs: every replay equals an eager Run."""
    its, lv, outs = items.convnet(32)
    plan = Plan(dev, its, graph=True)
    ex = Executor(dev)
    for seed in (0, 1, 2):
        inp = items.inputs(lv, data.convnet_inputs(seed=seed))
        got, want = plan.run(inp), ex.run(its, inp)
        for u in outs.values():
            np.testing.assert_array_equal(bits(got[u]), bits(want[u]))
    assert plan.stats() == (1, 2)
    plan.close()


@pytest.mark.parametrize("N", [1, 7, 256, 4096])
def test_config4_symbolic_plan_replay_vs_eager_and_reference(dev, N):
    """Config 4 (tensor.JIT over RealizeWithBinding): the item list bound to N through a graph-replayed
    plan equals ah_run_symbolic bit for bit on every replay, and matches the oracle (N <= 256) or its
    float64 closed form (N = 4096, pinned to the oracle on CPU)."""
    its, lv, outs = items.mlp_ce(N, 512, 2048, 512, symbolic=True)
    plan = Plan(dev, its, graph=True)
    ex = Executor(dev)
    for rep in range(3):
        p = data.mlp_ce_inputs(N, 512, 2048, 512, seed=rep, x_lo=-1.0, x_hi=1.0)
        inp = items.inputs(lv, p)
        got = plan.run(inp, {"N": N})
        eager = ex.run_symbolic(its, inp, {"N": N})
        for u in outs.values():
            np.testing.assert_array_equal(bits(got[u]), bits(eager[u]))
    assert plan.stats() == (1, 2)
    res = {k: got[u] for k, u in outs.items()}
    if N <= 256:
        wl, g, _ = O.mlp_ce_step(p, 0.01)
    else:
        from oracle_np import mlp_ce_step_f64, relu_ambiguous_units
        wl, g, _ = mlp_ce_step_f64(p, 0.01)
        amb = relu_ambiguous_units(p)
        assert len(amb) < 128
        res["dW1"] = np.delete(res["dW1"].reshape(2048, 512), amb, 0)
        res["db1"] = np.delete(res["db1"], amb)
        g["dW1"], g["db1"] = np.delete(g["dW1"], amb, 0), np.delete(g["db1"], amb)
    assert abs(res["loss"][0] - wl) <= 1e-4 * max(1, abs(wl))
    check_grads(res, g, 1e-4, ("dW1", "db1", "dW2", "db2"))
    plan.close()


def test_plan_grows_with_the_binding(dev):
    """One symbolic plan run at N = 7, then 256, then 7 again: buffers grow for the larger binding (the
    captured graphs are dropped and captured again) and every result matches an eager run."""
    its, lv, outs = items.mlp_ce(64, 512, 2048, 512, symbolic=True)   # -1/64 baked in; N varies
    plan = Plan(dev, its, graph=True)
    ex = Executor(dev)
    for N in (7, 256, 7):
        inp = items.inputs(lv, data.mlp_ce_inputs(N, 512, 2048, 512, seed=N, x_lo=-1.0, x_hi=1.0))
        got, want = plan.run(inp, {"N": N}), ex.run_symbolic(its, inp, {"N": N})
        for u in outs.values():
            np.testing.assert_array_equal(bits(got[u]), bits(want[u]))
    plan.close()


def test_unknown_template_and_bad_keys_fail_closed(dev):
    ex = Executor(dev)
    for src in ("tmpl:nosuch;M=1", "tmpl:gemm;dtype=f32;epi=store;M=4;N=4", "tmpl:gemm;dtype=f32;epi=mse;M=4;N=4;K=4",
                "tmpl:reduce;op=prod;M=2;N=2", "tmpl:maxpool2d;N=1;C=1;H=2;W=2;kh=3;kw=3;sh=1;sw=1"):
        with pytest.raises(L.AnnealHipError, match="kernel 0"):
            ex.run([ExecItem(src, [Buffer(10, 16, [16]), Buffer(1, 16, [16]), Buffer(2, 16, [16])])], {})


@pytest.mark.parametrize("z_f16", [False, True])
def test_masked_column_sum_template(dev, monkeypatch, z_f16):
    """A ReLU layer's bias gradient, db[n] = Sum_m Where(Z == max(Z, 0), G, 0)[m, n], as the reference's
    lowering renders it (configs 1 and 4 with an f32 Z; config 3 with an f16 Z read widened): the selected
    reduce template with the mask prologue matches float64 at the f32 reduction bar, and the same kernel
    rendered (selection off) to summation order; Z = -0.0 and 0.0 both pass the mask, as Z == max(Z, 0)
    holds for them."""
    from anneal_amd.backend import Device
    if z_f16:
        ks, _, _ = WL.mlp3_step(300, 32, 48, 70, 24)
        name, M, N, ia, iz = "db2", 300, 70, 1, 2
    else:
        ks, _, _ = WL.mlp_ce_step(300, 784, 70, 10)
        name, M, N, ia, iz = "db1", 300, 70, 2, 1
    _, src, bufs, ws, wc, plan = next(k for k in ks if k[0] == name)
    assert L.wgsl_plan(src) == plan and ";pa=mask" in plan
    rng = np.random.default_rng(5)
    G = rng.standard_normal((M, N)).astype(np.float32)
    Z = rng.standard_normal((M, N)).astype(np.float32)
    Z[0, :8] = -0.0
    Z[1, :8] = 0.0
    if z_f16:
        Z = Z.astype(np.float16).astype(np.float32)
    uid = {i: b[0] for i, b in enumerate(bufs)}
    inp = {uid[ia]: G.ravel(), uid[iz]: Z.ravel()}
    item = ExecItem(src, [Buffer(u, n, sh, dtype=dt) for (u, n, dt, sh) in bufs], local_size=ws, workgroup_count=wc)
    got = Executor(dev).run([item], inp)[uid[0]]
    want = np.where(Z >= 0, G.astype(np.float64), 0.0).sum(0)
    assert O.relerr(got, want) < 1e-6
    monkeypatch.setenv("AH_WGSL_TEMPLATES", "0")
    with Device(0) as d2:
        ref = Executor(d2).run([item], inp)[uid[0]]
    assert O.relerr(got, ref) < 1e-6


def test_reduce_template_rejects_bad_mask_keys(dev):
    """The mask prologue is for column sums with its two PARAMs named; anything else fails at plan time."""
    ex = Executor(dev)
    bufs = [Buffer(10, 4, [4]), Buffer(1, 16, [4, 4]), Buffer(2, 16, [4, 4])]
    for key in ("tmpl:reduce;op=sum;axis=1;M=4;N=4;pa=mask;in_a=1;za=2",   # row sums
                "tmpl:reduce;op=max;axis=0;M=4;N=4;pa=mask;in_a=1;za=2",   # max
                "tmpl:reduce;op=sum;axis=0;M=4;N=4;pa=mask;in_a=1;za=1",   # Z is A
                "tmpl:reduce;op=sum;axis=0;M=4;N=4;pa=relu",               # no such prologue
                "tmpl:reduce;op=sum;axis=0;M=4;N=4;wza=1"):                # widening without the mask
        with pytest.raises(L.AnnealHipError):
            ex.run([ExecItem(key, bufs)], {1: np.ones(16, np.float32), 2: np.ones(16, np.float32)})
