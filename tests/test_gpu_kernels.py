"""Kernel-level parity of the HIP hot path against the oracle / f64 restatements (GPU).

Tolerances: f32 contractions and reductions 1e-4 norm-wise relative error
(max|a-b| / max|b|); f16 outputs within one f16 ulp of the f64-accumulated value rounded at the same
points; index/tie work bit-exact.
"""
import numpy as np
import pytest

import oracle_lib as O
from anneal_amd import _lib as L

pytestmark = pytest.mark.gpu
RNG = np.random.default_rng(99)


def q16(a):
    return np.asarray(a, np.float32).astype(np.float16).astype(np.float32)


def store_operand(X, trans):
    return np.ascontiguousarray(X.T if trans else X)


GEMM_CASES = [
    # dtype, ta, tb, M, N, K, tile
    (L.AH_F32, 0, 0, 64, 128, 784, 0), (L.AH_F32, 0, 1, 64, 128, 10, 0), (L.AH_F32, 1, 1, 10, 128, 64, 0),
    (L.AH_F32, 1, 0, 70, 33, 37, 64), (L.AH_F32, 0, 0, 300, 260, 130, 128), (L.AH_F32, 1, 1, 256, 256, 96, 256),
    (L.AH_F16, 0, 0, 256, 256, 256, 0), (L.AH_F16, 0, 1, 130, 200, 72, 64), (L.AH_F16, 1, 1, 96, 160, 300, 128),
    (L.AH_F16, 1, 0, 512, 512, 128, 256), (L.AH_F16, 0, 0, 33, 17, 24, 64),
]


@pytest.mark.parametrize("case", GEMM_CASES, ids=lambda c: "dt%d_ta%d_tb%d_%dx%dx%d_t%d" % c)
def test_gemm_store_and_bias_relu(dev, case):
    dt, ta, tb, M, N, K, tile = case
    A = RNG.standard_normal((M, K)).astype(np.float32)
    B = RNG.standard_normal((N, K)).astype(np.float32)
    bias = RNG.standard_normal(N).astype(np.float32)
    if dt == L.AH_F16:
        A, B, bias = q16(A), q16(B), q16(bias)
    ref = A.astype(np.float64) @ B.astype(np.float64).T
    As, Bs = store_operand(A, ta), store_operand(B, tb)
    npdt = np.float16 if dt == L.AH_F16 else np.float32
    dA, dB = dev.buffer(As.astype(npdt), dt), dev.buffer(Bs.astype(npdt), dt)
    dbias = dev.buffer(bias.astype(npdt), dt)
    dC = dev.buffer(M * N, dt)
    common = dict(dtype=dt, ta=ta, tb=tb, M=M, N=N, K=K, A=dA, B=dB, lda=As.shape[1], ldb=Bs.shape[1], C_out=dC,
                  ldc=N, tile=tile)
    dev.gemm(epi=L.EPI_STORE, scale=0.5, **common)
    C = dC.read().astype(np.float32).reshape(M, N)
    if dt == L.AH_F32:
        assert O.relerr(C, 0.5 * ref) < 1e-5
    else:
        np.testing.assert_allclose(C, q16(0.5 * ref), rtol=2e-3, atol=2e-3 * np.abs(ref).max())
    dev.gemm(epi=L.EPI_BIAS_RELU, bias=dbias, **common)
    H = dC.read().astype(np.float32).reshape(M, N)
    if dt == L.AH_F32:
        z = ref + bias
        assert O.relerr(H, np.maximum(z, 0)) < 1e-5
    else:
        z = q16(q16(ref) + bias)
        np.testing.assert_allclose(H, np.maximum(z, 0), rtol=2e-3, atol=2e-3 * np.abs(z).max())
    dead = np.signbit(H) & (H == 0)
    assert np.array_equal(dead, z < 0), "ReLU tag (-0 for z<0) mismatch"
    for b in (dA, dB, dbias, dC):
        b.free()


@pytest.mark.parametrize("dt", [L.AH_F32, L.AH_F16])
def test_gemm_mask_colsum_and_sgd(dev, dt):
    M, N, K = 192, 160, 96
    npdt = np.float16 if dt == L.AH_F16 else np.float32
    A = RNG.standard_normal((M, K)).astype(np.float32)
    Bm = RNG.standard_normal((K, N)).astype(np.float32)       # stored [K,N] (tb = 1)
    if dt == L.AH_F16:
        A, Bm = q16(A), q16(Bm)
    Hact = RNG.standard_normal((M, N)).astype(np.float32)
    Hact = np.where(Hact < 0, np.float32(-0.0), Hact).astype(npdt)
    ref = A.astype(np.float64) @ Bm.astype(np.float64)
    masked = np.where(np.signbit(Hact.astype(np.float32)) & (Hact == 0), 0.0, 2.0 * ref)
    dA, dB, dH = dev.buffer(A.astype(npdt), dt), dev.buffer(Bm.astype(npdt), dt), dev.buffer(Hact, dt)
    dC = dev.buffer(M * N, dt)
    cs = dev.buffer(np.zeros(N, np.float32), L.AH_F32)
    dev.gemm(dtype=dt, epi=L.EPI_MASK, ta=0, tb=1, M=M, N=N, K=K, A=dA, B=dB, lda=K, ldb=N, C_out=dC, ldc=N,
             aux=dH, ldaux=N, scale=2.0, colsum=cs)
    C = dC.read().astype(np.float32).reshape(M, N)
    tol = 1e-5 if dt == L.AH_F32 else 2e-3
    assert O.relerr(C, masked) < tol
    assert O.relerr(cs.read(), masked.sum(0)) < 1e-4
    # SGD epilogue: W -= lr * (scale * A^T-contraction); dW[n,k] = sum_m G[m,n] X[m,k]
    G, X = A, RNG.standard_normal((M, 48)).astype(np.float32)
    if dt == L.AH_F16:
        X = q16(X)
    W = RNG.standard_normal((K, 48)).astype(np.float32)
    dG, dX = dev.buffer(G.astype(npdt), dt), dev.buffer(X.astype(npdt), dt)
    dW, dg = dev.buffer(W, L.AH_F32), dev.buffer(K * 48, L.AH_F32)
    dW16 = dev.buffer(K * 48, L.AH_F16)
    dev.gemm(dtype=dt, epi=L.EPI_SGD, ta=1, tb=1, M=K, N=48, K=M, A=dG, B=dX, lda=K, ldb=48, ldc=48, scale=0.25,
             W32=dW, W16=dW16, lr=0.1, gout=dg)
    gref = 0.25 * (G.astype(np.float64).T @ X.astype(np.float64))
    assert O.relerr(dg.read().reshape(K, 48), gref) < (1e-5 if dt == L.AH_F32 else 1e-4)
    Wn = dW.read().reshape(K, 48)
    assert O.relerr(Wn - W, -0.1 * gref) < 1e-4
    np.testing.assert_array_equal(dW16.read(), Wn.astype(np.float16).ravel())


def test_gemm_mse_epilogue(dev):
    M, N, K = 128, 96, 64
    A, B = q16(RNG.standard_normal((M, K))), q16(RNG.standard_normal((N, K)) * 0.2)
    bias, T = q16(RNG.standard_normal(N) * 0.1), q16(RNG.standard_normal((M, N)))
    dA, dB = dev.buffer(A.astype(np.float16), L.AH_F16), dev.buffer(B.astype(np.float16), L.AH_F16)
    db, dT = dev.buffer(bias.astype(np.float16), L.AH_F16), dev.buffer(T.astype(np.float16), L.AH_F16)
    dD = dev.buffer(M * N, L.AH_F16)
    cs, la = dev.buffer(np.zeros(N, np.float32), L.AH_F32), dev.buffer(np.zeros(1, np.float32), L.AH_F32)
    dev.gemm(dtype=L.AH_F16, epi=L.EPI_MSE, ta=0, tb=0, M=M, N=N, K=K, A=dA, B=dB, lda=K, ldb=K, C_out=dD, ldc=N,
             bias=db, aux=dT, ldaux=N, colsum=cs, lossacc=la)
    P = q16(q16(A.astype(np.float64) @ B.astype(np.float64).T) + bias)
    d = q16(P - T)
    got = dD.read().astype(np.float32).reshape(M, N)
    assert np.mean(got == d) > 0.99 and O.relerr(got, d) < 2e-3
    assert O.relerr(cs.read(), d.astype(np.float64).sum(0)) < 1e-3
    assert abs(la.read()[0] - ((P - T).astype(np.float64) ** 2).sum()) < 1e-3 * ((P - T) ** 2).sum()


@pytest.mark.parametrize("B,C", [(64, 10), (7, 512), (4096, 512), (3, 1)])
def test_softmax_ce_kernel(dev, B, C):
    z = (RNG.standard_normal((B, C)) * 3).astype(np.float32)
    z[0, : min(C, 3)] = z[0].max() + 1.0          # a tied maximum
    lab = RNG.integers(0, C, B).astype(np.int32)
    wl, wdz = O.softmax_ce(z, lab)
    dz_, dl_, dd, dloss = dev.buffer(z), dev.buffer(lab, L.AH_I32), dev.buffer(B * C), dev.buffer(1)
    dev.softmax_ce(dz_, dl_, B, C, dd, dloss)
    assert O.relerr(dd.read().reshape(B, C), wdz) < 1e-5
    assert abs(dloss.read()[0] - wl) <= 1e-5 * max(1.0, abs(wl))


# (4096, 256), (8192, 64) and (8192, 528): the column-strip kernel that holds X on chip; the others: the
# three-kernel chain
@pytest.mark.parametrize("R,Cc,grow", [(64, 32, False), (257, 260, False), (1024, 512, False), (4096, 256, False),
                                       (8192, 64, False), (8192, 528, False), (4096, 256, True), (8192, 64, True)])
def test_chain_kernel_vs_oracle(dev, R, Cc, grow):
    """grow: half the columns jump by +50 in their second half of rows, far above the maximum of the
    rows the strip kernel's threads take their provisional max from (it then re-bases its sums)."""
    X = RNG.standard_normal((R, Cc)).astype(np.float32)
    if grow:
        X[R // 2:, : Cc // 2] += 50.0
    X[5, :] = X.max() + 0.5                             # every row of Y gets a tie candidate
    X[9, :] = X[5, :]
    g = (1 + 0.02 * RNG.standard_normal(Cc)).astype(np.float32)
    wl, wdX, wdg = O.chain_step(X, g)
    dXb, dgb, dX, dg, dl = dev.buffer(X), dev.buffer(g), dev.buffer(R * Cc), dev.buffer(Cc), dev.buffer(1)
    dev.chain_step(dXb, dgb, R, Cc, dX, dg, dl)
    # Each column's max elements carry the max-path tie share, zero in exact arithmetic and a rounding
    # residue in any f32 evaluation (it depends on how sum e was rounded): those are judged against the
    # float64 closed form, no further from it than the oracle is (plus 1e-4); the rest against the oracle.
    from oracle_np import chain_dX_f64
    got = dX.read().reshape(R, Cc)
    exact = chain_dX_f64(X, g)
    mask = X == X.max(0, keepdims=True)
    den = np.max(np.abs(wdX))
    assert np.max(np.abs(got - wdX)[~mask]) / den < 1e-4
    assert np.max(np.abs(got - exact)[mask]) / den <= np.max(np.abs(wdX - exact)[mask]) / den + 1e-4
    assert O.relerr(dg.read(), wdg) < 1e-5
    assert abs(dl.read()[0] - wl) < 1e-5 * abs(wl)
    for b in (dXb, dgb, dX, dg, dl):
        b.free()


F16_VARIANTS = list(range(1, 40))   # every gemm16 variant (gemm16_kernel.h Var<V>; 32-39 use 16x16x32 MFMAs)
KGROUP_VARIANTS = (10, 11, 15, 25, 28, 31, 35, 36, 37, 38)   # variants that add two k-halves
VARIANT_SHAPES = [
    # ta, tb, M, N, K: full tiles, ragged edges (scalar epilogue), short K, both layouts
    (0, 0, 512, 512, 192), (0, 1, 520, 300, 128), (1, 1, 264, 520, 64), (1, 0, 256, 256, 320),
    (0, 0, 384, 640, 512), (1, 1, 264, 256, 256),      # K in whole stage pairs: the k-group variants run
]


@pytest.mark.parametrize("variant", F16_VARIANTS)
@pytest.mark.parametrize("shape", VARIANT_SHAPES, ids=lambda s: "ta%d_tb%d_%dx%dx%d" % s)
def test_gemm16_variants_store_mask_sgd(dev, variant, shape):
    """Every f16 kernel variant (tile, wave layout, fetch mode) against an f64 contraction of the
    same f16 operands, through the STORE, MASK+colsum and SGD epilogues."""
    ta, tb, M, N, K = shape
    A = q16(RNG.standard_normal((M, K)))
    B = q16(RNG.standard_normal((N, K)))
    ref = A.astype(np.float64) @ B.astype(np.float64).T
    As, Bs = store_operand(A, ta), store_operand(B, tb)
    dA, dB = dev.buffer(As.astype(np.float16), L.AH_F16), dev.buffer(Bs.astype(np.float16), L.AH_F16)
    dC = dev.buffer(M * N, L.AH_F16)
    common = dict(dtype=L.AH_F16, ta=ta, tb=tb, M=M, N=N, K=K, A=dA, B=dB, lda=As.shape[1], ldb=Bs.shape[1],
                  ldc=N, variant=variant)
    dev.gemm(epi=L.EPI_STORE, scale=1.0, C_out=dC, **common)
    C = dC.read().astype(np.float32).reshape(M, N)
    np.testing.assert_allclose(C, q16(ref), rtol=2e-3, atol=2e-3 * np.abs(ref).max())
    Hact = RNG.standard_normal((M, N)).astype(np.float32)
    Hact = np.where(Hact < 0, np.float32(-0.0), Hact).astype(np.float16)
    dH = dev.buffer(Hact, L.AH_F16)
    cs = dev.buffer(np.zeros(N, np.float32), L.AH_F32)
    dev.gemm(epi=L.EPI_MASK, scale=0.5, C_out=dC, aux=dH, ldaux=N, colsum=cs, **common)
    masked = np.where(np.signbit(Hact.astype(np.float32)) & (Hact == 0), 0.0, 0.5 * ref)
    assert O.relerr(dC.read().astype(np.float32).reshape(M, N), masked) < 2e-3
    assert O.relerr(cs.read(), masked.sum(0)) < 1e-4
    W = RNG.standard_normal((M, N)).astype(np.float32)
    dW, dg, dW16 = dev.buffer(W, L.AH_F32), dev.buffer(M * N, L.AH_F32), dev.buffer(M * N, L.AH_F16)
    dev.gemm(epi=L.EPI_SGD, scale=0.25, W32=dW, W16=dW16, lr=0.1, gout=dg, **common)
    assert O.relerr(dg.read().reshape(M, N), 0.25 * ref) < 1e-5
    Wn = dW.read().reshape(M, N)
    assert O.relerr(Wn - W, -0.025 * ref) < 1e-4
    np.testing.assert_array_equal(dW16.read(), Wn.astype(np.float16).ravel())
    for b in (dA, dB, dC, dH, cs, dW, dg, dW16):
        b.free()


@pytest.mark.parametrize("shape", [(0, 0, 512, 384, 256), (1, 1, 256, 512, 192), (0, 1, 300, 260, 128)],
                         ids=lambda s: "ta%d_tb%d_%dx%dx%d" % s)
def test_gemm16_variants_bit_identical_and_tune(dev, shape):
    """Variants without k-groups accumulate each output over k in the same order, so their results are
    bit-identical; k-group variants add two k-halves (f32 rounding differs, 1e-6 relative). The tuner
    picks one variant, caches it, and variant-0 launches reproduce that variant's result."""
    ta, tb, M, N, K = shape
    A, B = q16(RNG.standard_normal((M, K))), q16(RNG.standard_normal((N, K)))
    As, Bs = store_operand(A, ta), store_operand(B, tb)
    dA, dB = dev.buffer(As.astype(np.float16), L.AH_F16), dev.buffer(Bs.astype(np.float16), L.AH_F16)
    dC = dev.buffer(M * N, L.AH_F32)
    dW = dev.buffer(np.zeros(M * N, np.float32))
    common = dict(dtype=L.AH_F16, ta=ta, tb=tb, M=M, N=N, K=K, A=dA, B=dB, lda=As.shape[1], ldb=Bs.shape[1], ldc=N)
    outs = []
    for v in F16_VARIANTS:
        dW.write(np.zeros(M * N, np.float32))
        dev.gemm(epi=L.EPI_SGD, scale=1.0, W32=dW, lr=-1.0, variant=v, **common)   # W = 0 + acc, exact f32
        outs.append(dW.read())
    for v, o in zip(F16_VARIANTS, outs):
        if v in KGROUP_VARIANTS:
            assert O.relerr(o, outs[0]) < 1e-6, v      # two k-halves added: different f32 rounding
        else:
            np.testing.assert_array_equal(o.view(np.uint32), outs[0].view(np.uint32), err_msg=f"variant {v}")
    best, us = dev.gemm_tune(iterations=2, epi=L.EPI_SGD, scale=1.0, W32=dW, lr=-1.0, **common)
    assert best in F16_VARIANTS and us > 0
    dW.write(np.zeros(M * N, np.float32))
    dev.gemm(epi=L.EPI_SGD, scale=1.0, W32=dW, lr=-1.0, **common)
    np.testing.assert_array_equal(dW.read().view(np.uint32), outs[best - 1].view(np.uint32))
    for b in (dA, dB, dC, dW):
        b.free()


@pytest.mark.parametrize("dt", [L.AH_F32, L.AH_F16])
def test_gemm_dot_path_epilogues(dev, dt):
    """Few outputs with a long K (M*N <= 16384, K >= 256, A and B K-contiguous) take the
    wave-per-output path: bias+ReLU, mask+colsum and SGD epilogues against f64."""
    M, N, K = 24, 40, 300
    npdt = np.float16 if dt == L.AH_F16 else np.float32
    A, B = RNG.standard_normal((M, K)).astype(np.float32), RNG.standard_normal((N, K)).astype(np.float32)
    bias = RNG.standard_normal(N).astype(np.float32)
    if dt == L.AH_F16:
        A, B, bias = q16(A), q16(B), q16(bias)
    ref = A.astype(np.float64) @ B.astype(np.float64).T
    dA, dB, db = dev.buffer(A.astype(npdt), dt), dev.buffer(B.astype(npdt), dt), dev.buffer(bias.astype(npdt), dt)
    dC = dev.buffer(M * N, dt)
    common = dict(dtype=dt, ta=0, tb=0, M=M, N=N, K=K, A=dA, B=dB, lda=K, ldb=K, ldc=N)
    dev.gemm(epi=L.EPI_BIAS_RELU, bias=db, C_out=dC, **common)
    H = dC.read().astype(np.float32).reshape(M, N)
    z = ref + bias if dt == L.AH_F32 else q16(q16(ref) + bias)
    tol = 1e-5 if dt == L.AH_F32 else 2e-3
    assert O.relerr(H, np.maximum(z, 0)) < tol
    assert np.array_equal(np.signbit(H) & (H == 0), z < 0)
    Hact = np.where(RNG.standard_normal((M, N)) < 0, np.float32(-0.0), np.float32(1.0)).astype(npdt)
    dH, cs = dev.buffer(Hact, dt), dev.buffer(np.zeros(N, np.float32))
    dev.gemm(epi=L.EPI_MASK, scale=0.5, aux=dH, ldaux=N, colsum=cs, C_out=dC, **common)
    masked = np.where(np.signbit(Hact.astype(np.float32)), 0.0, 0.5 * ref)
    assert O.relerr(dC.read().astype(np.float32).reshape(M, N), masked) < tol
    assert O.relerr(cs.read(), masked.sum(0)) < 1e-4
    W = RNG.standard_normal((M, N)).astype(np.float32)
    dW, dg = dev.buffer(W), dev.buffer(M * N)
    dev.gemm(epi=L.EPI_SGD, scale=0.25, W32=dW, lr=0.1, gout=dg, **common)
    assert O.relerr(dg.read().reshape(M, N), 0.25 * ref) < 1e-5
    assert O.relerr(dW.read().reshape(M, N) - W, -0.025 * ref) < 1e-4
    for b in (dA, dB, db, dC, dH, cs, dW, dg):
        b.free()


def test_gemm_tune_disk_cache(dev, tmp_path):
    """Tuned choices survive a save/load through the disk cache, and a malformed file is rejected."""
    M, N, K = 256, 256, 128
    A, B = q16(RNG.standard_normal((M, K))), q16(RNG.standard_normal((N, K)))
    dA, dB = dev.buffer(A.astype(np.float16), L.AH_F16), dev.buffer(B.astype(np.float16), L.AH_F16)
    dC = dev.buffer(M * N, L.AH_F16)
    best, _ = dev.gemm_tune(iterations=1, dtype=L.AH_F16, epi=L.EPI_STORE, ta=0, tb=0, M=M, N=N, K=K, A=dA, B=dB,
                            lda=K, ldb=K, C_out=dC, ldc=N)
    path = tmp_path / "tune.txt"
    dev.gemm_tune_cache(str(path), True)
    lines = path.read_text().splitlines()
    assert lines[0].startswith("# anneal_hip gemm variants v1")
    assert f"1/0/0/{M}/{N}/{K} {best}" in lines
    dev.gemm_tune_cache(str(path), False)
    bad = tmp_path / "bad.txt"
    bad.write_text(lines[0] + "\n1/0/0/8/8/8 99\n")
    with pytest.raises(L.AnnealHipError, match="bad line"):
        dev.gemm_tune_cache(str(bad), False)
    for b in (dA, dB, dC):
        b.free()


@pytest.mark.parametrize("splits", [0, 1, 2, 4, 8, 16])
@pytest.mark.parametrize("epi", ["store", "bias_relu", "mask", "grad"])
def test_gemm_f32_split_k(dev, epi, splits):
    """The f32 tiled kernel with K split across workgroups (splits=s fixes the count, 0 lets the shape
    choose: 4 k-groups x 8 splits here): partials folded in split order by the last split to arrive, so
    every launch gives the same bits, and each launch leaves the tiles' arrival counters at zero for the
    next (checked by a second launch on other inputs)."""
    from anneal_amd.executor import Buffer, ExecItem, Executor
    M, N, K, ta, tb = (256, 512, 2048, 0, 0) if epi != "grad" else (512, 256, 2048, 1, 1)
    key = f"tmpl:gemm;dtype=f32;epi={epi};ta={ta};tb={tb};M={M};N={N};K={K};tile=64;splits={splits}"
    if splits == 0:
        key = f"tmpl:gemm;dtype=f32;epi={epi};ta={ta};tb={tb};M={M};N={N};K={K}"
    bufs = [Buffer(10, M * N, [M, N], L.AH_F32), Buffer(1, M * K, [K, M] if ta else [M, K], L.AH_F32),
            Buffer(2, N * K, [K, N] if tb else [N, K], L.AH_F32)]
    if epi in ("bias_relu", "mask"):
        bufs.append(Buffer(3, N if epi == "bias_relu" else M * N, [N] if epi == "bias_relu" else [M, N], L.AH_F32))
    ex = Executor(dev)
    prev = None
    for rep in range(2):
        rng = np.random.default_rng(1000 + rep)
        A = rng.standard_normal((M, K)).astype(np.float32)
        B = rng.standard_normal((N, K)).astype(np.float32)
        ins = {1: store_operand(A, ta).ravel(), 2: store_operand(B, tb).ravel()}
        ref = A.astype(np.float64) @ B.astype(np.float64).T
        if epi == "bias_relu":
            bias = rng.standard_normal(N).astype(np.float32)
            ins[3] = bias
            ref = np.maximum(ref + bias, 0)
        elif epi == "mask":
            H = rng.standard_normal((M, N)).astype(np.float32)
            H = np.where(H < 0, np.float32(-0.0), H).astype(np.float32)
            ins[3] = H.ravel()
            ref = np.where(np.signbit(H) & (H == 0), 0.0, ref)
        got = ex.run([ExecItem(key, bufs)], ins)[10].reshape(M, N)
        assert O.relerr(got, ref) < 1e-5, (epi, splits, rep)
        again = ex.run([ExecItem(key, bufs)], ins)[10].reshape(M, N)
        np.testing.assert_array_equal(again.view(np.uint32), got.view(np.uint32))
        assert prev is None or not np.array_equal(prev, got)
        prev = got


def test_gemm_f32_tune_and_cache(dev, tmp_path):
    """The tuner over the f32 kernel's (tile, k-groups, splits) configurations: it returns an index into
    the 58-entry table (38 register-staged, 5 direct-to-LDS, those 5 with K split 2 / 4 / 8 ways), later
    automatic launches of the shape use
    the winner (against float64), and the choice survives the disk cache, where an index past the table
    is rejected."""
    M, N, K = 256, 512, 2048
    A = RNG.standard_normal((M, K)).astype(np.float32)
    B = RNG.standard_normal((N, K)).astype(np.float32)
    dA, dB = dev.buffer(A), dev.buffer(B)
    dC = dev.buffer(M * N, L.AH_F32)
    common = dict(dtype=L.AH_F32, epi=L.EPI_STORE, ta=0, tb=0, M=M, N=N, K=K, A=dA, B=dB, lda=K, ldb=K, C_out=dC,
                  ldc=N)
    best, us = dev.gemm_tune(iterations=2, **common)
    assert 0 <= best < 58 and us > 0
    dev.gemm(**common)
    ref = A.astype(np.float64) @ B.astype(np.float64).T
    assert O.relerr(dC.read().reshape(M, N), ref) < 1e-5
    path = tmp_path / "tune32.txt"
    dev.gemm_tune_cache(str(path), True)
    lines = path.read_text().splitlines()
    assert f"0/0/0/{M}/{N}/{K} {best}" in lines
    dev.gemm_tune_cache(str(path), False)
    bad = tmp_path / "bad32.txt"
    bad.write_text(lines[0] + f"\n0/0/0/{M}/{N}/{K} 58\n")
    with pytest.raises(L.AnnealHipError, match="bad line"):
        dev.gemm_tune_cache(str(bad), False)
    for b in (dA, dB, dC):
        b.free()


# direct-to-LDS f32 configurations (gemm32d.hip): (tile, k per stage, stages)
DMA_CFGS = [(64, 64, 3), (64, 64, 4), (64, 32, 4), (128, 32, 4), (128, 64, 2)]


@pytest.mark.parametrize("shape", [(200, 300, 1024), (36, 20, 128)])
@pytest.mark.parametrize("dma", range(5))
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("epi", ["store", "bias_relu", "mask", "grad"])
def test_gemm_f32_dma_same_bits_as_register_staged(dev, dma, ta, tb, epi, shape):
    """The direct-to-LDS f32 kernel adds K in the order of the register-staged kernel with one k-group
    and no split, so each of its configurations gives the same bits as that kernel at the same tile, for
    every layout and epilogue, on ragged shapes (M, N not multiples of the tile, down to one tile smaller
    than the tile); both against float64.
    The 128-wide configurations take only the store and bias epilogues and run the automatic choice for
    the others, which must then match that choice's bits."""
    from anneal_amd.executor import Buffer, ExecItem, Executor
    tile = DMA_CFGS[dma][0]
    M, N, K = shape
    common = f"tmpl:gemm;dtype=f32;epi={epi};ta={ta};tb={tb};M={M};N={N};K={K}"
    dma_key = common + f";dma={dma}"
    fallback = tile == 128 and epi in ("mask", "grad")
    ref_key = common if fallback else common + f";tile={tile};kg=1;splits=1"
    bufs = [Buffer(10, M * N, [M, N], L.AH_F32), Buffer(1, M * K, [K, M] if ta else [M, K], L.AH_F32),
            Buffer(2, N * K, [K, N] if tb else [N, K], L.AH_F32)]
    rng = np.random.default_rng(31 + dma)
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = rng.standard_normal((N, K)).astype(np.float32)
    ins = {1: store_operand(A, ta).ravel(), 2: store_operand(B, tb).ravel()}
    ref = A.astype(np.float64) @ B.astype(np.float64).T
    if epi in ("bias_relu", "mask"):
        bufs.append(Buffer(3, N if epi == "bias_relu" else M * N, [N] if epi == "bias_relu" else [M, N], L.AH_F32))
    if epi == "bias_relu":
        bias = rng.standard_normal(N).astype(np.float32)
        ins[3] = bias
        ref = np.maximum(ref + bias, 0)
    elif epi == "mask":
        H = rng.standard_normal((M, N)).astype(np.float32)
        H = np.where(H < 0, np.float32(-0.0), H).astype(np.float32)
        ins[3] = H.ravel()
        ref = np.where(np.signbit(H) & (H == 0), 0.0, ref)
    elif epi == "grad":
        ref = -ref   # SGD with lr 1 on a zeroed array: the array becomes -g
    ex = Executor(dev)
    got = ex.run([ExecItem(dma_key, bufs)], ins)[10].reshape(M, N)
    want = ex.run([ExecItem(ref_key, bufs)], ins)[10].reshape(M, N)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
    if epi == "grad":
        return   # the grad key's scale and sign are the register-staged kernel's, checked by its own tests
    assert O.relerr(got, ref) < 1e-5


@pytest.mark.parametrize("dma,splits", [(0, 2), (2, 4), (1, 8), (3, 2), (4, 4)])
@pytest.mark.parametrize("epi", ["store", "mask", "grad"])
def test_gemm_f32_dma_split_k_same_bits(dev, dma, splits, epi):
    """The direct-to-LDS kernel splitting K across workgroups folds the partials as the register-staged
    kernel does (split order, the last arriver's own from registers), so dma=i with splits=s gives the bits
    of tile=BM with one k-group and s splits; two launches in a row give the same bits and leave the
    arrival counters at zero (a second launch on other inputs differs)."""
    from anneal_amd.executor import Buffer, ExecItem, Executor
    tile = DMA_CFGS[dma][0]
    M, N, K, ta, tb = (256, 192, 2048, 0, 0) if epi == "store" else (192, 256, 2048, 1, 1)
    if epi == "mask":
        ta, tb = 0, 1
    common = f"tmpl:gemm;dtype=f32;epi={epi};ta={ta};tb={tb};M={M};N={N};K={K}"
    fallback = tile == 128 and epi in ("mask", "grad")
    dma_key = common + f";dma={dma};splits={splits}"
    ref_key = common if fallback else common + f";tile={tile};kg=1;splits={splits}"
    bufs = [Buffer(10, M * N, [M, N], L.AH_F32), Buffer(1, M * K, [K, M] if ta else [M, K], L.AH_F32),
            Buffer(2, N * K, [K, N] if tb else [N, K], L.AH_F32)]
    if epi == "mask":
        bufs.append(Buffer(3, M * N, [M, N], L.AH_F32))
    ex = Executor(dev)
    prev = None
    for rep in range(2):
        rng = np.random.default_rng(50 + rep)
        A = rng.standard_normal((M, K)).astype(np.float32)
        B = rng.standard_normal((N, K)).astype(np.float32)
        ins = {1: store_operand(A, ta).ravel(), 2: store_operand(B, tb).ravel()}
        if epi == "mask":
            H = rng.standard_normal((M, N)).astype(np.float32)
            ins[3] = np.where(H < 0, np.float32(-0.0), H).astype(np.float32).ravel()
        got = ex.run([ExecItem(dma_key, bufs)], ins)[10]
        again = ex.run([ExecItem(dma_key, bufs)], ins)[10]
        want = ex.run([ExecItem(ref_key, bufs)], ins)[10]
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
        np.testing.assert_array_equal(again.view(np.uint32), got.view(np.uint32))
        if epi == "store":
            assert O.relerr(got.reshape(M, N), A.astype(np.float64) @ B.astype(np.float64).T) < 1e-5
        assert prev is None or not np.array_equal(prev, got)
        prev = got


def test_gemm_f32_dma_key_checks(dev):
    """dma=i is a configuration index, and it excludes tile / kg."""
    from anneal_amd.executor import Buffer, ExecItem, Executor
    bufs = [Buffer(10, 64 * 64, [64, 64], L.AH_F32), Buffer(1, 64 * 64, [64, 64], L.AH_F32),
            Buffer(2, 64 * 64, [64, 64], L.AH_F32)]
    ins = {1: np.ones(64 * 64, np.float32), 2: np.ones(64 * 64, np.float32)}
    for bad in ("dma=5", "dma=0;tile=64", "dma=1;kg=2"):
        with pytest.raises(L.AnnealHipError, match="dma|kg"):
            Executor(dev).run([ExecItem(f"tmpl:gemm;dtype=f32;epi=store;ta=0;tb=0;M=64;N=64;K=64;{bad}", bufs)], ins)


@pytest.mark.parametrize("cfg", [(64, 0, 4), (64, 4, 2), (128, 2, 8), (128, 0, 16), (64, 1, 3)])
def test_gemm_f32_split_k_ragged(dev, cfg):
    """Split-K on ragged tiles (M, N and K not multiples of the tile or the 32-wide k chunk), with fixed
    or automatic k-groups; splits=3 runs three splits (groups past K load zeros)."""
    from anneal_amd.executor import Buffer, ExecItem, Executor
    tile, kg, splits = cfg
    M, N, K = 200, 300, 1000
    key = f"tmpl:gemm;dtype=f32;epi=bias_relu;ta=1;tb=0;M={M};N={N};K={K};tile={tile};splits={splits}"
    if kg:
        key += f";kg={kg}"
    rng = np.random.default_rng(7)
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = rng.standard_normal((N, K)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    bufs = [Buffer(10, M * N, [M, N], L.AH_F32), Buffer(1, M * K, [K, M], L.AH_F32), Buffer(2, N * K, [N, K], L.AH_F32),
            Buffer(3, N, [N], L.AH_F32)]
    got = Executor(dev).run([ExecItem(key, bufs)], {1: store_operand(A, 1).ravel(), 2: B.ravel(), 3: bias})[10]
    ref = np.maximum(A.astype(np.float64) @ B.astype(np.float64).T + bias, 0)
    assert O.relerr(got.reshape(M, N), ref) < 1e-5
