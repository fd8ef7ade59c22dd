"""The reference's kernels as rendered WGSL, run through ah_run / ah_run_symbolic (WGSL -> HIP -> hiprtc).

ExecItems carry only the rendered source (as the schedule cache hands them over, schedule/cache.go:69-100);
outputs are compared with numpy restatements: bit-exact for the index/tie, known-answer and f16 cases,
1e-6 relative for transcendental and reordered sums.
"""
import numpy as np
import pytest

import wgsl_kernels as W
from anneal_amd.executor import Buffer, ExecItem, Executor

pytestmark = pytest.mark.gpu
EXACT = {"matmul_known_answer", "max_tie_mask", "f16_accumulate", "vec4_accumulators", "diag_fma_probe"}


@pytest.mark.parametrize("name", sorted(W.kernels()))
def test_wgsl_kernel_runs_and_matches(dev, name):
    src, bufs, ws, wc, inputs, want, sym = W.kernels()[name]
    b = [Buffer(u, n, (sh[0] if sh else [n]), dtype=dt) for (u, n, dt, *sh) in bufs]
    item = ExecItem(src, b, sym_vars=["N"] if sym else [], local_size=ws, workgroup_count=wc)
    ex = Executor(dev)
    out = ex.run_symbolic([item], inputs, {"N": sym}) if sym else ex.run([item], inputs)
    got = out[bufs[0][0]]
    assert got.size == want.size
    if name in EXACT:
        np.testing.assert_array_equal(got.view(np.uint32), want.astype(np.float32).view(np.uint32))
    else:
        np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("M,N,K,ta,tb,b_first", [(96, 80, 64, False, True, False), (257, 130, 77, True, False, True),
                                                 (512, 384, 256, False, False, False)])
def test_selected_contraction_matches_rendering(dev, monkeypatch, M, N, K, ta, tb, b_first):
    """A rendered contraction runs the MFMA template (selected from its WGSL, tests/test_wgsl_select.py);
    its output matches a float64 product at the f32 reduction bar (1e-5 here) and the rendered kernel's
    own output (selection off) to summation order."""
    from anneal_amd import _lib as L
    from anneal_amd.backend import Device
    src, ws, wc = W.matmul_wgsl(M, N, K, ta=ta, tb=tb, b_first=b_first)
    assert L.wgsl_template_key(src).startswith("tmpl:gemm")
    rng = np.random.default_rng(M + N + K)
    A = rng.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
    B = rng.standard_normal((K, N) if tb else (N, K)).astype(np.float32)
    want = (A.T if ta else A).astype(np.float64) @ (B if tb else B.T).astype(np.float64)
    bufs = [Buffer(30, M * N, [M * N]), Buffer(1, A.size, [A.size]), Buffer(2, B.size, [B.size])]
    item = ExecItem(src, bufs, local_size=ws, workgroup_count=wc)
    got = Executor(dev).run([item], {1: A.ravel(), 2: B.ravel()})[30].reshape(M, N)
    scale = np.abs(want).max()
    assert np.abs(got - want).max() / scale < 1e-5
    monkeypatch.setenv("AH_WGSL_TEMPLATES", "0")
    with Device(0) as d2:    # a fresh device: its module cache renders the WGSL
        ref = Executor(d2).run([item], {1: A.ravel(), 2: B.ravel()})[30].reshape(M, N)
    assert np.abs(ref - want).max() / scale < 1e-5
    assert np.abs(got - ref).max() / scale < 1e-5


@pytest.mark.parametrize("form", ["let", "inline"])
def test_selected_bias_contraction_matches_rendering(dev, monkeypatch, form):
    """The Linear forward with its bias (acc + b[n]) selected as tmpl:gemm epi=bias matches float64 and
    the rendered kernel."""
    from anneal_amd.backend import Device
    M, N, K = 200, 136, 96
    src, ws, wc = W.matmul_wgsl(M, N, K, bias=form)
    rng = np.random.default_rng(5)
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = rng.standard_normal((K, N)).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32)
    want = A.astype(np.float64) @ B.astype(np.float64) + b
    bufs = [Buffer(30, M * N, [M * N]), Buffer(1, A.size, [A.size]), Buffer(2, B.size, [B.size]), Buffer(3, N, [N])]
    item = ExecItem(src, bufs, local_size=ws, workgroup_count=wc)
    inp = {1: A.ravel(), 2: B.ravel(), 3: b}
    got = Executor(dev).run([item], inp)[30].reshape(M, N)
    scale = np.abs(want).max()
    assert np.abs(got - want).max() / scale < 1e-5
    monkeypatch.setenv("AH_WGSL_TEMPLATES", "0")
    with Device(0) as d2:
        ref = Executor(d2).run([item], inp)[30].reshape(M, N)
    assert np.abs(got - ref).max() / scale < 1e-5


# ── the configs-1/4 training step as rendered kernels (tests/wgsl_lower.py) ────────────────────────

import oracle_lib as O  # noqa: E402
import wgsl_lower as WL  # noqa: E402
from anneal_amd import data  # noqa: E402


def run_rendered_step(dev, B, D, H, C, symbolic, inputs):
    ks, lv, outs = WL.mlp_ce_step(B, D, H, C, symbolic=symbolic)
    items = [ExecItem(src, [Buffer(u, n, sh, dtype=dt) for (u, n, dt, sh) in bufs], sym_vars=["N"] if symbolic else [],
                      local_size=ws, workgroup_count=wc) for _, src, bufs, ws, wc, _ in ks]
    feed = {lv[k]: (inputs[k].view(np.float32) if k == "labels" else inputs[k].ravel()) for k in lv}
    ex = Executor(dev)
    got = ex.run_symbolic(items, feed, {"N": B}) if symbolic else ex.run(items, feed)
    return {k: got[u] for k, u in outs.items()}


@pytest.mark.parametrize("B,D,H,C,symbolic", [(64, 784, 128, 10, False), (7, 512, 2048, 512, True),
                                              (256, 512, 2048, 512, True)])
def test_rendered_mlp_ce_step_matches_oracle(dev, B, D, H, C, symbolic):
    """The configs-1/4 step as the reference's rendered kernels (14 WGSL kernels, restated from its
    scheduler's rules and lowering), run through ah_run / ah_run_symbolic: five contractions and two
    reductions on the hand-written templates, six prologue reductions on the wave rendering, dZ on the
    thread rendering. Loss and gradients match ora_mlp_ce_step at the f32 reduction bar (1e-4)."""
    p = data.mlp_ce_inputs(B, D, H, C, **({} if B == 64 else {"x_lo": -1.0, "x_hi": 1.0}))
    got = run_rendered_step(dev, B, D, H, C, symbolic, p)
    wl, g, _ = O.mlp_ce_step(p, 0.0)
    assert abs(got["loss"][0] - wl) <= 1e-4 * max(1.0, abs(wl))
    for k in ("dW1", "db1", "dW2", "db2"):
        assert O.relerr(got[k], g[k].ravel()) < 1e-4, k


def test_rendered_step_templates_match_the_plain_rendering(dev, monkeypatch):
    """The same rendered step with every kernel rendered one thread per output (templates and the wave
    form off) gives the same results to summation order."""
    from anneal_amd.backend import Device
    B, D, H, C = 64, 784, 128, 10
    p = data.mlp_ce_inputs(B, D, H, C)
    fast = run_rendered_step(dev, B, D, H, C, False, p)
    monkeypatch.setenv("AH_WGSL_TEMPLATES", "0")
    monkeypatch.setenv("AH_WGSL_WAVE", "0")
    with Device(0) as d2:
        plain = run_rendered_step(d2, B, D, H, C, False, p)
    for k in fast:
        assert O.relerr(fast[k], plain[k]) < 1e-5, k


@pytest.mark.parametrize("relu,relu_out", [(False, False), (True, False), (False, True)])
def test_selected_f16_contraction_matches_rendering(dev, monkeypatch, relu, relu_out):
    """An f16 Linear forward (widened loads, f16(acc) narrowing, f16 bias add, ReLU on the input or on
    the output) on the f16 MFMA template matches float64 within f16 rounding, and the WGSL rendering to
    the rounding of f16(acc) and the add (the template writes a dead unit as -0.0, equal to the
    rendering's +0.0)."""
    from anneal_amd import _lib as L
    from anneal_amd.backend import Device
    M, N, K = 256, 128, 192
    src, bufs, ws, wc, key = WL.f16_linear(M, N, K, bias=True, relu_a=relu, relu_out=relu_out)
    assert L.wgsl_template_key(src) == key
    rng = np.random.default_rng(11)
    A = rng.standard_normal((M, K)).astype(np.float16).astype(np.float32)
    W = (rng.standard_normal((N, K)) * 0.1).astype(np.float16).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float16).astype(np.float32)
    item = ExecItem(src, [Buffer(u, n, sh, dtype=dt) for (u, n, dt, sh) in bufs], local_size=ws, workgroup_count=wc)
    inp = {1: A.ravel(), 2: W.ravel(), 3: b}
    got = Executor(dev).run([item], inp)[30].reshape(M, N)
    Ar = np.maximum(A, 0) if relu else A
    want = (Ar.astype(np.float64) @ W.T.astype(np.float64)).astype(np.float16).astype(np.float64) + b
    if relu_out:
        want = np.maximum(want, 0)
    assert np.max(np.abs(got - want)) <= 2e-3 * np.max(np.abs(want))
    monkeypatch.setenv("AH_WGSL_TEMPLATES", "0")
    with Device(0) as d2:
        ref = Executor(d2).run([item], inp)[30].reshape(M, N)
    # f16(acc) may differ by one ulp of the accumulator (summation order), and the f16 bias add rounds once
    # more: one ulp at |acc| plus one at the result
    acc = np.abs(ref - b).astype(np.float16)   # (with relu_out, an upper bound where the output was clamped)
    ulp = np.abs(np.spacing(acc)).astype(np.float32) + np.abs(np.spacing(ref.astype(np.float16))).astype(np.float32)
    assert np.all(np.abs(got - ref) <= ulp + 1e-7)


@pytest.mark.parametrize("shape", [(128, 96, 128, 64, 32), (256, 128, 256, 256, 128)])
def test_rendered_mlp3_step_matches_oracle(dev, shape):
    """Config 3's step as the reference's rendered kernels (13 WGSL kernels: three f16 Linear layers on the
    f16 MFMA template with the bias epilogue and the ReLU prologue, the f16 MSE reduce, the loss adjoint,
    the f32 column sum on the reduce template, the mixed f32 x f16 backward contractions on the f32 template
    with widening prologues, the masked column sums on the wave rendering), run through ah_run: loss and
    gradients match ora_mlp3_f16_step at the config-3 bar (2e-2; the f16 forward's roundings differ with the summation order)."""
    B, D0, D1, D2, D3 = shape
    p = data.mlp3_inputs(B, D0, D1, D2, D3)
    q = dict(p)
    q["x"], q["t"] = data.f16_quantize(p["x"]), data.f16_quantize(p["t"])
    ks, lv, outs = WL.mlp3_step(B, D0, D1, D2, D3)
    from anneal_amd import _lib as L
    for name, src, _, _, _, plan in ks:
        assert L.wgsl_plan(src) == plan, name
    items = [ExecItem(src, [Buffer(u, n, sh, dtype=dt) for (u, n, dt, sh) in bufs], local_size=ws, workgroup_count=wc)
             for _, src, bufs, ws, wc, _ in ks]
    got = Executor(dev).run(items, {lv[k]: q[k].ravel() for k in lv})
    wl, g, _ = O.mlp3_step(q, 0.0)
    loss = got[outs["loss"]][0]
    assert abs(loss - wl) < 2e-2 * abs(wl)
    for k in ("dW1", "db1", "dW2", "db2", "dW3", "db3"):
        assert O.relerr(got[outs[k]], g[k].ravel()) < 2e-2, k


@pytest.mark.parametrize("name", ["dW3", "dH2", "dW2", "dH1", "dW1"])
def test_selected_mixed_type_contraction_matches_rendering(dev, monkeypatch, name):
    """Each f32 x f16 backward contraction of config 3's rendered step, alone on random inputs, runs the f32
    template with its f16 operand (and the f16 pre-activation its mask reads) widened by a prologue: the
    output matches float64 and the wave rendering (selection off) at the f32 reduction bar (1e-5 of the
    output's scale; widening f16 -> f32 is exact, so only the summation order differs)."""
    from anneal_amd import _lib as L
    from anneal_amd.backend import Device
    ks, _, _ = WL.mlp3_step(192, 96, 160, 128, 64)
    _, src, bufs, ws, wc, plan = next(k for k in ks if k[0] == name)
    assert L.wgsl_plan(src) == plan and plan.startswith("tmpl:gemm;dtype=f32")
    rng = np.random.default_rng(len(name) * 7 + ord(name[-1]))
    inp = {}
    for u, n, dt, sh in bufs[1:]:
        v = rng.standard_normal(n).astype(np.float32)
        inp[u] = v.astype(np.float16).astype(np.float32) if dt == L.AH_F16 else v
    item = ExecItem(src, [Buffer(u, n, sh, dtype=dt) for (u, n, dt, sh) in bufs], local_size=ws, workgroup_count=wc)
    out = bufs[0][0]
    got = Executor(dev).run([item], inp)[out]
    monkeypatch.setenv("AH_WGSL_TEMPLATES", "0")
    with Device(0) as d2:
        ref = Executor(d2).run([item], inp)[out]
    scale = np.abs(ref).max()
    assert scale > 0 and np.abs(got - ref).max() / scale < 1e-5


@pytest.mark.parametrize("R,Cc", [(64, 48), (257, 33), (1024, 96)])
def test_rendered_chain_step_matches_oracle(dev, R, Cc):
    """Config 5's step as the reference's rendered kernels (10 WGSL kernels, the permute / pad / shrink
    chain as index arithmetic in every load of Y, tests/wgsl_lower.py chain_step), run through ah_run:
    loss and dg match ora_chain_step at 1e-5, dX at 1e-4 of max |dX| away from the column maxima, and the
    tie elements (whose share is a rounding residue of the max path) no further from the float64 closed
    form than the oracle is, plus 1e-4, as test_chain_kernel_vs_oracle judges the hand-written kernels."""
    rng = np.random.default_rng(R + Cc)
    X = rng.standard_normal((R, Cc)).astype(np.float32)
    X[5, :] = X.max() + 0.5                              # every row of Y gets a tie
    X[9, :] = X[5, :]
    g = (1 + 0.02 * rng.standard_normal(Cc)).astype(np.float32)
    ks, lv, outs = WL.chain_step(R, Cc)
    items = [ExecItem(src, [Buffer(u, n, sh, dtype=dt) for (u, n, dt, sh) in bufs], local_size=ws, workgroup_count=wc)
             for _, src, bufs, ws, wc, _ in ks]
    got = Executor(dev).run(items, {lv["X"]: X.ravel(), lv["g"]: g})
    wl, wdX, wdg = O.chain_step(X, g)
    from oracle_np import chain_dX_f64
    dX = got[outs["dX"]].reshape(R, Cc)
    exact = chain_dX_f64(X, g)
    mask = X == X.max(0, keepdims=True)
    den = np.max(np.abs(wdX))
    assert np.max(np.abs(dX - wdX)[~mask]) / den < 1e-4
    assert np.max(np.abs(dX - exact)[mask]) / den <= np.max(np.abs(wdX - exact)[mask]) / den + 1e-4
    assert O.relerr(got[outs["dg"]], wdg) < 1e-5
    assert abs(got[outs["loss"]][0] - wl) < 1e-5 * abs(wl)
