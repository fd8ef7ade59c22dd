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
