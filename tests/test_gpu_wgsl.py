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
