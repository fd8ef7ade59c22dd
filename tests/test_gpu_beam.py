"""BEAM retargeted to time HIP candidates (codegen/beam.go:271-541), on the GPU: the search keeps only
candidates bit-identical to the unmodified kernel, never returns one slower than it, caches the winner
per kernel key, and the cache persists to disk and guards the applied key by its hash."""
import numpy as np
import pytest

from anneal_amd import _lib as L
from anneal_amd.executor import (Buffer, ExecItem, Executor, action_space, apply_opts, beam_apply, beam_cache,
                                 beam_reset, beam_search)

pytestmark = pytest.mark.gpu

CASES = [
    ("tmpl:gemm;dtype=f16;epi=store;ta=0;tb=0;M=1024;N=1024;K=512", L.AH_F16, (1024, 1024, 512)),
    # K short enough that the f32 kernel does not split K across workgroups (a candidate with fixed
    # k-groups never splits, so a split baseline would leave no bit-identical candidate)
    ("tmpl:gemm;dtype=f32;epi=store;ta=1;tb=1;M=2048;N=2048;K=128", L.AH_F32, (2048, 2048, 128)),
]


def gemm_item(key, dt, shape):
    M, N, K = shape
    return ExecItem(key, [Buffer(10, M * N, [M, N], dt), Buffer(1, M * K, [M, K], dt), Buffer(2, N * K, [N, K], dt)])


@pytest.mark.parametrize("case", range(len(CASES)))
def test_beam_search_value_guard_cache_and_apply(dev, case, tmp_path):
    key, dt, shape = CASES[case]
    beam_reset()
    assert action_space(key)
    item = gemm_item(key, dt, shape)
    r = beam_search(dev, item, width=2, depth=2, warmup=1, iters=3)
    assert not r.from_cache and r.searched > 0
    assert r.min_us <= r.base_us + 1e-9
    best = apply_opts(key, r.opts)
    # the winner computes the same bits as the unmodified kernel
    M, N, K = shape
    rng = np.random.default_rng(case)
    a = rng.standard_normal(M * K).astype(np.float32)
    b = rng.standard_normal(N * K).astype(np.float32)
    ex = Executor(dev)
    want = ex.run([item], {1: a, 2: b})[10]
    got = ex.run([gemm_item(best, dt, shape)], {1: a, 2: b})[10]
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
    # cached: a second search re-times the stored winner
    r2 = beam_search(dev, item, width=2, depth=2, warmup=1, iters=3)
    assert r2.from_cache and r2.opts == r.opts
    assert beam_apply(key) == best
    # disk cache round trip
    path = tmp_path / "beam.txt"
    beam_cache(path, True)
    beam_reset()
    assert beam_apply(key) == key
    beam_cache(path, False)
    assert beam_apply(key) == best
    beam_reset()
