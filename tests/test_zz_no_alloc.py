"""ah_chain_step_noalloc (the config-5 chain with its workspace in the library's per-GPU static array)
against ah_chain_step (the same kernels with a hipMalloc'd workspace), through the C ABI: two calls in a
row, the second on a smaller input, so a stale workspace from the first call would show. The chain writes
every workspace entry before reading it, so the two must agree bit for bit."""
import numpy as np
import pytest

from anneal_amd import _lib as L

pytestmark = pytest.mark.gpu


def _run(dev, fn, X, g):
    R, Cc = X.shape
    bufs = [dev.buffer(X), dev.buffer(g), dev.buffer(R * Cc), dev.buffer(Cc), dev.buffer(1)]
    fn(bufs[0], bufs[1], R, Cc, bufs[2], bufs[3], bufs[4])
    dev.sync()
    out = [b.read() for b in bufs[2:]]
    for b in bufs:
        b.free()
    return out


def test_noalloc_matches_allocating_entry_point(dev):
    rng = np.random.default_rng(7)
    for R, Cc in ((8192, 4096), (1000, 516)):      # config-5 shape, then a smaller ragged one
        X = rng.standard_normal((R, Cc)).astype(np.float32)
        X[3, :] = X.max() + 1.0                    # tied column maxima exercise the tie-share path
        X[11, :] = X[3, :]
        g = (1 + 0.02 * rng.standard_normal(Cc)).astype(np.float32)
        want = _run(dev, dev.chain_step, X, g)
        got = _run(dev, dev.chain_step_noalloc, X, g)
        for a, b in zip(got, want):
            np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))
        assert np.isfinite(got[2][0])


def test_noalloc_rejects_shapes_beyond_the_workspace(dev):
    R, Cc = 65536, 4096                            # needs 1024*4096*4 floats > 2^22
    bufs = [dev.buffer(4), dev.buffer(4), dev.buffer(4), dev.buffer(4), dev.buffer(1)]
    with pytest.raises(L.AnnealHipError, match="maximum"):
        dev.chain_step_noalloc(bufs[0], bufs[1], R, Cc, bufs[2], bufs[3], bufs[4])
    for b in bufs:
        b.free()
