"""backend.Executor mirror (ah_run / ah_run_symbolic / ah_benchmark) on the GPU.

Checks the Run contract of backend/webgpu/executor.go:26-237 and :576-922 through the C ABI:
bufs[0] is the output, PARAM order for inputs, slot sharing, final outputs = outputs no item reads,
inputs for unknown buffers ignored, f16 buffers widened to f32 on download (codec bit-exact against the
oracle), symbolic batch bound per call, errors as exceptions with the kernel index in the message.
"""
import numpy as np
import pytest

import oracle_lib as O
from anneal_amd import _lib as L
from anneal_amd.executor import Buffer, ExecItem, Executor

pytestmark = pytest.mark.gpu

ADD = r'''
extern "C" __global__ void kernel(float *data0, const float *data1, const float *data2) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < 1000) data0[i] = data1[i] + data2[i];
}'''
RELU2 = r'''
extern "C" __global__ void kernel(float *data0, const float *data1) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < 1000) data0[i] = fmaxf(data1[i], 0.0f) * 2.0f;
}'''
# symbolic kernel: params_n arrives as four int32 scalars after the buffers
SYM_SCALE = r'''
extern "C" __global__ void kernel(float *data0, const float *data1, int n, int, int, int) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n * 16) data0[i] = data1[i] * 0.5f;
}'''
# f16 buffers hold IEEE binary16; _Float16 arithmetic (x*1 + 0 is exact, NaN payloads aside)
F16_COPY = r'''
extern "C" __global__ void kernel(_Float16 *data0, const _Float16 *data1) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < 256) data0[i] = data1[i];
}'''


def test_run_two_items_final_output_and_slot(dev):
    ex = Executor(dev)
    rng = np.random.default_rng(0)
    a, b = rng.standard_normal(1000, dtype=np.float32), rng.standard_normal(1000, dtype=np.float32)
    items = [ExecItem(ADD, [Buffer(10, 1000, [1000], slot=0), Buffer(1, 1000, [1000]), Buffer(2, 1000, [1000])],
                      local_size=(64, 1, 1), workgroup_count=(16, 1, 1)),
             ExecItem(RELU2, [Buffer(11, 1000, [1000]), Buffer(10, 1000, [1000], slot=0)],
                      local_size=(64, 1, 1), workgroup_count=(16, 1, 1))]
    out = ex.run(items, {1: a, 2: b, 99: np.ones(4, np.float32)})   # uop 99 is unknown: ignored
    assert set(out) == {11}
    np.testing.assert_array_equal(out[11], np.maximum(a + b, 0) * 2)


def test_run_gemm_template_bias_relu(dev):
    ex = Executor(dev)
    rng = np.random.default_rng(1)
    M, N, K = 64, 128, 784
    x = rng.random((M, K), dtype=np.float32)
    W = rng.standard_normal((N, K), dtype=np.float32) * 0.05
    bias = rng.standard_normal(N, dtype=np.float32)
    src = f"tmpl:gemm;dtype=f32;epi=bias_relu;ta=0;tb=0;M={M};N={N};K={K}"
    item = ExecItem(src, [Buffer(5, M * N, [M, N]), Buffer(1, M * K, [M, K]), Buffer(2, N * K, [N, K]),
                          Buffer(3, N, [N])])
    out = ex.run([item], {1: x, 2: W, 3: bias})[5].reshape(M, N)
    want = np.maximum(x.astype(np.float64) @ W.T.astype(np.float64) + bias, 0)
    assert np.max(np.abs(out - want)) <= 1e-4 * max(1.0, np.max(np.abs(want)))


@pytest.mark.parametrize("n", [1, 7, 256])
def test_run_symbolic_binds_batch(dev, n):
    ex = Executor(dev)
    rng = np.random.default_rng(n)
    K, N = 512, 64
    x = rng.uniform(-1, 1, (n, K)).astype(np.float32)
    W = rng.standard_normal((N, K), dtype=np.float32) * 0.05
    g = ExecItem(f"tmpl:gemm;dtype=f32;epi=store;ta=0;tb=0;M=sym;N={N};K={K}",
                 [Buffer(7, 0, [0, N]), Buffer(1, 0, [0, K]), Buffer(2, N * K, [N, K])], sym_vars=["N"])
    h = ExecItem(SYM_SCALE, [Buffer(8, 0, [0, 16]), Buffer(7, 0, [0, N])], sym_vars=["N"],
                 local_size=(64, 1, 1))
    out = ex.run_symbolic([g, h], {1: x, 2: W}, {"N": n})
    assert set(out) == {8}
    y = x.astype(np.float64) @ W.T.astype(np.float64)
    got = out[8]
    assert got.size == n * 16
    want = (y.ravel()[: n * 16] * 0.5)
    assert np.max(np.abs(got - want)) <= 1e-4 * max(1.0, np.max(np.abs(want)))


def test_f16_buffers_use_reference_codec(dev):
    ex = Executor(dev)
    rng = np.random.default_rng(3)
    v = (rng.standard_normal(256) * 100).astype(np.float32)
    v[:4] = [65520.0, 1e-8, -0.0, 5.9604645e-08]   # overflow to inf, underflow, signed zero, min subnormal
    item = ExecItem(F16_COPY, [Buffer(2, 256, [256], dtype=L.AH_F16), Buffer(1, 256, [256], dtype=L.AH_F16)],
                    local_size=(64, 1, 1), workgroup_count=(4, 1, 1))
    out = ex.run([item], {1: v})[2]
    ora = O.load()
    want = np.array([ora.ora_f16_to_f32(ora.ora_f32_to_f16(float(f))) for f in v], np.float32)
    np.testing.assert_array_equal(out.view(np.uint32), want.view(np.uint32))


def test_compile_error_names_the_kernel(dev):
    ex = Executor(dev)
    bad = ExecItem("extern \"C\" __global__ void kernel(float *data0) { this is not C++ }",
                   [Buffer(1, 4, [4])])
    with pytest.raises(L.AnnealHipError, match="kernel 0"):
        ex.run([bad], {})


def test_benchmark_stats(dev):
    ex = Executor(dev)
    item = ExecItem(ADD, [Buffer(10, 1000, [1000]), Buffer(1, 1000, [1000]), Buffer(2, 1000, [1000])],
                    local_size=(64, 1, 1), workgroup_count=(16, 1, 1))
    r = ex.benchmark(item, 2, 10)
    assert 0 < r.min_us <= r.median_us <= r.max_us
    assert r.stddev_us >= 0 and r.cv >= 0
    with pytest.raises(L.AnnealHipError):
        ex.benchmark(item, 0, 0)


@pytest.mark.parametrize("which", ["A", "B", "C", "bias"])
def test_template_key_larger_than_its_buffers_is_refused(dev, which):
    """A tmpl:gemm key whose M/N/K need more elements than a bound buffer holds is an error before any
    launch (the hand-written kernels index by the key's shape), naming the PARAM; the same item with
    buffers of the right size runs."""
    M, N, K = 64, 96, 128
    sizes = {"C": M * N, "A": M * K, "B": N * K, "bias": N}
    short = dict(sizes)
    short[which] -= 1
    key = f"tmpl:gemm;dtype=f32;epi=bias;ta=0;tb=0;M={M};N={N};K={K}"

    def item(sz):
        return ExecItem(key, [Buffer(10, sz["C"], [sz["C"]]), Buffer(1, sz["A"], [sz["A"]]),
                              Buffer(2, sz["B"], [sz["B"]]), Buffer(3, sz["bias"], [sz["bias"]])])
    rng = np.random.default_rng(3)
    ins = {1: rng.standard_normal(M * K, dtype=np.float32), 2: rng.standard_normal(N * K, dtype=np.float32),
           3: np.zeros(N, np.float32)}
    with pytest.raises(L.AnnealHipError, match="PARAM"):
        Executor(dev).run([item(short)], ins)
    out = Executor(dev).run([item(sizes)], ins)[10].reshape(M, N)
    want = ins[1].reshape(M, K).astype(np.float64) @ ins[2].reshape(N, K).T.astype(np.float64)
    assert np.abs(out - want).max() < 1e-4 * np.abs(want).max()


def test_symbolic_template_checked_against_the_binding(dev):
    """With a symbolic M the check uses the bound value: a binding larger than the fixed-size A buffer
    allows is refused."""
    N, K = 32, 64
    key = f"tmpl:gemm;dtype=f32;epi=store;ta=0;tb=0;M=sym;N={N};K={K}"
    it = ExecItem(key, [Buffer(10, 0, [0, N]), Buffer(1, 8 * K, [8 * K]), Buffer(2, N * K, [N * K])], sym_vars=["N"])
    ins = {1: np.ones(8 * K, np.float32), 2: np.ones(N * K, np.float32)}
    out = Executor(dev).run_symbolic([it], ins, {"N": 8})
    np.testing.assert_array_equal(out[10], np.full(8 * N, K, np.float32))
    with pytest.raises(L.AnnealHipError, match="PARAM 1"):
        Executor(dev).run_symbolic([it], ins, {"N": 9})
