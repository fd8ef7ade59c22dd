"""WGSL -> HIP rendering of the kernels anneal's codegen emits (host side: no GPU needed).

Each kernel of tests/wgsl_kernels.py is rendered through the library's C ABI (ah_translate_wgsl) and
the result is compiled for gfx950 with hipcc, so the rendering is checked as real HIP here; the GPU
test (test_gpu_wgsl.py) runs the same kernels through ah_run and compares their outputs.
"""
import os
import shutil
import subprocess

import pytest

import wgsl_kernels as W
from anneal_amd import _lib as L

HIPCC = "/opt/rocm/bin/hipcc"


@pytest.mark.parametrize("name", sorted(W.kernels()))
def test_render_and_compile_for_gfx950(name, tmp_path):
    src = W.kernels()[name][0]
    hip = L.translate_wgsl(src)
    assert 'extern "C" __global__' in hip and " kernel(" in hip
    if not os.path.exists(HIPCC) or shutil.which("ld.lld") is None and not os.path.exists("/opt/rocm/llvm/bin/ld.lld"):
        pytest.skip("hipcc not available")
    f = tmp_path / "k.hip"
    f.write_text("#include <hip/hip_runtime.h>\n" + hip)
    r = subprocess.run([HIPCC, "--offload-arch=gfx950", "--cuda-device-only", "-O3", "-std=c++17", "-ffp-contract=off",
                        "-fwrapv", "-c", str(f), "-o", str(tmp_path / "k.o")], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]


def test_symbolic_kernel_takes_params_n_scalars():
    hip = L.translate_wgsl(W.kernels()["symbolic_batch"][0])
    assert "int wg_n0, int wg_n1, int wg_n2, int wg_n3" in hip and "params_n" in hip


@pytest.mark.parametrize("bad", [
    "@group(0) @binding(0) var<storage, read_write> data0: array<f32>;\n@compute @workgroup_size(1, 1, 1)\n"
    "fn main(@builtin(global_invocation_id) gid: vec3<u32>) {\n  data0[0] = textureLoad(t, 0);\n}\n",
    "@group(0) @binding(0) var<storage, read_write> data0: array<mat4x4<f32>>;\n",
])
def test_outside_the_subset_is_rejected(bad):
    with pytest.raises(L.AnnealHipError, match="wgsl"):
        L.translate_wgsl(bad)
