"""Argument validation of the C ABI (no device needed): every entry point rejects null handles and
malformed arguments with an AH_ERR_* code and a message in ah_last_error(), instead of crashing.
The reference's executor returns wrapped Go errors with no partial results (backend/webgpu/executor.go)."""
import ctypes as C

import pytest

from anneal_amd import _lib as L

lib = L.load()


def last_error() -> str:
    m = lib.ah_last_error()
    return m.decode() if m else ""


def test_null_device_calls_fail_cleanly():
    assert lib.ah_sync(None) == 1 and "null" in last_error()
    d = L.ah_gemm_desc()
    assert lib.ah_gemm(None, C.byref(d)) == 1
    v, us = C.c_int32(), C.c_double()
    assert lib.ah_gemm_tune(None, C.byref(d), 1, C.byref(v), C.byref(us)) == 1
    outs, n = C.POINTER(L.ah_output)(), C.c_int32()
    assert lib.ah_run(None, None, 0, None, 0, C.byref(outs), C.byref(n)) == 1
    assert lib.ah_timer_start(None) == 1
    assert lib.ah_graph_begin(None) == 1
    assert lib.ah_graph_replay(None, None) == 1
    h = C.c_void_p()
    dims = (C.c_int64 * 4)(64, 784, 128, 10)
    assert lib.ah_trainer_create(None, L.TRAIN_MLP_CE, dims, 4, C.c_float(0.01), C.byref(h)) == 1
    assert lib.ah_trainer_step(None, 64, 0) == 1
    assert lib.ah_trainer_probe(None, 0) == 1
    assert lib.ah_trainer_probe_span(None, 0, 0) == 1
    assert lib.ah_chain_step(None, None, None, 8, 8, None, None, None) == 1
    assert lib.ah_softmax_ce(None, None, None, 4, 4, None, None) == 1


def test_translate_rejects_null_and_reports_compile_class_error():
    assert lib.ah_translate_wgsl(None, None, 0, None) == 1
    bad = b"fn main() {\n  data0[0] = frobnicate(1.0);\n}\n"
    assert lib.ah_translate_wgsl(bad, None, 0, None) == 4          # AH_ERR_COMPILE
    assert "frobnicate" in last_error() or "unsupported" in last_error()


@pytest.mark.parametrize("f", [0.0, -0.0, 1.0, 65504.0, 65520.0, 1e-8, float("inf")])
def test_codec_round_trip_is_idempotent(f):
    """f16(f32(f16(x))) == f16(x): the codec entry points need no device."""
    lib.ah_f32_to_f16.restype = C.c_uint16
    lib.ah_f32_to_f16.argtypes = [C.c_float]
    lib.ah_f16_to_f32.restype = C.c_float
    lib.ah_f16_to_f32.argtypes = [C.c_uint16]
    h = lib.ah_f32_to_f16(f)
    assert lib.ah_f32_to_f16(lib.ah_f16_to_f32(h)) == h
