"""ctypes binding of libanneal_hip.so (declarations mirror include/anneal_hip.h).

The library is the product: if it is missing or fails to load this module raises, and nothing falls
back to a CPU path.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libanneal_hip.so")

AH_OK = 0
AH_F32, AH_F16, AH_BF16, AH_I32, AH_BOOL, AH_U32 = 0, 1, 2, 3, 4, 5
EPI_STORE, EPI_BIAS, EPI_BIAS_RELU, EPI_MSE, EPI_MASK, EPI_SGD = range(6)
TRAIN_MLP_CE, TRAIN_CONVNET, TRAIN_MLP3_F16, TRAIN_CHAIN = 1, 2, 3, 4
STEP_STORE_GRADS, STEP_GRAPH = 1, 2
PLAN_GRAPH = 1


class ah_caps(C.Structure):
    _fields_ = [("has_f16", C.c_int32), ("has_bf16", C.c_int32), ("cu_count", C.c_int32),
                ("wavefront", C.c_int32), ("hbm_bytes", C.c_int64), ("lds_bytes_per_block", C.c_int64),
                ("arch", C.c_char * 64)]


class ah_bench_result(C.Structure):
    _fields_ = [("min_us", C.c_double), ("median_us", C.c_double), ("max_us", C.c_double),
                ("mean_us", C.c_double), ("stddev_us", C.c_double), ("cv", C.c_double)]


class ah_buffer_desc(C.Structure):
    _fields_ = [("uop_idx", C.c_uint32), ("size", C.c_int64), ("dtype", C.c_int32), ("slot", C.c_int32),
                ("rank", C.c_int32), ("shape", C.POINTER(C.c_int64))]


class ah_exec_item(C.Structure):
    _fields_ = [("source", C.c_char_p), ("bufs", C.POINTER(ah_buffer_desc)), ("n_bufs", C.c_int32),
                ("sym_vars", C.POINTER(C.c_char_p)), ("n_sym_vars", C.c_int32),
                ("local_size", C.c_int32 * 3), ("workgroup_count", C.c_int32 * 3)]


class ah_input(C.Structure):
    _fields_ = [("uop_idx", C.c_uint32), ("data", C.POINTER(C.c_float)), ("n", C.c_int64)]


class ah_output(C.Structure):
    _fields_ = [("uop_idx", C.c_uint32), ("data", C.POINTER(C.c_float)), ("n", C.c_int64)]


class ah_gemm_desc(C.Structure):
    _fields_ = [("dtype", C.c_int32), ("epi", C.c_int32), ("ta", C.c_int32), ("tb", C.c_int32),
                ("M", C.c_int32), ("N", C.c_int32), ("K", C.c_int32),
                ("A", C.c_void_p), ("B", C.c_void_p), ("lda", C.c_int64), ("ldb", C.c_int64),
                ("C", C.c_void_p), ("ldc", C.c_int64), ("bias", C.c_void_p), ("aux", C.c_void_p),
                ("ldaux", C.c_int64), ("scale", C.c_float), ("colsum", C.c_void_p), ("W32", C.c_void_p),
                ("W16", C.c_void_p), ("lr", C.c_float), ("gout", C.c_void_p), ("lossacc", C.c_void_p),
                ("tile", C.c_int32), ("variant", C.c_int32)]


class ah_opt(C.Structure):
    _fields_ = [("kind", C.c_int32), ("axis", C.c_int32), ("arg", C.c_int32)]


class ah_beam_result(C.Structure):
    _fields_ = [("min_us", C.c_double), ("base_us", C.c_double), ("searched", C.c_int32), ("from_cache", C.c_int32),
                ("n_opts", C.c_int32), ("opts", ah_opt * 8)]


OPT_IDENTITY, OPT_LOCAL, OPT_TILE, OPT_UPCAST, OPT_VECTORIZE, OPT_GROUP, OPT_SCHEDULE, OPT_MFMA = range(8)

# name -> (restype, argtypes)
_P = C.c_void_p
SIGNATURES = {
    "ah_last_error": (C.c_char_p, []),
    "ah_open": (C.c_int, [C.c_int, C.POINTER(_P)]),
    "ah_close": (None, [_P]),
    "ah_get_caps": (C.c_int, [_P, C.POINTER(ah_caps)]),
    "ah_sync": (C.c_int, [_P]),
    "ah_buf_alloc": (C.c_int, [_P, C.c_int64, C.c_int32, C.POINTER(_P)]),
    "ah_buf_free": (C.c_int, [_P, _P]),
    "ah_upload": (C.c_int, [_P, _P, C.POINTER(C.c_float), C.c_int64, C.c_int32]),
    "ah_download": (C.c_int, [_P, C.POINTER(C.c_float), _P, C.c_int64, C.c_int32]),
    "ah_upload_bytes": (C.c_int, [_P, _P, _P, C.c_int64]),
    "ah_download_bytes": (C.c_int, [_P, _P, _P, C.c_int64]),
    "ah_f32_to_f16": (C.c_uint16, [C.c_float]),
    "ah_f16_to_f32": (C.c_float, [C.c_uint16]),
    "ah_module_get": (C.c_int, [_P, C.c_char_p, C.c_char_p, C.POINTER(_P)]),
    "ah_launch": (C.c_int, [_P, _P, C.POINTER(C.c_uint32), C.POINTER(C.c_uint32), C.POINTER(_P), C.c_int32,
                            C.POINTER(C.c_int32), C.c_int32]),
    "ah_timer_start": (C.c_int, [_P]),
    "ah_timer_stop": (C.c_int, [_P, C.POINTER(C.c_double)]),
    "ah_graph_begin": (C.c_int, [_P]),
    "ah_graph_end": (C.c_int, [_P, C.POINTER(_P)]),
    "ah_graph_replay": (C.c_int, [_P, _P]),
    "ah_graph_destroy": (None, [_P]),
    "ah_run": (C.c_int, [_P, C.POINTER(ah_exec_item), C.c_int32, C.POINTER(ah_input), C.c_int32,
                         C.POINTER(C.POINTER(ah_output)), C.POINTER(C.c_int32)]),
    "ah_run_symbolic": (C.c_int, [_P, C.POINTER(ah_exec_item), C.c_int32, C.POINTER(ah_input), C.c_int32,
                                  C.POINTER(C.c_char_p), C.POINTER(C.c_int64), C.c_int32,
                                  C.POINTER(C.POINTER(ah_output)), C.POINTER(C.c_int32)]),
    "ah_benchmark": (C.c_int, [_P, C.POINTER(ah_exec_item), C.c_int32, C.c_int32, C.POINTER(ah_bench_result)]),
    "ah_outputs_free": (None, [C.POINTER(ah_output), C.c_int32]),
    "ah_plan_create": (C.c_int, [_P, C.POINTER(ah_exec_item), C.c_int32, C.POINTER(_P)]),
    "ah_plan_run": (C.c_int, [_P, C.POINTER(ah_input), C.c_int32, C.POINTER(C.c_char_p), C.POINTER(C.c_int64),
                              C.c_int32, C.c_int32, C.POINTER(C.POINTER(ah_output)), C.POINTER(C.c_int32)]),
    "ah_plan_stats": (C.c_int, [_P, C.POINTER(C.c_int64), C.POINTER(C.c_int64)]),
    "ah_plan_destroy": (None, [_P]),
    "ah_apply_opts": (C.c_int, [C.c_char_p, C.POINTER(ah_opt), C.c_int32, C.c_char_p, C.c_int64, C.POINTER(C.c_int64)]),
    "ah_action_space": (C.c_int, [C.c_char_p, C.POINTER(ah_opt), C.c_int32, C.POINTER(C.c_int32)]),
    "ah_beam_search": (C.c_int, [_P, C.POINTER(ah_exec_item), C.c_int32, C.c_int32, C.c_int32, C.c_int32,
                                 C.POINTER(ah_beam_result)]),
    "ah_beam_apply": (C.c_int, [C.c_char_p, C.c_char_p, C.c_int64, C.POINTER(C.c_int64)]),
    "ah_beam_cache": (C.c_int, [C.c_char_p, C.c_int32]),
    "ah_beam_reset": (None, []),
    "ah_gemm": (C.c_int, [_P, C.POINTER(ah_gemm_desc)]),
    "ah_translate_wgsl": (C.c_int, [C.c_char_p, C.c_char_p, C.c_int64, C.POINTER(C.c_int64)]),
    "ah_wgsl_template_key": (C.c_int, [C.c_char_p, C.c_char_p, C.c_int32]),
    "ah_wgsl_plan": (C.c_int, [C.c_char_p, C.c_char_p, C.c_int32]),
    "ah_ckpt_open": (C.c_int, [C.c_char_p, C.POINTER(_P)]),
    "ah_ckpt_count": (C.c_int32, [_P]),
    "ah_ckpt_entry": (C.c_int, [_P, C.c_int32, C.POINTER(C.c_char_p), C.POINTER(C.c_char_p), C.POINTER(C.c_int32),
                                C.POINTER(C.POINTER(C.c_int64)), C.POINTER(C.c_int64)]),
    "ah_ckpt_read": (C.c_int, [_P, C.c_int32, C.POINTER(C.c_float), C.c_int64]),
    "ah_ckpt_close": (None, [_P]),
    "ah_safetensors_save": (C.c_int, [C.c_char_p, C.c_int32, C.POINTER(C.c_char_p), C.POINTER(C.POINTER(C.c_float)),
                                      C.POINTER(C.POINTER(C.c_int64)), C.POINTER(C.c_int32)]),
    "ah_gemm_tune_cache": (C.c_int, [_P, C.c_char_p, C.c_int32]),
    "ah_gemm_tune": (C.c_int, [_P, C.POINTER(ah_gemm_desc), C.c_int32, C.POINTER(C.c_int32), C.POINTER(C.c_double)]),
    "ah_softmax_ce": (C.c_int, [_P, _P, _P, C.c_int32, C.c_int32, _P, _P]),
    "ah_chain_step": (C.c_int, [_P, _P, _P, C.c_int32, C.c_int32, _P, _P, _P]),
    "ah_chain_step_noalloc": (C.c_int, [_P, _P, _P, C.c_int32, C.c_int32, _P, _P, _P]),
    "ah_trainer_create": (C.c_int, [_P, C.c_int32, C.POINTER(C.c_int64), C.c_int32, C.c_float, C.POINTER(_P)]),
    "ah_trainer_destroy": (None, [_P]),
    "ah_trainer_set": (C.c_int, [_P, C.c_int32, _P, C.c_int64]),
    "ah_trainer_get": (C.c_int, [_P, C.c_int32, _P, C.c_int64]),
    "ah_trainer_step": (C.c_int, [_P, C.c_int64, C.c_int32]),
    "ah_trainer_steps": (C.c_int, [_P, C.c_int64, C.c_int32, C.c_int32]),
    "ah_trainer_probe": (C.c_int, [_P, C.c_int32]),
    "ah_trainer_probe_span": (C.c_int, [_P, C.c_int32, C.c_int32]),
    "ah_trainer_probe_read": (C.c_int, [_P, C.POINTER(C.c_double), C.POINTER(C.c_int64)]),
    "ah_trainer_kernel_count": (C.c_int, [_P, C.c_int64, C.POINTER(C.c_int32)]),
    "ah_trainer_kernel_name": (C.c_int, [_P, C.c_int32, C.c_char_p, C.c_int32]),
}

_lib = None


def load() -> C.CDLL:
    """Load and declare libanneal_hip.so. Raises RuntimeError if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'`")
    lib = C.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


class AnnealHipError(RuntimeError):
    pass


def translate_wgsl(src: str) -> str:
    """HIP C++ rendering of a WGSL kernel in the subset anneal's codegen emits (host only, no device)."""
    lib = load()
    need = C.c_int64()
    check(lib.ah_translate_wgsl(src.encode(), None, 0, C.byref(need)))
    buf = C.create_string_buffer(need.value)
    check(lib.ah_translate_wgsl(src.encode(), buf, need.value, C.byref(need)))
    return buf.value.decode()


def wgsl_template_key(src: str) -> str:
    """The "tmpl:..." key ah_module_get runs in place of a WGSL kernel that is a plain contraction, or ""."""
    buf = C.create_string_buffer(256)
    check(load().ah_wgsl_template_key(src.encode(), buf, 256))
    return buf.value.decode()


def wgsl_plan(src: str) -> str:
    """How ah_module_get runs a rendered WGSL kernel: its "tmpl:..." key, "wave" or "thread"."""
    buf = C.create_string_buffer(256)
    check(load().ah_wgsl_plan(src.encode(), buf, 256))
    return buf.value.decode()


def check(rc: int) -> None:
    if rc != AH_OK:
        msg = load().ah_last_error()
        raise AnnealHipError(f"anneal_hip error {rc}: {msg.decode() if msg else ''}")
