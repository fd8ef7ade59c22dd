"""The C-ABI library loads on a GPU-less host and exports every function include/anneal_hip.h declares.

No compute calls are made here (there is no GPU in the build container); the codec entry points are
pure host functions and are checked against the oracle's table."""
import ctypes as C
import os
import re

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "anneal_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"^\s*(?:const\s+)?[A-Za-z_][\w ]*?[\s\*]+(ah_\w+)\s*\(", text, flags=re.M)
    return sorted(set(names))


def test_header_declares_the_boundary():
    names = declared_functions()
    for must in ("ah_open", "ah_close", "ah_buf_alloc", "ah_upload", "ah_download", "ah_module_get",
                 "ah_launch", "ah_graph_begin", "ah_graph_replay", "ah_run", "ah_run_symbolic",
                 "ah_benchmark", "ah_gemm", "ah_trainer_step", "ah_last_error"):
        assert must in names, must


def test_library_exports_every_declared_symbol():
    from anneal_amd import _lib as L
    lib = C.CDLL(L.LIB_PATH)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_codec_entry_points_match_oracle():
    import oracle_lib as O
    from anneal_amd import _lib as L
    lib = C.CDLL(L.LIB_PATH)
    lib.ah_f32_to_f16.restype = C.c_uint16
    lib.ah_f32_to_f16.argtypes = [C.c_float]
    lib.ah_f16_to_f32.restype = C.c_float
    lib.ah_f16_to_f32.argtypes = [C.c_uint16]
    ora = O.load()
    rng = np.random.default_rng(0)
    bits = np.concatenate([rng.integers(0, 2**32, 4000, dtype=np.uint64).astype(np.uint32),
                           np.array([0, 0x80000000, 0x7F800000, 0xFF800000, 0x7FC00000, 0x477FF000,
                                     0x477FF001, 0x33000000, 0x33000001, 0x387FC000], np.uint32)])
    for b in bits:
        f = float(np.uint32(b).view(np.float32))
        assert lib.ah_f32_to_f16(f) == ora.ora_f32_to_f16(f), hex(b)
    for h in range(0, 65536, 7):
        a, o = lib.ah_f16_to_f32(h), ora.ora_f16_to_f32(h)
        assert (a == o) or (np.isnan(a) and np.isnan(o)), hex(h)
