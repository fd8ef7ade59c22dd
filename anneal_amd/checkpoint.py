"""Checkpoint IO over the C ABI: safetensors save/load and .npy/.npz load with the reference's dtype
policy (tensor/safetensors/safetensors.go, tensor/npy/npy.go), plus the Parameter-map forms the
reference exposes (Save(path, map[name]*Parameter) / Load(path, into)) for device-resident trainers.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib as L


def load_tensors(path: str) -> dict:
    """name -> float32 ndarray (shape as stored) for every tensor of a .safetensors / .npy / .npz file
    (safetensors.LoadTensors, npy.Load / LoadNPZ). Raises AnnealHipError on a policy violation."""
    lib = L.load()
    h = C.c_void_p()
    L.check(lib.ah_ckpt_open(str(path).encode(), C.byref(h)))
    try:
        out = {}
        for i in range(lib.ah_ckpt_count(h)):
            name, dtype, rank = C.c_char_p(), C.c_char_p(), C.c_int32()
            shape, n = C.POINTER(C.c_int64)(), C.c_int64()
            L.check(lib.ah_ckpt_entry(h, i, C.byref(name), C.byref(dtype), C.byref(rank), C.byref(shape), C.byref(n)))
            arr = np.empty(n.value, np.float32)
            L.check(lib.ah_ckpt_read(h, i, arr.ctypes.data_as(C.POINTER(C.c_float)), n.value))
            out[name.value.decode()] = arr.reshape([shape[d] for d in range(rank.value)])
        return out
    finally:
        lib.ah_ckpt_close(h)


def save_safetensors(path: str, tensors: dict) -> None:
    """Writes name -> array as an F32 safetensors file in the reference's layout (safetensors.Save)."""
    lib = L.load()
    names = list(tensors)
    arrs = [np.ascontiguousarray(tensors[k], np.float32) for k in names]
    shapes = [(C.c_int64 * max(a.ndim, 1))(*a.shape) for a in arrs]
    cn = (C.c_char_p * max(len(names), 1))(*[k.encode() for k in names])
    cd = (C.POINTER(C.c_float) * max(len(names), 1))(*[a.ctypes.data_as(C.POINTER(C.c_float)) for a in arrs])
    cs = (C.POINTER(C.c_int64) * max(len(names), 1))(*[C.cast(s, C.POINTER(C.c_int64)) for s in shapes])
    cr = (C.c_int32 * max(len(names), 1))(*[a.ndim for a in arrs])
    L.check(lib.ah_safetensors_save(str(path).encode(), len(names), cn, cd, cs, cr))


def save_params(path: str, trainer, names: dict) -> None:
    """safetensors.Save for a device-resident trainer: names maps checkpoint name -> (slot name, shape)."""
    save_safetensors(path, {k: trainer.get(slot, int(np.prod(shape))).reshape(shape)
                            for k, (slot, shape) in names.items()})


def load_params(path: str, trainer, names: dict) -> None:
    """safetensors.Load into a device-resident trainer: every requested name must exist with the same
    shape (a mismatch is an error, safetensors.go:150-180)."""
    tensors = load_tensors(path)
    for k, (slot, shape) in names.items():
        if k not in tensors:
            raise L.AnnealHipError(f"checkpoint: tensor {k!r} not in {path}")
        if tuple(tensors[k].shape) != tuple(shape):
            raise L.AnnealHipError(f"checkpoint: tensor {k!r} has shape {tensors[k].shape}, want {tuple(shape)}")
        trainer.set(slot, tensors[k].ravel())
