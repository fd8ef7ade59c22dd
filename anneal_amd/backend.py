"""Host-side handles over the C ABI: Device, DeviceBuffer and Trainer.

Device mirrors the reference's backend.Executor owner (backend/webgpu/open.go:89, backend/device.go:10-37):
one handle, one HIP stream, calls serialized by the caller. Trainer runs one BASELINE config's training
step with parameters resident on the device (the reference re-uploads parameters and realizes each
gradient separately every step: examples/mlp.go:112-142).
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib as L

_NP_DTYPES = {L.AH_F32: np.float32, L.AH_F16: np.float16, L.AH_I32: np.int32, L.AH_U32: np.uint32}


class DeviceBuffer:
    def __init__(self, dev: "Device", n: int, dtype: int):
        self.dev, self.n, self.dtype = dev, int(n), dtype
        p = C.c_void_p()
        L.check(dev.lib.ah_buf_alloc(dev.h, self.n, dtype, C.byref(p)))
        self.ptr = p.value

    @property
    def nbytes(self) -> int:
        return self.n * (2 if self.dtype == L.AH_F16 else 4)

    def write(self, arr: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(arr, dtype=_NP_DTYPES[self.dtype])
        if a.size > self.n:
            raise ValueError(f"array of {a.size} elements does not fit a buffer of {self.n}")
        L.check(self.dev.lib.ah_upload_bytes(self.dev.h, self.ptr, a.ctypes.data, a.nbytes))
        return self

    def read(self, n: int | None = None) -> np.ndarray:
        n = self.n if n is None else n
        out = np.empty(n, dtype=_NP_DTYPES[self.dtype])
        L.check(self.dev.lib.ah_download_bytes(self.dev.h, out.ctypes.data, self.ptr, out.nbytes))
        return out

    def free(self) -> None:
        if self.ptr:
            self.dev.lib.ah_buf_free(self.dev.h, self.ptr)
            self.ptr = None


class Device:
    def __init__(self, ordinal: int = 0):
        self.lib = L.load()
        h = C.c_void_p()
        L.check(self.lib.ah_open(ordinal, C.byref(h)))
        self.h = h.value

    def caps(self) -> dict:
        c = L.ah_caps()
        L.check(self.lib.ah_get_caps(self.h, C.byref(c)))
        return {"arch": c.arch.decode(), "cu_count": c.cu_count, "wavefront": c.wavefront,
                "hbm_bytes": c.hbm_bytes, "lds_bytes_per_block": c.lds_bytes_per_block,
                "has_f16": bool(c.has_f16), "has_bf16": bool(c.has_bf16)}

    def buffer(self, arr_or_n, dtype: int = L.AH_F32) -> DeviceBuffer:
        if isinstance(arr_or_n, np.ndarray):
            b = DeviceBuffer(self, arr_or_n.size, dtype)
            return b.write(arr_or_n)
        return DeviceBuffer(self, int(arr_or_n), dtype)

    def sync(self) -> None:
        L.check(self.lib.ah_sync(self.h))

    def timer_start(self) -> None:
        L.check(self.lib.ah_timer_start(self.h))

    def timer_stop(self) -> float:
        """Milliseconds of device-stream time since timer_start (waits for the stream)."""
        ms = C.c_double()
        L.check(self.lib.ah_timer_stop(self.h, C.byref(ms)))
        return ms.value

    @staticmethod
    def _gemm_desc(dtype, epi, ta, tb, M, N, K, A, B, lda, ldb, C_out=None, ldc=0, bias=None, aux=None, ldaux=0,
                   scale=1.0, colsum=None, W32=None, W16=None, lr=0.0, gout=None, lossacc=None, tile=0, variant=0):
        p = lambda b: None if b is None else b.ptr  # noqa: E731
        return L.ah_gemm_desc(dtype=dtype, epi=epi, ta=ta, tb=tb, M=M, N=N, K=K, A=p(A), B=p(B), lda=lda, ldb=ldb,
                              C=p(C_out), ldc=ldc, bias=p(bias), aux=p(aux), ldaux=ldaux, scale=scale,
                              colsum=p(colsum), W32=p(W32), W16=p(W16), lr=lr, gout=p(gout), lossacc=p(lossacc),
                              tile=tile, variant=variant)

    def gemm(self, **kw):
        """One contraction with a fused epilogue (keyword arguments mirror ah_gemm_desc)."""
        d = self._gemm_desc(**kw)
        L.check(self.lib.ah_gemm(self.h, C.byref(d)))

    def gemm_tune(self, iterations: int = 3, **kw):
        """Times every f16 variant (or f32 configuration) of the contraction and caches the fastest;
        returns (variant or configuration index, mean us)."""
        d = self._gemm_desc(**kw)
        v, us = C.c_int32(), C.c_double()
        L.check(self.lib.ah_gemm_tune(self.h, C.byref(d), iterations, C.byref(v), C.byref(us)))
        return v.value, us.value

    def gemm_tune_cache(self, path: str, save: bool) -> None:
        """Saves the tuned f16 variants and f32 configurations to path, or merges a saved file into this device's cache."""
        L.check(self.lib.ah_gemm_tune_cache(self.h, str(path).encode(), 1 if save else 0))

    def softmax_ce(self, z: DeviceBuffer, labels: DeviceBuffer, B: int, Cn: int, dz: DeviceBuffer,
                   loss: DeviceBuffer) -> None:
        L.check(self.lib.ah_softmax_ce(self.h, z.ptr, labels.ptr, B, Cn, dz.ptr, loss.ptr))

    def chain_step(self, X, g, R, Cc, dX, dg, loss) -> None:
        L.check(self.lib.ah_chain_step(self.h, X.ptr, g.ptr, R, Cc, dX.ptr, dg.ptr, loss.ptr))

    def chain_step_noalloc(self, X, g, R, Cc, dX, dg, loss) -> None:
        """chain_step with the workspace in the library's per-GPU static array (enqueues only)."""
        L.check(self.lib.ah_chain_step_noalloc(self.h, X.ptr, g.ptr, R, Cc, dX.ptr, dg.ptr, loss.ptr))

    def close(self) -> None:
        if self.h:
            self.lib.ah_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


class Trainer:
    """One BASELINE config's device-resident training step (slot numbering in include/anneal_hip.h)."""

    SLOTS = {
        L.TRAIN_MLP_CE: ["x", "labels", "W1", "b1", "W2", "b2", "loss", "dW1", "db1", "dW2", "db2", "H1"],
        L.TRAIN_CONVNET: ["x", "labels", "cw1", "cb1", "cw2", "cb2", "fw", "fb", "loss", "dcw1", "dcb1", "dcw2",
                          "dcb2", "dfw", "dfb"],
        L.TRAIN_MLP3_F16: ["x", "t", "W1", "b1", "W2", "b2", "W3", "b3", "loss", "dW1", "db1", "dW2", "db2", "dW3",
                           "db3", "loss_sum", "H1", "H2", "d"],
        L.TRAIN_CHAIN: ["X", "g", "loss", "dX", "dg"],
    }

    def __init__(self, dev: Device, kind: int, dims, lr: float = 0.0):
        self.dev, self.kind, self.dims = dev, kind, list(dims)
        arr = (C.c_int64 * len(dims))(*dims)
        h = C.c_void_p()
        L.check(dev.lib.ah_trainer_create(dev.h, kind, arr, len(dims), C.c_float(lr), C.byref(h)))
        self.h = h.value
        self.slots = {n: i for i, n in enumerate(self.SLOTS[kind])}

    def set(self, name: str, arr: np.ndarray) -> None:
        a = np.ascontiguousarray(arr)
        if a.dtype not in (np.float32, np.int32):
            a = a.astype(np.float32)
        L.check(self.dev.lib.ah_trainer_set(self.h, self.slots[name], a.ctypes.data, a.size))

    def get(self, name: str, n: int, dtype=np.float32) -> np.ndarray:
        out = np.empty(n, dtype=dtype)
        L.check(self.dev.lib.ah_trainer_get(self.h, self.slots[name], out.ctypes.data, n))
        return out

    def step(self, batch: int, store_grads: bool = False, graph: bool = False) -> None:
        flags = (L.STEP_STORE_GRADS if store_grads else 0) | (L.STEP_GRAPH if graph else 0)
        L.check(self.dev.lib.ah_trainer_step(self.h, int(batch), flags))

    def steps(self, batch: int, n: int, store_grads: bool = False, graph: bool = False) -> None:
        """n consecutive steps; with graph=True as hipGraph launches of up to 16 steps each."""
        flags = (L.STEP_STORE_GRADS if store_grads else 0) | (L.STEP_GRAPH if graph else 0)
        L.check(self.dev.lib.ah_trainer_steps(self.h, int(batch), flags, int(n)))

    def probe(self, kernel_index: int) -> None:
        L.check(self.dev.lib.ah_trainer_probe(self.h, kernel_index))

    def probe_span(self, first: int, last: int) -> None:
        """hipEvents before launch `first` and after launch `last` of each following step."""
        L.check(self.dev.lib.ah_trainer_probe_span(self.h, first, last))

    def probe_read(self):
        ms, n = C.c_double(), C.c_int64()
        L.check(self.dev.lib.ah_trainer_probe_read(self.h, C.byref(ms), C.byref(n)))
        return ms.value, n.value

    def kernel_count(self, batch: int) -> int:
        c = C.c_int32()
        L.check(self.dev.lib.ah_trainer_kernel_count(self.h, int(batch), C.byref(c)))
        return c.value

    def kernel_names(self, batch: int) -> list:
        """Names of the step's launches in order (ah_trainer_kernel_count, then ah_trainer_kernel_name)."""
        n = self.kernel_count(batch)
        buf = C.create_string_buffer(64)
        out = []
        for i in range(n):
            L.check(self.dev.lib.ah_trainer_kernel_name(self.h, i, buf, 64))
            out.append(buf.value.decode())
        return out

    def close(self) -> None:
        if self.h:
            self.dev.lib.ah_trainer_destroy(self.h)
            self.h = None
