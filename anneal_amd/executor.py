"""backend.Executor / Benchmarker / SymbolicExecutor mirror over the C ABI (backend/device.go:10-37),
and Plan, the device half of tensor.JIT (tensor/jit.go:47-359).

ExecItem fields follow schedule/exec.go:6-32; `source` replaces the WGSL string and is HIP source
(compiled once per device by hiprtc) or a "tmpl:" key naming a hand-written kernel.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field

import numpy as np

from . import _lib as L


@dataclass
class Buffer:
    uop_idx: int
    size: int
    shape: list
    dtype: int = L.AH_F32
    slot: int = -1


@dataclass
class ExecItem:
    source: str
    bufs: list
    sym_vars: list = field(default_factory=list)
    local_size: tuple = (64, 1, 1)
    workgroup_count: tuple = (1, 1, 1)


@dataclass
class BenchmarkResult:
    min_us: float
    median_us: float
    max_us: float
    mean_us: float
    stddev_us: float
    cv: float


class _Marshal:
    """Keeps the ctypes arrays alive for the duration of one call."""

    def __init__(self, items):
        self.keep = []
        self.arr = (L.ah_exec_item * len(items))()
        for i, it in enumerate(items):
            bufs = (L.ah_buffer_desc * len(it.bufs))()
            for j, b in enumerate(it.bufs):
                shp = (C.c_int64 * max(len(b.shape), 1))(*b.shape)
                self.keep.append(shp)
                bufs[j] = L.ah_buffer_desc(b.uop_idx, b.size, b.dtype, b.slot, len(b.shape),
                                           C.cast(shp, C.POINTER(C.c_int64)))
            sv = (C.c_char_p * max(len(it.sym_vars), 1))(*[s.encode() for s in it.sym_vars])
            src = it.source.encode()
            self.keep += [bufs, sv, src]
            self.arr[i] = L.ah_exec_item(src, C.cast(bufs, C.POINTER(L.ah_buffer_desc)), len(it.bufs),
                                         C.cast(sv, C.POINTER(C.c_char_p)), len(it.sym_vars),
                                         (C.c_int32 * 3)(*it.local_size), (C.c_int32 * 3)(*it.workgroup_count))


class Executor:
    """Run / RunSymbolic / Benchmark with the reference's argument meaning and error behaviour."""

    def __init__(self, device):
        self.dev = device

    def _inputs(self, inputs: dict):
        arr = (L.ah_input * max(len(inputs), 1))()
        keep = []
        for i, (k, v) in enumerate(inputs.items()):
            a = np.ascontiguousarray(v, dtype=np.float32)
            keep.append(a)
            arr[i] = L.ah_input(k, a.ctypes.data_as(C.POINTER(C.c_float)), a.size)
        return arr, keep

    def _collect(self, outs, n):
        res = {}
        for i in range(n.value):
            o = outs[i]
            res[o.uop_idx] = np.ctypeslib.as_array(o.data, shape=(o.n,)).copy()
        self.dev.lib.ah_outputs_free(outs, n)
        return res

    def _bind(self, binding: dict):
        names = (C.c_char_p * max(len(binding), 1))(*[k.encode() for k in binding])
        vals = (C.c_int64 * max(len(binding), 1))(*binding.values())
        return names, vals

    def run(self, items, inputs: dict) -> dict:
        m = _Marshal(items)
        ins, keep = self._inputs(inputs)
        outs, n = C.POINTER(L.ah_output)(), C.c_int32()
        L.check(self.dev.lib.ah_run(self.dev.h, m.arr, len(items), ins, len(inputs), C.byref(outs), C.byref(n)))
        _ = keep
        return self._collect(outs, n)

    def run_symbolic(self, items, inputs: dict, binding: dict) -> dict:
        m = _Marshal(items)
        ins, keep = self._inputs(inputs)
        names, vals = self._bind(binding)
        outs, n = C.POINTER(L.ah_output)(), C.c_int32()
        L.check(self.dev.lib.ah_run_symbolic(self.dev.h, m.arr, len(items), ins, len(inputs), names, vals,
                                             len(binding), C.byref(outs), C.byref(n)))
        _ = keep
        return self._collect(outs, n)

    def benchmark(self, item, warmup: int, iterations: int) -> BenchmarkResult:
        m = _Marshal([item])
        r = L.ah_bench_result()
        L.check(self.dev.lib.ah_benchmark(self.dev.h, m.arr, warmup, iterations, C.byref(r)))
        return BenchmarkResult(r.min_us, r.median_us, r.max_us, r.mean_us, r.stddev_us, r.cv)


class Plan:
    """An item list kept alive on the device: kernels resolved and buffers allocated once, and with
    graph=True each binding's kernel sequence captured once as a HIP graph and replayed afterwards.
    run() has Run / RunSymbolic's contract (binding None for a static list)."""

    def __init__(self, device, items, graph: bool = True):
        self.dev, self.ex, self.graph = device, Executor(device), graph
        m = _Marshal(items)
        h = C.c_void_p()
        L.check(device.lib.ah_plan_create(device.h, m.arr, len(items), C.byref(h)))
        self.h = h.value

    def run(self, inputs: dict, binding: dict | None = None) -> dict:
        ins, keep = self.ex._inputs(inputs)
        binding = binding or {}
        names, vals = self.ex._bind(binding)
        outs, n = C.POINTER(L.ah_output)(), C.c_int32()
        L.check(self.dev.lib.ah_plan_run(self.h, ins, len(inputs), names, vals, len(binding),
                                         L.PLAN_GRAPH if self.graph else 0, C.byref(outs), C.byref(n)))
        _ = keep
        return self.ex._collect(outs, n)

    def stats(self):
        """(captures, replays), as tensor.JIT.JITStats."""
        c, r = C.c_int64(), C.c_int64()
        L.check(self.dev.lib.ah_plan_stats(self.h, C.byref(c), C.byref(r)))
        return c.value, r.value

    def close(self) -> None:
        if self.h:
            self.dev.lib.ah_plan_destroy(self.h)
            self.h = None
