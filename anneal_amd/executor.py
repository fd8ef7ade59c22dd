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


@dataclass
class BeamResult:
    opts: list          # [(kind, axis, arg), ...]; empty: the unmodified kernel won
    min_us: float
    base_us: float
    searched: int
    from_cache: bool


def _key_out(fn, *args) -> str:
    need = C.c_int64()
    L.check(fn(*args, None, 0, C.byref(need)))
    buf = C.create_string_buffer(need.value)
    L.check(fn(*args, buf, need.value, C.byref(need)))
    return buf.value.decode()


def apply_opts(key: str, opts) -> str:
    """codegen.ApplyOpts on a template key: the key with the Opt sequence applied to its parameters."""
    arr = (L.ah_opt * max(len(opts), 1))(*[L.ah_opt(*o) for o in opts])
    return _key_out(L.load().ah_apply_opts, key.encode(), arr, len(opts))


def action_space(key: str) -> list:
    """codegen.ActionSpace: every single Opt (kind, axis, arg) that changes the key's kernel."""
    lib = L.load()
    n = C.c_int32()
    L.check(lib.ah_action_space(key.encode(), None, 0, C.byref(n)))
    arr = (L.ah_opt * max(n.value, 1))()
    L.check(lib.ah_action_space(key.encode(), arr, n.value, C.byref(n)))
    return [(o.kind, o.axis, o.arg) for o in arr[:n.value]]


def beam_apply(key: str) -> str:
    """The cached BEAM winner's key for key (or key itself on a miss)."""
    return _key_out(L.load().ah_beam_apply, key.encode())


def beam_cache(path: str, save: bool) -> None:
    L.check(L.load().ah_beam_cache(str(path).encode(), 1 if save else 0))


def beam_reset() -> None:
    L.load().ah_beam_reset()


def beam_search(device, item, width: int = 4, depth: int = 4, warmup: int = 2, iters: int = 5) -> BeamResult:
    """codegen.BeamSearch over the template parameters of a "tmpl:" item (cached per process)."""
    m = _Marshal([item])
    r = L.ah_beam_result()
    L.check(device.lib.ah_beam_search(device.h, m.arr, width, depth, warmup, iters, C.byref(r)))
    return BeamResult([(o.kind, o.axis, o.arg) for o in r.opts[:r.n_opts]], r.min_us, r.base_us, r.searched,
                      bool(r.from_cache))


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
