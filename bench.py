"""Benchmark of anneal's training hot path on one MI355X.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 3]
  python bench.py --library-probe     (config-3 GEMM shapes here vs hipBLASLt, store epilogue;
                                       with --config 4 the config-4 f32 shapes at N = 4096)

One "step" is one full training step of a BASELINE config (forward, backward, SGD) with inputs and
parameters resident in HBM. Prints ONE JSON line: steps/s for the config, the roofline of its dominant
kernel (timed live with hipEvents on the library's stream during the timed steps), per-kernel timings,
and a CPU baseline (the oracle restatement, timed on a bounded sample on the host cores).
The default workload is config 3 (f16 GEMM-bound MLP), the config the north-star roofline target names.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_F16 = 2.5e15     # MI355X dense f16/bf16 MFMA, FLOP/s
PEAK_F32 = 157.3e12   # MI355X f32 matrix/vector, FLOP/s
PEAK_HBM = 8.0e12     # MI355X HBM3E, B/s

# HBM bytes per launch of the dominant kernels, from rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs
# scaled by a plain copy of known size (read factor 2.0, write factor 1.0): profiles/hbm_traffic_pmc.md,
# profiles/chain_resident_config5.md.
# The CPU baseline is the oracle (a C restatement of the reference's step, OpenMP over the host cores);
# the reference's own WebGPU path needs Go and a software Vulkan adapter, neither of which is on the box.
CPU_LABEL = "CPU restatement \u2014 not the reference binary"

TRAFFIC_BYTES = {(3, "dW2"): 270.7e6 + 102.8e6, (5, "chain_resident"): 135.2e6 + 136.0e6,
                 (5, "chain_grad"): 134.4e6 + 134.4e6,
                 (5, "chain_stats"): 134.3e6 + 4.2e6}


def config_workload(cfg: int, batch4: int = 4096):
    """Returns (trainer kind, dims, lr, batch, inputs dict, kernels [(name, kind, amount)], meta)."""
    from anneal_amd import _lib as L
    from anneal_amd import data
    if cfg == 3:
        B, D0, D1, D2, D3 = 4096, 1024, 4096, 4096, 1024
        p = data.mlp3_inputs(B, D0, D1, D2, D3)
        f = lambda m, n, k: ("flop16", 2.0 * m * n * k)  # noqa: E731
        ks = [("fc1", *f(B, D1, D0)), ("fc2", *f(B, D2, D1)), ("fc3_mse", *f(B, D3, D2)), ("dH2", *f(B, D2, D3)),
              ("dW3", *f(D3, D2, B)), ("dH1", *f(B, D1, D2)), ("dW2", *f(D2, D1, B)), ("dW1", *f(D1, D0, B)),
              # the tail's distinct bytes: the partial rows of the bias gradients that the step's
              # contractions write (every second of R = B/32 for db1 and db2 from the 64-row waves of
              # the 256x256 tiles, all R for db3 from fc3's k-group tiles), read once; the R x D3/32 loss
              # partials read and re-zeroed; then f32 bias read + write and f16 write
              ("tail", "bytes", 4 * (B // 64) * (D1 + D2) + 4 * (B // 32) * D3 + 8 * (B // 32) * (D3 // 32)
               + 10 * (D1 + D2 + D3))]
        meta = {"workload": "config3_f16_mlp_1024-4096-4096-1024_b4096_mse_sgd", "batch": B,
                "flop_per_step": sum(a for _, k, a in ks if k.startswith("flop")), "dtype": "f16"}
        return L.TRAIN_MLP3_F16, [B, D0, D1, D2, D3], 1e-3, B, p, ks, meta
    if cfg == 5:
        R, Cc = 8192, 4096
        p = data.chain_inputs(R, Cc)
        ks = [("chain_resident", "bytes", 8.0 * R * Cc),
              ("chain_stats", "bytes", 4.0 * R * Cc), ("chain_finalize", "bytes", 0.0),
              ("chain_grad", "bytes", 8.0 * R * Cc)]
        meta = {"workload": "config5_chain_8192x4096_permute_pad_shrink_softmax_rmsnorm", "batch": Cc,
                "bytes_per_step": 8.0 * R * Cc + 8 * Cc, "dtype": "f32"}
        return L.TRAIN_CHAIN, [R, Cc], 0.0, R, p, ks, meta
    if cfg in (1, 4):
        B, D, H, C = (64, 784, 128, 10) if cfg == 1 else (batch4, 512, 2048, 512)
        p = data.mlp_ce_inputs(B, D, H, C, **({} if cfg == 1 else {"x_lo": -1.0, "x_hi": 1.0}))
        ks = mlp_ce_kernels(B, D, H, C)
        wl = "config1_mlp_784-128-10_b64_f32" if cfg == 1 else f"config4_dynmlp_512-2048-512_f32_N{B}"
        meta = {"workload": wl, "batch": B, "dtype": "f32",
                "flop_per_step": sum(a for _, k, a in ks if k.startswith("flop"))}
        return L.TRAIN_MLP_CE, [B, D, H, C], 0.01, B, p, ks, meta
    if cfg == 2:
        p = data.convnet_inputs()
        ks = convnet_kernels()
        meta = {"workload": "config2_convnet_b32_f32", "batch": 32, "dtype": "f32",
                "flop_per_step": sum(a for _, k, a in ks if k.startswith("flop"))}
        return L.TRAIN_CONVNET, [32, 28, 8, 16, 10], 0.01, 32, p, ks, meta
    raise SystemExit(f"bench: unknown config {cfg}")


def cpu_baseline(cfg: int, inputs: dict, full: bool = False):
    """Oracle (CPU restatement, OpenMP over the host cores) on a bounded sample of the same workload,
    about 10-20 s of CPU work; full=True times config 3's whole batch-4096 step once (about a minute)."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as O
    threads = O.load().ora_num_threads()
    if cfg == 3:
        from anneal_amd.data import f16_quantize
        Bs = 4096 if full else 1024
        q = {k: v for k, v in inputs.items()}
        q["x"], q["t"] = f16_quantize(inputs["x"][:Bs]), f16_quantize(inputs["t"][:Bs])
        t0 = time.perf_counter()
        O.mlp3_step(q, 1e-3)
        dt = time.perf_counter() - t0
        full = dt * (4096 / Bs)   # seconds per full step
        if Bs == 4096:
            sample = f"one full oracle step (batch 4096, full layer widths), {dt:.1f} s"
        else:
            sample = f"one oracle step at batch {Bs} of 4096 (full layer widths), {dt:.1f} s, scaled x{4096 // Bs} to a full step"
        return {"value": 1.0 / full, "unit": "train steps/s", "cores": threads, "kind": "port",
                "label": CPU_LABEL, "sample": sample}
    if cfg == 4:
        B = len(inputs["labels"])
        Bs = min(512, B)
        q = dict(inputs)
        q["x"], q["labels"] = inputs["x"][:Bs], inputs["labels"][:Bs]
        t0 = time.perf_counter()
        O.mlp_ce_step(q, 0.01)
        dt = time.perf_counter() - t0
        return {"value": Bs / (dt * B), "unit": "train steps/s", "cores": threads, "kind": "port",
                "label": CPU_LABEL,
                "sample": f"one oracle step at batch {Bs} of {B}, {dt:.1f} s, scaled x{B / Bs:g} to a full step"}
    if cfg in (1, 2):
        n, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < 10.0:
            if cfg == 2:
                O.convnet_step(inputs, 0.01)
            else:
                O.mlp_ce_step(inputs, 0.01)
            n += 1
        dt = time.perf_counter() - t0
        return {"value": n / dt, "unit": "train steps/s", "cores": threads, "kind": "port",
                "label": CPU_LABEL, "sample": f"{n} full oracle steps in {dt:.1f} s"}
    if cfg == 5:
        n, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < 10.0:
            O.chain_step(inputs["X"], inputs["g"])
            n += 1
        dt = time.perf_counter() - t0
        return {"value": n / dt, "unit": "train steps/s", "cores": threads, "kind": "port",
                "label": CPU_LABEL, "sample": f"{n} full oracle steps (X[8192,4096]) in {dt:.1f} s"}
    return None


def mlp_ce_kernels(B, D, H, C):
    """The MLP_CE trainer's launches (configs 1 and 4) with their algorithmic work. Shapes up to
    B = 64, D = 896, H = 128, C = 16 (config 1) take the three-kernel step (hidden layer; softmax-CE
    and dH; weight gradients with SGD), batches up to 8 at wider layers (config 4 at N = 1, 7) a
    four-kernel step (the two layers; softmax-CE and dH; one streaming pass of SGD over W1 and W2),
    the rest the GEMM-based step."""
    f = lambda m, n, k: ("flop32", 2.0 * m * n * k)  # noqa: E731
    if B <= 8 and D % 4 == 0 and H % 4 == 0 and C <= 512 and not (D <= 896 and H <= 128 and C <= 16):
        return [("fc1", *f(B, H, D)), ("fc2", *f(B, C, H)), ("dH1", *f(B, H, C)),
                ("grad", "bytes", 4.0 * (2 * (H * D + C * H) + B * (D + H + C)))]
    if B <= 64 and D <= 896 and H <= 128 and C <= 16:
        return [("hidden", *f(B, H, D)), ("head", "flop32", 2 * 2.0 * B * C * H),
                ("grad", "flop32", 2.0 * B * H * D + 2.0 * B * C * H)]
    # softmax-CE (C <= 1024) also writes the output bias gradient's column sums as min(256, B/16)
    # partial rows, which the tail sums; a wider C takes a separate column-sum launch (db2)
    parts = min(256, max(1, (B + 15) // 16)) if C <= 1024 else 0
    return [("fc1", *f(B, H, D)), ("fc2", *f(B, C, H)), ("softmax_ce", "bytes", 8.0 * B * C + 8.0 * B + 4.0 * parts * C),
            ("db2", "bytes", 4.0 * B * C), ("dH1", *f(B, H, C)), ("dW1", *f(H, D, B)), ("dW2", *f(C, H, B)),
            ("tail", "bytes", 4.0 * B + 16.0 * (H + C) + 4.0 * parts * C)]


def convnet_kernels(N=32, Hin=28, C1=8, C2=16, NC=10):
    """The CONVNET trainer's launches (config 2) with their algorithmic work: the forward and backward
    kernels (direct-convolution and fc FLOPs; conv1 has no input gradient), then the tail, which reads
    the N per-sample gradient rows and reads/writes each parameter and its gradient."""
    P1, P2 = Hin // 2, Hin // 4
    F = C2 * P2 * P2
    c1 = 2.0 * N * C1 * Hin * Hin * 9          # conv1: Ci = 1
    c2 = 2.0 * N * C2 * P1 * P1 * 9 * C1       # conv2
    fc = 2.0 * N * NC * F
    nparam = C1 * 10 + C2 * C1 * 9 + C2 + NC * F + NC
    return [("convnet_fwd", "flop32", c1 + c2 + fc), ("convnet_bwd", "flop32", c1 + 2 * c2 + 2 * fc),
            ("tail", "bytes", 4.0 * N * nparam + 12.0 * nparam)]


def step_kernels(t, batch, kernels):
    """The step's launches as (name, kind, amount), in launch order: the trainer's own launch names looked
    up in `kernels`; a paired launch "a+b" carries the sum of a's and b's work. Falls back to `kernels`
    by position when a name is not listed."""
    names = t.kernel_names(batch)
    known = {k[0]: k for k in kernels}
    out = []
    for n in names:
        parts = [known.get(x) for x in n.split("+")]
        if any(q is None for q in parts) or len({q[1] for q in parts}) != 1:
            assert len(names) == len(kernels), (names, kernels)
            return list(kernels)
        out.append((n, parts[0][1], sum(q[2] for q in parts)))
    return out


def kernel_table(t, batch, kernels, steps=20, warmup=50):
    """Average duration of each launch of the step (hipEvents on the trainer's stream, eager steps), the
    dominant one's roofline, and the per-kernel entries. A launch's duration is the difference of two
    probes that differ by that launch alone: events before launch i-1 and after launch i, less events
    before launch i-1 and after launch i-1 (for launch 0: events around it, less the two events back to
    back). The events' own cost is in both terms and cancels, so the launches' durations add up to the
    step: each is the kernel's run time plus the dispatch gap in front of it. `warmup` untimed steps run
    first, whatever the command line's --warmup, so the first kernels probed see the same clocks and
    cache state as the last."""
    kernels = step_kernels(t, batch, kernels)
    nk = t.kernel_count(batch)
    assert nk == len(kernels), (nk, len(kernels))
    for _ in range(warmup):
        t.step(batch)

    def span(first, last):
        t.probe_span(first, last)
        for _ in range(steps):
            t.step(batch)
        ms, n = t.probe_read()
        return ms / max(n, 1)
    per = []
    for i in range(nk):
        j = max(i - 1, 0)
        per.append(max(span(j, i) - span(j, i - 1), 1e-6))
    t.probe(-1)
    rows = []
    for (kname, kkind, amt), ms in zip(kernels, per):
        e = {"name": kname, "avg_us": round(ms * 1e3, 2)}
        if kkind.startswith("flop"):
            tf = amt / (ms / 1e3) / 1e12 if ms > 0 else 0.0
            e.update(tflops=round(tf, 3), frac=round(tf * 1e12 / (PEAK_F16 if kkind == "flop16" else PEAK_F32), 4))
        elif amt > 0:
            gbs = amt / (ms / 1e3) / 1e9 if ms > 0 else 0.0
            e.update(gbs=round(gbs, 1), frac=round(gbs * 1e9 / PEAK_HBM, 4))
        rows.append(e)
    dom = int(np.argmax(per))
    name, kk, amount = kernels[dom]
    s = per[dom] / 1e3
    if kk.startswith("flop"):
        peak = PEAK_F16 if kk == "flop16" else PEAK_F32
        roof = {"kernel": name, "bound": "mfma", "achieved": amount / s / 1e12, "peak": peak / 1e12, "unit": "TFLOP/s"}
    else:
        roof = {"kernel": name, "bound": "hbm", "achieved": amount / s / 1e9, "peak": PEAK_HBM / 1e9, "unit": "GB/s"}
    roof["frac"] = roof["achieved"] / roof["peak"]
    roof["avg_us"] = per[dom] * 1e3
    return roof, rows


def other_configs(dev, skip: int) -> dict:
    """Each other BASELINE config at its own shape: steps/s (graph replay of the device-resident step,
    the tensor.JIT pattern; config 4 per bound batch N) and the roofline of its dominant kernel with the
    per-kernel table (eager steps, hipEvents around each launch). Parity for each is in tests/."""
    from anneal_amd import _lib as L
    from anneal_amd import data
    from anneal_amd.backend import Trainer

    def rate(t, batch, steps, graph, per_launch=None):
        # steps run by one library call (ah_trainer_steps): eager launches, or hipGraphs of up to 16 steps;
        # per_launch=1 replays a one-step graph per step instead (one hipGraphLaunch per step)
        def run(n):
            if per_launch == 1:
                for _ in range(n):
                    t.step(batch, graph=True)
            else:
                t.steps(batch, n, graph=graph)
        run(min(steps, 32))
        dev.sync()
        t0 = time.perf_counter()
        run(steps)
        dev.sync()
        return steps / (time.perf_counter() - t0)

    def entry(t, batch, kernels, steps=50, cfg=None, jit=False):
        # eager launches and hipGraph replay both timed; jit=True (config 4: the step captured once by
        # tensor.JIT and replayed) reports the graph replay as the config's rate
        eager, graph = rate(t, batch, steps, False), rate(t, batch, steps, True)
        graph1 = rate(t, batch, steps, True, per_launch=1)
        roof, rows = kernel_table(t, batch, kernels)
        if cfg is not None and (cfg, roof["kernel"]) in TRAFFIC_BYTES:
            roof["traffic"] = TRAFFIC_BYTES[(cfg, roof["kernel"])]   # measured HBM bytes per launch
        return {"steps_per_s": graph if jit else max(eager, graph), "eager_steps_per_s": eager,
                "graph_steps_per_s": graph, "graph_1step_launch_steps_per_s": graph1,
                "roofline": roof, "kernels": rows, "kernels_sum_us": round(sum(r["avg_us"] for r in rows), 2)}

    out = {}
    if skip != 1:
        p = data.mlp_ce_inputs(64, 784, 128, 10)
        t = Trainer(dev, L.TRAIN_MLP_CE, [64, 784, 128, 10], 0.01)
        for k in ("x", "labels", "W1", "b1", "W2", "b2"):
            t.set(k, p[k])
        out["config1_mlp_784-128-10_b64_f32"] = entry(t, 64, mlp_ce_kernels(64, 784, 128, 10))
        t.close()
    if skip != 2:
        p = data.convnet_inputs()
        t = Trainer(dev, L.TRAIN_CONVNET, [32, 28, 8, 16, 10], 0.01)
        for k in ("x", "labels", "cw1", "cb1", "cw2", "cb2", "fw", "fb"):
            t.set(k, p[k])
        out["config2_convnet_b32_f32"] = entry(t, 32, convnet_kernels())
        t.close()
    if skip != 4:
        p = data.mlp_ce_inputs(4096, 512, 2048, 512, x_lo=-1.0, x_hi=1.0)
        t = Trainer(dev, L.TRAIN_MLP_CE, [4096, 512, 2048, 512], 0.01)
        for k in ("x", "labels", "W1", "b1", "W2", "b2"):
            t.set(k, p[k])
        out["config4_dynmlp_512-2048-512_f32"] = {f"N={n}": entry(t, n, mlp_ce_kernels(n, 512, 2048, 512), 100, jit=True)
                                                  for n in (1, 7, 256, 4096)}
        t.close()
    if skip != 5:
        kind, dims, lr, batch, p, ks, _ = config_workload(5)
        t = Trainer(dev, kind, dims, lr)
        for k, v in p.items():
            t.set(k, v)
        out["config5_chain_8192x4096_f32"] = entry(t, batch, ks, cfg=5)
        t.close()
    if skip != 3:
        kind, dims, lr, batch, p, ks, _ = config_workload(3)
        t = Trainer(dev, kind, dims, lr)
        for k, v in p.items():
            t.set(k, v)
        out["config3_f16_mlp_b4096"] = entry(t, batch, ks, 20)
        t.close()
    # config 3 with the reference's f32 adjoints (dims[5] = 1: the masked adjoints as two f16 planes, so
    # dH1, dW2 and dW1 contract twice over K); the kernel table's FLOP figures stay the algorithmic ones
    kind, dims, lr, batch, p, ks, _ = config_workload(3)
    t = Trainer(dev, kind, dims + [1], lr)
    for k, v in p.items():
        t.set(k, v)
    out["config3_f16_mlp_b4096_f32_adjoint"] = entry(t, batch, ks, 20)
    t.close()
    return out


def copy_probe(mib: int):
    """Plain copy of a known size: FETCH_SIZE / WRITE_SIZE of this kernel calibrate the HBM counters."""
    import torch
    n = mib * (1 << 20) // 4
    a = torch.ones(n, dtype=torch.float32, device="cuda:0")
    b = torch.empty_like(a)
    for _ in range(5):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_bytes_read": n * 4, "copy_probe_bytes_written": n * 4, "launches": 5}))


def library_probe(cfg: int = 3, batch: int = 4096):
    """A config's contractions with a plain store epilogue: this library (each shape tuned, then timed)
    next to hipBLASLt (torch.matmul on the same layouts), 20 launches each, hipEvents. Config 3: the
    eight f16 shapes; config 4: the five f32 shapes at N = batch (torch with TF32 off, so both run the
    f32 MFMA path)."""
    import torch
    from anneal_amd import _lib as L
    from anneal_amd.backend import Device
    dev = Device(0)
    if cfg == 4:
        torch.backends.cuda.matmul.allow_tf32 = False
        N, D, H, C = batch, 512, 2048, 512
        shapes = [("fc1", 0, 0, N, H, D), ("fc2", 0, 0, N, C, H), ("dH1", 0, 1, N, H, C), ("dW2", 1, 1, C, H, N),
                  ("dW1", 1, 1, H, D, N)]
        dt, ndt, tdt = L.AH_F32, np.float32, torch.float32
    else:
        B, D0, D1, D2, D3 = 4096, 1024, 4096, 4096, 1024
        shapes = [("fc1", 0, 0, B, D1, D0), ("fc2", 0, 0, B, D2, D1), ("fc3", 0, 0, B, D3, D2), ("dH2", 0, 1, B, D2, D3),
                  ("dW3", 1, 1, D3, D2, B), ("dH1", 0, 1, B, D1, D2), ("dW2", 1, 1, D2, D1, B), ("dW1", 1, 1, D1, D0, B)]
        dt, ndt, tdt = L.AH_F16, np.float16, torch.float16
    rng = np.random.default_rng(0)
    big = max(max(M * K, N_ * K, M * N_) for _, _, _, M, N_, K in shapes)   # elements of the largest operand
    A = dev.buffer((rng.standard_normal(big) * 0.1).astype(ndt), dt)
    Bb = dev.buffer((rng.standard_normal(big) * 0.1).astype(ndt), dt)
    Cc = dev.buffer(big, dt)
    rows = []
    for name, ta, tb, M, N, K in shapes:
        kw = dict(dtype=dt, epi=L.EPI_STORE, ta=ta, tb=tb, M=M, N=N, K=K, A=A, B=Bb, lda=M if ta else K,
                  ldb=N if tb else K, C_out=Cc, ldc=N, scale=1.0)
        variant, _ = dev.gemm_tune(iterations=3, **kw)
        for _ in range(3):
            dev.gemm(**kw)
        dev.sync()
        dev.timer_start()
        for _ in range(20):
            dev.gemm(**kw)
        ours = dev.timer_stop() / 20 * 1e3
        a = torch.randn((K, M) if ta else (M, K), device="cuda", dtype=tdt)
        b = torch.randn((K, N) if tb else (N, K), device="cuda", dtype=tdt)
        a2, b2 = (a.t() if ta else a), (b if tb else b.t())
        for _ in range(3):
            c = a2 @ b2
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(20):
            c = a2 @ b2
        e1.record()
        torch.cuda.synchronize()
        blas = e0.elapsed_time(e1) / 20 * 1e3
        fl = 2.0 * M * N * K
        rows.append({"gemm": name, "M": M, "N": N, "K": K, "ta": ta, "tb": tb, "variant": variant,
                     "us": round(ours, 1), "tflops": round(fl / ours / 1e6), "hipblaslt_us": round(blas, 1),
                     "hipblaslt_tflops": round(fl / blas / 1e6)})
    print(json.dumps({"library_probe": rows, "config": cfg}))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--config", type=int, default=3)
    ap.add_argument("--batch", type=int, default=4096, help="config 4's batch N (1 to 4096)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-full", action="store_true", help="config 3: time one whole batch-4096 oracle step")
    ap.add_argument("--no-others", action="store_true", help="skip the steps/s of the other configs")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="only run a plain device-to-device copy of MIB MiB 5 times (HBM counter calibration)")
    ap.add_argument("--library-probe", action="store_true",
                    help="only time the config-3 contraction shapes here and in hipBLASLt (store epilogue)")
    args = ap.parse_args()
    if args.library_probe:
        library_probe(args.config if args.config == 4 else 3, args.batch)
        return
    if args.copy_probe:
        copy_probe(args.copy_probe)
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU: sharding across GPUs is designed, not built",
                          "n_gpus": args.gpus}))
        sys.exit(2)

    from anneal_amd.backend import Device, Trainer
    if not 1 <= args.batch <= 4096:
        raise SystemExit("bench: --batch is 1 to 4096")
    kind, dims, lr, batch, p, kernels, meta = config_workload(args.config, args.batch)
    dev = Device(0)
    caps = dev.caps()
    t = Trainer(dev, kind, dims, lr)
    for k, v in p.items():
        t.set(k, v)
    for _ in range(args.warmup):
        t.step(batch)
    dev.sync()
    # Calibration (outside the timed region): 50 more untimed steps, then each kernel's average duration
    # over 20 steps.
    kernels = step_kernels(t, batch, kernels)
    _, kinfo = kernel_table(t, batch, kernels)
    dom = int(np.argmax([k["avg_us"] for k in kinfo]))
    # Timed region: K steps. The dominant kernel's duration is measured as in kernel_table, on steps of
    # the timed region itself: hipEvents before launch dom-1 and after launch dom on the first P steps,
    # before launch dom-1 and after launch dom-1 on the last P; the difference of the two averages is the
    # launch. P = K/20 (at least 1): each probe event costs the stream a few microseconds, which would be
    # a sixth of config 5's step if every step carried them. Reading the first probes' events
    # synchronizes the stream once, inside the timed region. Steps are enqueued by one library call per
    # run of steps (ah_trainer_steps), so a short step is not held up by a Python call per step.
    j = max(dom - 1, 0)
    P = max(1, args.steps // 20)
    rest = max(args.steps - 2 * P, 0)
    t.probe_span(j, dom)
    dev.sync()
    t0 = time.perf_counter()
    t.steps(batch, P)
    a_ms, a_n = t.probe_read()
    t.probe(-1)
    t.steps(batch, rest)
    t.probe_span(j, dom - 1)
    t.steps(batch, args.steps - P - rest)
    dev.sync()
    elapsed = time.perf_counter() - t0
    b_ms, b_n = t.probe_read()
    t.probe(-1)
    dom_ms, dom_n = (a_ms / max(a_n, 1) - (b_ms / b_n if b_n else 0.0)), 1
    dom_avg_s = dom_ms / max(dom_n, 1) / 1e3

    name, kk, amount = kernels[dom]
    if kk.startswith("flop"):
        peak = PEAK_F16 if kk == "flop16" else PEAK_F32
        roof = {"bound": "mfma", "achieved": amount / dom_avg_s / 1e12, "peak": peak / 1e12, "unit": "TFLOP/s"}
    else:
        roof = {"bound": "hbm", "achieved": amount / dom_avg_s / 1e9, "peak": PEAK_HBM / 1e9, "unit": "GB/s"}
    roof["frac"] = roof["achieved"] / roof["peak"]
    roof["traffic"] = TRAFFIC_BYTES.get((args.config, name))
    roof["kernel"] = name
    roof["avg_us"] = dom_avg_s * 1e6

    sps = args.steps / elapsed
    out = {
        "metric": "train steps/s + per-kernel TFLOP/s or HBM GB/s vs peak, 1xMI355X",
        "value": sps, "unit": "train steps/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": elapsed / args.steps * 1e3, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": meta["dtype"], "data": "synthetic (splitmix64 seed 0, anneal_amd/data.py)",
        "config": {"workload": meta["workload"], "batch": meta["batch"], "parallelism": "single-gpu"},
        "roofline": roof, "kernels": kinfo, "kernels_sum_us": round(sum(k["avg_us"] for k in kinfo), 2),
        "device": caps["arch"], "cu_count": caps["cu_count"],
    }
    if "flop_per_step" in meta:
        out["step_tflops"] = meta["flop_per_step"] * sps / 1e12
    out["cpu_baseline"] = None if args.no_cpu else cpu_baseline(args.config, p, full=args.cpu_full)
    t.close()
    if not args.no_others:
        out["other_configs"] = other_configs(dev, args.config)
    dev.close()
    print(json.dumps(out))


if __name__ == "__main__":
    main()
