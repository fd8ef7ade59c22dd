"""Synthetic inputs for the five BASELINE configs, from one language-neutral PRNG.

Every tensor is drawn from its own splitmix64 stream: state_i = (seed << 32 | tag) + i * 0x9E3779B97F4A7C15
(i = 1, 2, ...), output = the standard splitmix64 finaliser of state_i. Derived draws:

  uniform [0,1)   : (z >> 40) * 2**-24                       (exact in f32)
  uniform [a,b)   : a + (b - a) * u, evaluated in f64, rounded to f32
  normal N(0,1)   : Box-Muller on consecutive pairs (z_2i, z_2i+1):
                    u1 = ((z_2i >> 11) + 1) * 2**-53, u2 = (z_2i+1 >> 11) * 2**-53,
                    n  = sqrt(-2 ln u1) * cos(2 pi u2)   (f64, rounded to f32)
  labels          : (z >> 32) % classes, as int32
  Kaiming uniform : U(-sqrt(6/fan_in), sqrt(6/fan_in)) as in BASELINE configs 1, 2, 4

The reference takes any []float32 through Tensor.SetData (tensor/tensor.go:58-68); the same bytes are
fed to the oracle and to the HIP path, so the generator is part of the harness definition.
"""
from __future__ import annotations

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed: int, tag: int, n: int) -> np.ndarray:
    base = np.uint64(((seed & 0xFFFFFFFF) << 32) | (tag & 0xFFFFFFFF))
    with np.errstate(over="ignore"):
        z = base + np.arange(1, n + 1, dtype=np.uint64) * _GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        z = z ^ (z >> np.uint64(31))
    return z


def uniform01(seed: int, tag: int, n: int) -> np.ndarray:
    z = splitmix64(seed, tag, n)
    return ((z >> np.uint64(40)).astype(np.float64) * 2.0**-24).astype(np.float32)


def uniform(seed: int, tag: int, shape, lo: float, hi: float) -> np.ndarray:
    n = int(np.prod(shape))
    z = splitmix64(seed, tag, n)
    u = (z >> np.uint64(40)).astype(np.float64) * 2.0**-24
    return (lo + (hi - lo) * u).astype(np.float32).reshape(shape)


def normal(seed: int, tag: int, shape, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    n = int(np.prod(shape))
    z = splitmix64(seed, tag, 2 * n)
    u1 = ((z[0::2] >> np.uint64(11)).astype(np.float64) + 1.0) * 2.0**-53
    u2 = (z[1::2] >> np.uint64(11)).astype(np.float64) * 2.0**-53
    g = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)
    return (mean + std * g).astype(np.float32).reshape(shape)


def labels(seed: int, tag: int, n: int, classes: int) -> np.ndarray:
    z = splitmix64(seed, tag, n)
    return ((z >> np.uint64(32)) % np.uint64(classes)).astype(np.int32)


def kaiming_uniform(seed: int, tag: int, shape, fan_in: int) -> np.ndarray:
    b = float(np.sqrt(6.0 / fan_in))
    return uniform(seed, tag, shape, -b, b)


# ── Config definitions ───────────────────────────────────────────────────────
# Tags are fixed per tensor so any sub-shape of a config draws a prefix-stable stream.

def mlp_ce_inputs(B: int, D: int, H: int, C: int, seed: int = 0, x_lo: float = 0.0, x_hi: float = 1.0):
    """Configs 1 and 4: x U[x_lo,x_hi), int32 labels, Kaiming-uniform W, zero biases."""
    return {
        "x": uniform(seed, 1, (B, D), x_lo, x_hi),
        "labels": labels(seed, 2, B, C),
        "W1": kaiming_uniform(seed, 3, (H, D), D),
        "b1": np.zeros(H, np.float32),
        "W2": kaiming_uniform(seed, 4, (C, H), H),
        "b2": np.zeros(C, np.float32),
    }


def convnet_inputs(N: int = 32, Hin: int = 28, C1: int = 8, C2: int = 16, NC: int = 10, seed: int = 0):
    """Config 2: x U[0,1) [N,1,Hin,Hin]; conv biases and fc bias zero (recorded choice)."""
    F = C2 * (Hin // 4) ** 2
    return {
        "x": uniform(seed, 11, (N, 1, Hin, Hin), 0.0, 1.0),
        "labels": labels(seed, 12, N, NC),
        "cw1": kaiming_uniform(seed, 13, (C1, 1, 3, 3), 9),
        "cb1": np.zeros(C1, np.float32),
        "cw2": kaiming_uniform(seed, 14, (C2, C1, 3, 3), C1 * 9),
        "cb2": np.zeros(C2, np.float32),
        "fw": kaiming_uniform(seed, 15, (NC, F), F),
        "fb": np.zeros(NC, np.float32),
    }


def mlp3_inputs(B: int = 4096, D0: int = 1024, D1: int = 4096, D2: int = 4096, D3: int = 1024, seed: int = 0):
    """Config 3: x, targets N(0,1); W N(0, 1/fan_in); zero biases (recorded choice). f32 masters."""
    return {
        "x": normal(seed, 21, (B, D0)),
        "t": normal(seed, 22, (B, D3)),
        "W1": normal(seed, 23, (D1, D0), 0.0, float(np.sqrt(1.0 / D0))),
        "b1": np.zeros(D1, np.float32),
        "W2": normal(seed, 24, (D2, D1), 0.0, float(np.sqrt(1.0 / D1))),
        "b2": np.zeros(D2, np.float32),
        "W3": normal(seed, 25, (D3, D2), 0.0, float(np.sqrt(1.0 / D2))),
        "b3": np.zeros(D3, np.float32),
    }


def chain_inputs(R: int = 8192, Cc: int = 4096, seed: int = 0):
    """Config 5: X N(0,1) [R,Cc]; gain g N(1, 0.02) [Cc]."""
    return {"X": normal(seed, 31, (R, Cc)), "g": normal(seed, 32, (Cc,), 1.0, 0.02)}


def f16_quantize(a: np.ndarray) -> np.ndarray:
    """f32 -> f16 (round to nearest even) -> f32, as Tensor.SetData does for f16 leaves.
    numpy's float16 cast is IEEE RTNE, identical to uop/dtype.go:392 for finite inputs."""
    return a.astype(np.float16).astype(np.float32)
