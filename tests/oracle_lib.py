"""ctypes binding of the CPU oracle (oracle/liboracle.so). Test infrastructure only."""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_DIR = os.path.join(ROOT, "oracle")
ORACLE_SO = os.path.join(ORACLE_DIR, "liboracle.so")

_lib = None
F = C.POINTER(C.c_float)
D = C.POINTER(C.c_double)
I = C.POINTER(C.c_int32)


def load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(ORACLE_SO):
        subprocess.run(["make", "-C", ORACLE_DIR], check=True, capture_output=True)
    lib = C.CDLL(ORACLE_SO)
    lib.ora_f32_to_f16.restype = C.c_uint16
    lib.ora_f32_to_f16.argtypes = [C.c_float]
    lib.ora_f16_to_f32.restype = C.c_float
    lib.ora_f16_to_f32.argtypes = [C.c_uint16]
    lib.ora_num_threads.restype = C.c_int
    for name in ("ora_mlp_ce_loss_f64", "ora_convnet_loss_f64", "ora_mlp3_loss_f64", "ora_chain_loss_f64"):
        getattr(lib, name).restype = C.c_double
    _lib = lib
    return lib


def fp(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(F)


def dp(a: np.ndarray):
    assert a.dtype == np.float64 and a.flags.c_contiguous
    return a.ctypes.data_as(D)


def ip(a: np.ndarray):
    assert a.dtype == np.int32 and a.flags.c_contiguous
    return a.ctypes.data_as(I)


def f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


# ── wrappers returning numpy results ────────────────────────────────────────

def matmul(A, B):
    A, B = f32(A), f32(B)
    M, K = A.shape
    N = B.shape[1]
    out = np.zeros((M, N), np.float32)
    load().ora_matmul(fp(A), fp(B), M, K, N, fp(out))
    return out


def linear_mse(x, W, t):
    x, W, t = f32(x), f32(W), f32(t)
    M, K = x.shape
    N = W.shape[1]
    loss = np.zeros(1, np.float32)
    gx, gW = np.zeros_like(x), np.zeros_like(W)
    load().ora_linear_mse(fp(x), fp(W), fp(t), M, K, N, fp(loss), fp(gx), fp(gW))
    return float(loss[0]), gx, gW


def exp2_sum_grad(x):
    x = f32(x)
    loss = np.zeros(1, np.float32)
    g = np.zeros_like(x)
    load().ora_exp2_sum_grad(fp(x), x.size, fp(loss), fp(g))
    return float(loss[0]), g


def maxpool2d(x, kH, kW, sH, sW, adj=None, grad=True):
    x = f32(x)
    N, Cn, H, W = x.shape
    oH, oW = (H - kH) // sH + 1, (W - kW) // sW + 1
    out = np.zeros((N, Cn, oH, oW), np.float32)
    gx = np.zeros_like(x) if grad else None
    adj_p = fp(f32(adj)) if adj is not None else None
    load().ora_maxpool2d(fp(x), N, Cn, H, W, kH, kW, sH, sW, fp(out), adj_p, fp(gx) if grad else None)
    return out, gx


def softmax_ce(z, labels):
    z = f32(z)
    labels = np.ascontiguousarray(labels, np.int32)
    B, Cn = z.shape
    loss = np.zeros(1, np.float32)
    dz = np.zeros_like(z)
    load().ora_softmax_ce(fp(z), ip(labels), B, Cn, fp(loss), fp(dz))
    return float(loss[0]), dz


def mlp_ce_step(p: dict, lr: float):
    """Returns (loss, grads dict, updated params dict)."""
    x, lab = f32(p["x"]), np.ascontiguousarray(p["labels"], np.int32)
    W1, b1, W2, b2 = (f32(p[k]).copy() for k in ("W1", "b1", "W2", "b2"))
    B, D = x.shape
    H, Cn = W1.shape[0], W2.shape[0]
    loss = np.zeros(1, np.float32)
    g = {k: np.zeros_like(v) for k, v in (("dW1", W1), ("db1", b1), ("dW2", W2), ("db2", b2))}
    load().ora_mlp_ce_step(fp(x), ip(lab), B, D, H, Cn, fp(W1), fp(b1), fp(W2), fp(b2), C.c_float(lr), fp(loss),
                           fp(g["dW1"]), fp(g["db1"]), fp(g["dW2"]), fp(g["db2"]))
    return float(loss[0]), g, {"W1": W1, "b1": b1, "W2": W2, "b2": b2}


def convnet_step(p: dict, lr: float):
    x, lab = f32(p["x"]), np.ascontiguousarray(p["labels"], np.int32)
    prm = {k: f32(p[k]).copy() for k in ("cw1", "cb1", "cw2", "cb2", "fw", "fb")}
    N, _, Hin, _ = x.shape
    C1, C2, NC = prm["cw1"].shape[0], prm["cw2"].shape[0], prm["fw"].shape[0]
    loss = np.zeros(1, np.float32)
    g = {"d" + k: np.zeros_like(v) for k, v in prm.items()}
    load().ora_convnet_step(fp(x), ip(lab), N, Hin, C1, C2, NC, fp(prm["cw1"]), fp(prm["cb1"]), fp(prm["cw2"]),
                            fp(prm["cb2"]), fp(prm["fw"]), fp(prm["fb"]), C.c_float(lr), fp(loss), fp(g["dcw1"]),
                            fp(g["dcb1"]), fp(g["dcw2"]), fp(g["dcb2"]), fp(g["dfw"]), fp(g["dfb"]))
    return float(loss[0]), g, prm


def mlp3_step(p: dict, lr: float):
    """x and t must already be f16-representable (the reference quantizes f16 leaves on upload)."""
    x, t = f32(p["x"]), f32(p["t"])
    prm = {k: f32(p[k]).copy() for k in ("W1", "b1", "W2", "b2", "W3", "b3")}
    B, D0 = x.shape
    D1, D2, D3 = prm["W1"].shape[0], prm["W2"].shape[0], prm["W3"].shape[0]
    loss = np.zeros(1, np.float32)
    g = {"d" + k: np.zeros_like(v) for k, v in prm.items()}
    load().ora_mlp3_f16_step(fp(x), fp(t), B, D0, D1, D2, D3, fp(prm["W1"]), fp(prm["b1"]), fp(prm["W2"]),
                             fp(prm["b2"]), fp(prm["W3"]), fp(prm["b3"]), C.c_float(lr), fp(loss), fp(g["dW1"]),
                             fp(g["db1"]), fp(g["dW2"]), fp(g["db2"]), fp(g["dW3"]), fp(g["db3"]))
    return float(loss[0]), g, prm


def chain_step(X, g):
    X, g = f32(X), f32(g)
    R, Cc = X.shape
    loss = np.zeros(1, np.float32)
    dX, dg = np.zeros_like(X), np.zeros_like(g)
    load().ora_chain_step(fp(X), fp(g), R, Cc, fp(loss), fp(dX), fp(dg))
    return float(loss[0]), dX, dg


def f64(a):
    return np.ascontiguousarray(a, np.float64)


def mlp_ce_loss_f64(x, lab, W1, b1, W2, b2):
    B, D = x.shape
    return load().ora_mlp_ce_loss_f64(dp(f64(x)), ip(np.ascontiguousarray(lab, np.int32)), B, D, W1.shape[0],
                                      W2.shape[0], dp(f64(W1)), dp(f64(b1)), dp(f64(W2)), dp(f64(b2)))


def convnet_loss_f64(x, lab, cw1, cb1, cw2, cb2, fw, fb):
    N, _, Hin, _ = x.shape
    return load().ora_convnet_loss_f64(dp(f64(x)), ip(np.ascontiguousarray(lab, np.int32)), N, Hin, cw1.shape[0],
                                       cw2.shape[0], fw.shape[0], dp(f64(cw1)), dp(f64(cb1)), dp(f64(cw2)),
                                       dp(f64(cb2)), dp(f64(fw)), dp(f64(fb)))


def mlp3_loss_f64(x, t, W1, b1, W2, b2, W3, b3):
    B, D0 = x.shape
    return load().ora_mlp3_loss_f64(dp(f64(x)), dp(f64(t)), B, D0, W1.shape[0], W2.shape[0], W3.shape[0],
                                    dp(f64(W1)), dp(f64(b1)), dp(f64(W2)), dp(f64(b2)), dp(f64(W3)), dp(f64(b3)))


def chain_loss_f64(X, g):
    R, Cc = X.shape
    return load().ora_chain_loss_f64(dp(f64(X)), dp(f64(g)), R, Cc)


def relerr(a, b) -> float:
    """Norm-wise relative error max|a-b| / max|b| (the tolerance metric used by the parity tests)."""
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    den = np.max(np.abs(b))
    return float(np.max(np.abs(a - b)) / (den if den > 0 else 1.0))
