"""Blocked numpy restatement of ora_mlp3_f16_step (oracle/anneal_oracle.c) for full config-3 sizes.

TEST INFRASTRUCTURE ONLY. The C oracle's serial loops need about a minute for one full config-3 step
(584 GFLOP); this restatement keeps the oracle's f16 rounding points (f16 leaves, f16(f16(acc)+b)
narrowing, f16 loss accumulator, f16 Sub before the MSE gradient) and differs only in f32 summation
order (BLAS sgemm instead of the serial k-loop). test_oracle_np_matches_c_oracle pins it to the C
oracle at small sizes; full-size GPU parity uses it at the config-3 tolerance (2e-2).
"""
import numpy as np


def q16(a):
    return np.asarray(a, np.float32).astype(np.float16).astype(np.float32)


def mlp3_step_np(p: dict, lr: float):
    """Same contract as oracle_lib.mlp3_step: x, t f16-representable; returns (loss, grads, new params);
    grads also holds "loss_sum", the f32 sum of squared differences before the f16 narrowing."""
    x, t = np.asarray(p["x"], np.float32), np.asarray(p["t"], np.float32)
    prm = {k: np.asarray(p[k], np.float32).copy() for k in ("W1", "b1", "W2", "b2", "W3", "b3")}
    w1, w2, w3 = q16(prm["W1"]), q16(prm["W2"]), q16(prm["W3"])
    c1, c2, c3 = q16(prm["b1"]), q16(prm["b2"]), q16(prm["b3"])
    B, D3 = x.shape[0], w3.shape[0]
    Z1 = q16(q16(x @ w1.T) + c1)
    H1 = np.maximum(Z1, 0)
    Z2 = q16(q16(H1 @ w2.T) + c2)
    H2 = np.maximum(Z2, 0)
    P = q16(q16(H2 @ w3.T) + c3)
    scale = np.float32(1.0 / (float(B) * float(D3)))
    d32 = P - t
    acc = np.float32(np.sum(d32.astype(np.float64) ** 2))
    loss = float(q16(acc) * scale)
    d = q16(d32)
    gP = scale * d + scale * d
    g = {"loss_sum": float(acc)}   # the f32 sum of squares before the f16 narrowing
    g["db3"] = gP.sum(0, dtype=np.float64).astype(np.float32)
    g["dW3"] = gP.T @ H2
    dH2 = np.where(Z2 == H2, gP @ w3, np.float32(0))
    g["db2"] = dH2.sum(0, dtype=np.float64).astype(np.float32)
    g["dW2"] = dH2.T @ H1
    dH1 = np.where(Z1 == H1, dH2 @ w2, np.float32(0))
    g["db1"] = dH1.sum(0, dtype=np.float64).astype(np.float32)
    g["dW1"] = dH1.T @ x
    new = {k: (v - np.float32(lr) * g["d" + k]).astype(np.float32) for k, v in prm.items()}
    return loss, g, new


def chain_dX_f64(X, g):
    """Closed-form f64 gradient of Sum(S * recip(sqrt(mean(S^2)+1e-6)) * g) w.r.t. X (S = softmax over
    X's columns). In exact arithmetic the row-max path contributes nothing (softmax is shift
    invariant); in f32 its tie share is a rounding residue, so column-max elements are judged here."""
    R = X.shape[0]
    Y = X.astype(np.float64).T
    e = np.exp(Y - Y.max(1, keepdims=True))
    S = e / e.sum(1, keepdims=True)
    r = 1.0 / np.sqrt((S * S).mean(1, keepdims=True) + 1e-6)
    G = np.asarray(g, np.float64)[:, None]
    dS = G * r - G * S.sum(1, keepdims=True) * r ** 3 * S / R
    return (S * (dS - (S * dS).sum(1, keepdims=True))).T


def mlp_ce_step_f64(p: dict, lr: float):
    """Float64 closed form of ora_mlp_ce_step (configs 1 and 4) for batches the C oracle's serial loops
    take tens of seconds on: Linear ReLU Linear, loss = Sum(onehot * logsoftmax) * (-1/B), ReLU'(0) = 1
    (Where(z == relu(z)), tensor/gradient_ruleset.go:153-161), dz = (softmax - onehot) / B (the row-max
    path's tie share is zero in exact arithmetic). test_oracle_np_matches_c_oracle pins it to the C
    oracle at small batches. Returns (loss, grads, new params) like oracle_lib.mlp_ce_step."""
    x = np.asarray(p["x"], np.float64)
    lab = np.asarray(p["labels"], np.int64)
    W1, b1, W2, b2 = (np.asarray(p[k], np.float64) for k in ("W1", "b1", "W2", "b2"))
    B = x.shape[0]
    Z1 = x @ W1.T + b1
    H1 = np.maximum(Z1, 0.0)
    Z = H1 @ W2.T + b2
    Zs = Z - Z.max(1, keepdims=True)
    lse = np.log(np.exp(Zs).sum(1, keepdims=True))
    logp = Zs - lse
    onehot = np.zeros_like(Z)
    onehot[np.arange(B), lab] = 1.0
    loss = float((onehot * logp).sum() * (-1.0 / B))
    dZ = (np.exp(logp) - onehot) / B
    dZ1 = np.where(Z1 >= 0, dZ @ W2, 0.0)
    g = {"dW2": dZ.T @ H1, "db2": dZ.sum(0), "dW1": dZ1.T @ x, "db1": dZ1.sum(0)}
    new = {k: np.asarray(p[k], np.float64) - lr * g["d" + k] for k in ("W1", "b1", "W2", "b2")}
    return loss, g, new


def mlp_ce_grads_given_hidden_f64(p: dict, H1):
    """The float64 backward of mlp_ce_step_f64 from a given hidden layer H1 (an f32 device readback of
    the ReLU outputs, -0.0 marking a unit whose pre-activation was negative): the loss and the gradients
    with the device's own ReLU mask, so rows whose mask f32 rounding decides can be checked too. With
    H1 = relu(Z1) and a mask Z1 >= 0 it reduces to mlp_ce_step_f64 (tested on the CPU)."""
    x = np.asarray(p["x"], np.float64)
    lab = np.asarray(p["labels"], np.int64)
    W2, b2 = (np.asarray(p[k], np.float64) for k in ("W2", "b2"))
    h32 = np.ascontiguousarray(H1, np.float32)
    live = h32.view(np.uint32) != np.uint32(0x80000000)
    Hd = h32.astype(np.float64)
    B = x.shape[0]
    Z = Hd @ W2.T + b2
    Zs = Z - Z.max(1, keepdims=True)
    logp = Zs - np.log(np.exp(Zs).sum(1, keepdims=True))
    onehot = np.zeros_like(Z)
    onehot[np.arange(B), lab] = 1.0
    loss = float((onehot * logp).sum() * (-1.0 / B))
    dZ = (np.exp(logp) - onehot) / B
    dZ1 = np.where(live, dZ @ W2, 0.0)
    return loss, {"dW2": dZ.T @ Hd, "db2": dZ.sum(0), "dW1": dZ1.T @ x, "db1": dZ1.sum(0)}


def relu_ambiguous_units(p: dict, atol: float = 1e-5):
    """Hidden units whose ReLU mask an f32 evaluation may set differently from another one: some batch
    row has |z| below atol (about ten times the f32 rounding of these 512-term pre-activations). Rounding decides Where(z == relu(z)) there, so a gradient row of such
    a unit is an O(1) difference between two correct f32 implementations; large-batch checks against the
    float64 closed form leave these rows (a few of thousands) out."""
    x = np.asarray(p["x"], np.float64)
    Z1 = x @ np.asarray(p["W1"], np.float64).T + np.asarray(p["b1"], np.float64)
    return np.nonzero((np.abs(Z1) < atol).any(0))[0]
