"""ExecItem lists for the five BASELINE training steps, written with "tmpl:" keys.

This is the kernel partition a HIP renderer would hand the executor for one forward+backward step:
each item is one fused kernel of the reference's schedule (bufs[0] the output, inputs in PARAM order,
schedule/exec.go:6-32), with the hot contractions, reductions, pooling, convolution and chain kernels
named by template key instead of source. The partition is restated from the gradient rules
(tensor/gradient_ruleset.go) and the layers (tensor/nn/nn.go), not read from the reference's scheduler,
which needs a Go toolchain to run. Leaves carry uop indices 1..; intermediates 10..; labels travel as
int32 bits in float32 slots (backend/webgpu/executor.go:470-528).

Each builder returns (items, leaves, outputs): `leaves` maps names to leaf uop indices (the keys of the
inputs dict), `outputs` maps names to the uop indices of the final outputs.
"""
from __future__ import annotations

import numpy as np

from . import _lib as L
from .executor import Buffer, ExecItem

F32, F16, I32 = L.AH_F32, L.AH_F16, L.AH_I32


def f32_key(v: float) -> str:
    """A float parameter spelled exactly: the hex form of its f32 value (read back by strtof)."""
    return float(np.float32(v)).hex()


def _buf(uop, shape, dtype=F32, sym=False):
    """A buffer of `shape`; sym=True makes the leading dimension the symbolic one (size 0, shape[0] = 0)."""
    if sym:
        return Buffer(uop, 0, [0] + list(shape[1:]), dtype)
    return Buffer(uop, int(np.prod(shape)), list(shape), dtype)


def mlp_ce(B, D, H, C, symbolic=False, sgd_lr=None):
    """Configs 1 and 4: Linear(D->H) ReLU Linear(H->C), softmax cross-entropy (Sum(onehot*logp)*(-1/B),
    examples/mlp.go and examples/dynmlp.go:136), backward; with sgd_lr the updated parameters are the
    outputs (Parameter.SGDStep, nn.go:69-76) in place of the gradients. symbolic=True binds B to "N"
    (NewSymbolicBatchInput): B then only sets the -1/B constant, which the reference bakes into the graph."""
    Bk = "sym" if symbolic else str(B)
    sv = ["N"] if symbolic else []
    lv = dict(x=1, labels=2, W1=3, b1=4, W2=5, b2=6)
    bx = lambda u, cols, dt=F32: _buf(u, (B, cols), dt, symbolic)   # noqa: E731  batch-major buffers
    x, lab = bx(1, D), _buf(2, (B,), I32, symbolic)
    W1, b1, W2, b2 = _buf(3, (H, D)), _buf(4, (H,)), _buf(5, (C, H)), _buf(6, (C,))
    H1, Z, dZ, rl = bx(10, H), bx(11, C), bx(12, C), _buf(13, (B,), F32, symbolic)
    loss, db2, dZ1, db1, dW2, dW1 = _buf(14, (1,)), _buf(15, (C,)), bx(16, H), _buf(17, (H,)), _buf(18, (C, H)), _buf(19, (H, D))
    g = "tmpl:gemm;dtype=f32"
    items = [
        ExecItem(f"{g};epi=bias_relu;ta=0;tb=0;M={Bk};N={H};K={D}", [H1, x, W1, b1], sv),
        ExecItem(f"{g};epi=bias;ta=0;tb=0;M={Bk};N={C};K={H}", [Z, H1, W2, b2], sv),
        ExecItem(f"tmpl:softmax_ce;B={Bk};C={C}", [dZ, Z, lab, rl], sv),
        ExecItem(f"tmpl:reduce;op=sum;axis=1;M=1;N={Bk};scale={f32_key(-1.0 / B)}", [loss, rl], sv),
        ExecItem(f"tmpl:reduce;op=sum;axis=0;M={Bk};N={C}", [db2, dZ], sv),
        ExecItem(f"{g};epi=mask;ta=0;tb=1;M={Bk};N={H};K={C}", [dZ1, dZ, W2, H1], sv),
        ExecItem(f"tmpl:reduce;op=sum;axis=0;M={Bk};N={H}", [db1, dZ1], sv),
        ExecItem(f"{g};epi=store;ta=1;tb=1;M={C};N={H};K={Bk}", [dW2, dZ, H1], sv),
        ExecItem(f"{g};epi=store;ta=1;tb=1;M={H};N={D};K={Bk}", [dW1, dZ1, x], sv),
    ]
    outs = dict(loss=14, db2=15, db1=17, dW2=18, dW1=19)
    if sgd_lr is not None:
        lr = f32_key(sgd_lr)
        items = items[:-2]   # the weight gradients are formed inside the fused SGD contractions instead
        items += [ExecItem(f"{g};epi=sgd;ta=1;tb=1;M={H};N={D};K={Bk};lr={lr}", [_buf(20, (H, D)), dZ1, x, W1], sv),
                  ExecItem(f"tmpl:sgd;n={H};lr={lr}", [_buf(21, (H,)), b1, db1], sv),
                  ExecItem(f"{g};epi=sgd;ta=1;tb=1;M={C};N={H};K={Bk};lr={lr}", [_buf(22, (C, H)), dZ, H1, W2], sv),
                  ExecItem(f"tmpl:sgd;n={C};lr={lr}", [_buf(23, (C,)), b2, db2], sv)]
        # the bias gradients are read by the updates; the updated parameters and the loss are the outputs
        outs = dict(loss=14, W1=20, b1=21, W2=22, b2=23)
    return items, lv, outs


def convnet(N, Hin=28, C1=8, C2=16, NC=10):
    """Config 2: Conv2d(1->C1, 3x3, pad 1) ReLU MaxPool2D(2,2), Conv2d(C1->C2) ReLU MaxPool2D(2,2),
    Linear(C2*(Hin/4)^2 -> NC), softmax cross-entropy, backward (nn.go:217-386)."""
    H2, H4 = Hin // 2, Hin // 4
    F = C2 * H4 * H4
    lv = dict(x=1, labels=2, cw1=3, cb1=4, cw2=5, cb2=6, fw=7, fb=8)
    x, lab = _buf(1, (N, 1, Hin, Hin)), _buf(2, (N,), I32)
    cw1, cb1, cw2, cb2 = _buf(3, (C1, 1, 3, 3)), _buf(4, (C1,)), _buf(5, (C2, C1, 3, 3)), _buf(6, (C2,))
    fw, fb = _buf(7, (NC, F)), _buf(8, (NC,))
    P1, A1 = _buf(10, (N, C1, H2, H2)), _buf(11, (N, C1, Hin, Hin))
    P2, A2 = _buf(12, (N, C2, H4, H4)), _buf(13, (N, C2, H2, H2))
    lg, dlg, rl, loss = _buf(14, (N, NC)), _buf(15, (N, NC)), _buf(16, (N,)), _buf(17, (1,))
    dfb, dfw, dP2, dZ2 = _buf(18, (NC,)), _buf(19, (NC, F)), _buf(20, (N, F)), _buf(21, (N, C2, H2, H2))
    dcw2, dcb2, dP1, dZ1 = _buf(22, (C2, C1, 3, 3)), _buf(23, (C2,)), _buf(24, (N, C1, H2, H2)), _buf(25, (N, C1, Hin, Hin))
    dcw1, dcb1 = _buf(26, (C1, 1, 3, 3)), _buf(27, (C1,))
    items = [
        ExecItem(f"tmpl:conv2d_relu_pool;N={N};Ci=1;Co={C1};H={Hin}", [P1, x, cw1, cb1, A1]),
        ExecItem(f"tmpl:conv2d_relu_pool;N={N};Ci={C1};Co={C2};H={H2}", [P2, P1, cw2, cb2, A2]),
        ExecItem(f"tmpl:gemm;dtype=f32;epi=bias;ta=0;tb=0;M={N};N={NC};K={F}", [lg, P2, fw, fb]),
        ExecItem(f"tmpl:softmax_ce;B={N};C={NC}", [dlg, lg, lab, rl]),
        ExecItem(f"tmpl:reduce;op=sum;axis=1;M=1;N={N};scale={f32_key(-1.0 / N)}", [loss, rl]),
        ExecItem(f"tmpl:reduce;op=sum;axis=0;M={N};N={NC}", [dfb, dlg]),
        ExecItem(f"tmpl:gemm;dtype=f32;epi=store;ta=1;tb=1;M={NC};N={F};K={N}", [dfw, dlg, P2]),
        ExecItem(f"tmpl:gemm;dtype=f32;epi=store;ta=0;tb=1;M={N};N={F};K={NC}", [dP2, dlg, fw]),
        ExecItem(f"tmpl:pool_relu_bwd;N={N};C={C2};H={H2}", [dZ2, dP2, A2, P2]),
        ExecItem(f"tmpl:conv2d_bwd_w;N={N};Ci={C1};Co={C2};H={H2}", [dcw2, P1, dZ2]),
        ExecItem(f"tmpl:conv2d_bwd_b;N={N};Co={C2};H={H2}", [dcb2, dZ2]),
        ExecItem(f"tmpl:conv2d_bwd_x;N={N};Ci={C1};Co={C2};H={H2}", [dP1, dZ2, cw2]),
        ExecItem(f"tmpl:pool_relu_bwd;N={N};C={C1};H={Hin}", [dZ1, dP1, A1, P1]),
        ExecItem(f"tmpl:conv2d_bwd_w;N={N};Ci=1;Co={C1};H={Hin}", [dcw1, x, dZ1]),
        ExecItem(f"tmpl:conv2d_bwd_b;N={N};Co={C1};H={Hin}", [dcb1, dZ1]),
    ]
    outs = dict(loss=17, dfb=18, dfw=19, dcw2=22, dcb2=23, dcw1=26, dcb1=27)
    return items, lv, outs


def mlp3_f16(B, D0, D1, D2, D3):
    """Config 3: f16 Linear(D0->D1) ReLU Linear(D1->D2) ReLU Linear(D2->D3), MSE-mean loss, backward.
    f16 storage and MFMA with f32 accumulation; the MSE adjoint is carried as f16(P - T) and the factor
    2/(B*D3) applied in f32 where the gradients are formed (the weight gradients are f32 outputs)."""
    sc = 1.0 / (B * D3)
    bs = f32_key(2.0 * np.float32(sc))
    lv = dict(x=1, t=2, W1=3, b1=4, W2=5, b2=6, W3=7, b3=8)
    x, t = _buf(1, (B, D0), F16), _buf(2, (B, D3), F16)
    W1, b1, W2, b2 = _buf(3, (D1, D0), F16), _buf(4, (D1,), F16), _buf(5, (D2, D1), F16), _buf(6, (D2,), F16)
    W3, b3 = _buf(7, (D3, D2), F16), _buf(8, (D3,), F16)
    H1, H2, Dd = _buf(10, (B, D1), F16), _buf(11, (B, D2), F16), _buf(12, (B, D3), F16)
    parts = ((B + 31) // 32) * ((D3 + 31) // 32)
    lp, loss = _buf(13, (parts,)), _buf(14, (1,))
    db3, dZ2, db2, dW3 = _buf(15, (D3,)), _buf(16, (B, D2), F16), _buf(17, (D2,)), _buf(18, (D3, D2))
    dZ1, db1, dW2, dW1 = _buf(19, (B, D1), F16), _buf(20, (D1,)), _buf(21, (D2, D1)), _buf(22, (D1, D0))
    g = "tmpl:gemm;dtype=f16"
    items = [
        ExecItem(f"{g};epi=bias_relu;ta=0;tb=0;M={B};N={D1};K={D0}", [H1, x, W1, b1]),
        ExecItem(f"{g};epi=bias_relu;ta=0;tb=0;M={B};N={D2};K={D1}", [H2, H1, W2, b2]),
        ExecItem(f"{g};epi=mse;ta=0;tb=0;M={B};N={D3};K={D2}", [Dd, H2, W3, b3, t, lp]),
        ExecItem(f"tmpl:mse_loss;parts={parts};scale={f32_key(sc)}", [loss, lp]),
        ExecItem(f"tmpl:reduce;dtype=f16;op=sum;axis=0;M={B};N={D3};scale={bs}", [db3, Dd]),
        ExecItem(f"{g};epi=mask;ta=0;tb=1;M={B};N={D2};K={D3}", [dZ2, Dd, W3, H2]),
        ExecItem(f"{g};epi=grad;ta=1;tb=1;M={D3};N={D2};K={B};scale={bs}", [dW3, Dd, H2]),
        ExecItem(f"tmpl:reduce;dtype=f16;op=sum;axis=0;M={B};N={D2};scale={bs}", [db2, dZ2]),
        ExecItem(f"{g};epi=mask;ta=0;tb=1;M={B};N={D1};K={D2}", [dZ1, dZ2, W2, H1]),
        ExecItem(f"{g};epi=grad;ta=1;tb=1;M={D2};N={D1};K={B};scale={bs}", [dW2, dZ2, H1]),
        ExecItem(f"tmpl:reduce;dtype=f16;op=sum;axis=0;M={B};N={D1};scale={bs}", [db1, dZ1]),
        ExecItem(f"{g};epi=grad;ta=1;tb=1;M={D1};N={D0};K={B};scale={bs}", [dW1, dZ1, x]),
    ]
    outs = dict(loss=14, db3=15, dW3=18, db2=17, dW2=21, db1=20, dW1=22)
    return items, lv, outs


def chain(R, Cc):
    """Config 5: Y = Shrink(Pad(Permute(X, (1, 0)))), row softmax, RMS normalisation times g, Sum, and the
    backward into X and g, as one chain item (its three kernels share a workspace)."""
    lv = dict(X=1, g=2)
    items = [ExecItem(f"tmpl:chain;R={R};Cc={Cc}", [_buf(10, (R, Cc)), _buf(1, (R, Cc)), _buf(2, (Cc,)),
                                                     _buf(11, (Cc,)), _buf(12, (1,))])]
    return items, lv, dict(dX=10, dg=11, loss=12)


def inputs(leaves: dict, values: dict) -> dict:
    """The inputs dict of a Run: leaf uop index -> float32 data (int32 labels as raw bits)."""
    out = {}
    for name, uop in leaves.items():
        v = np.asarray(values[name])
        out[uop] = v.view(np.float32).ravel() if v.dtype == np.int32 else np.ascontiguousarray(v, np.float32).ravel()
    return out
