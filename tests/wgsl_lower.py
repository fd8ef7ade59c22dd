"""The configs-1/4 and config-3 training steps as the WGSL kernels anneal's codegen renders, for the
template-selection tests (tests/test_wgsl_select.py, host) and the rendered-step parity tests
(tests/test_gpu_wgsl.py, GPU).

TEST INFRASTRUCTURE ONLY. Without a Go toolchain the reference's scheduler cannot be run, so the kernel
partition is restated from its rules and the text from its lowering, not captured:
  - partition (schedule/kernels.go, SPEC.md sections 7.5-7.6): every REDUCE materialises its output; an
    elementwise consumer that is a reduce's sole consumer is fused after it (Pass 5, epilogue fusion: the
    Linear bias add); other elementwise chains are inlined into the kernels that read them (ReLU's
    Maximum(z, 0) into the contractions that read the activation, the ReLU backward's
    Where(z == relu(z), adj, 0) into the reductions over the batch, tensor/gradient_ruleset.go:153-161);
    the softmax-CE adjoint dZ, read by three reductions, is materialised by its own elementwise kernel;
  - text (codegen/lower.go:98-719, codegen/wgsl.go:41-386): GIDVar lets per output range (dims assigned
    from the innermost range, `i32(flat_gid_C % R)` with an axis guard, symbolic ranges all on x as
    `i32(flat_gid_x / S)` with a params_n bounds check), one `let tN: T = ...;` per load and ALU node,
    one accumulator per reduce (`var acc0: f32 = <identity>;`, `acc0 = acc0 + tN;` or
    `acc0 = max(acc0, tN);`), loops `for (var rN: i32 = 0; rN < K; rN++)` (`i32(params_n.n0)` when
    symbolic), f32 constants in FormatFloat(v, 'f', -1, 32) form, and one store
    `data0[(u32(r0) * S) + u32(r1)] = v;`.
The softmax cross-entropy and its backward follow the graph the oracle restates (ora_softmax_ce,
oracle/anneal_oracle.c): m = Max(z), zs = z - m, e = Exp2(zs * 1/ln2), s = Sum(e), logp = zs -
Log2(s) * ln2, loss = Sum(logp * onehot) * (-1/B), and the rule-by-rule backward with the row max's
tie split.
"""
from __future__ import annotations

import struct

import numpy as np

from wgsl_kernels import F16, F32, I32, header, main_open

LOG2E = "1.442695"   # FormatFloat(1/ln2, 'f', -1, 32)
LN2 = "0.6931472"    # FormatFloat(ln2, 'f', -1, 32)
R0 = "r0"


def f32_lit(v: float) -> str:
    """A constant as constLiteral writes it: the shortest decimal that reads back as the same f32."""
    f = struct.unpack("f", struct.pack("f", v))[0]
    for digits in range(1, 12):
        s = f"{f:.{digits}g}"
        if struct.unpack("f", struct.pack("f", float(s)))[0] == f:
            break
    if "e" in s:
        s = f"{float(s):.{12}f}".rstrip("0")
    if "." not in s:
        s += ".0"
    return s


class Kernel:
    """Builds one kernel's text in the lowering's emit order."""

    def __init__(self, bufs, out_axes, sym=False, f16=False):
        """bufs: [(uop, shape, dtype)] in PARAM order (data0 the output); out_axes: the output ranges,
        outermost first, as sizes (the string "N" for the symbolic batch, None for a kept size-1 dim)."""
        self.bufs, self.sym, self.f16 = bufs, sym, f16
        self.lines = []
        self.depth = 1
        self.t = 5
        self.next_r = 0
        self.out = []                 # (range name or None, size)
        for size in out_axes:
            if size is None:
                self.out.append((None, 1))
            else:
                self.out.append((f"r{self.next_r}", size))
                self.next_r += 1
        self._gid()

    def emit(self, s):
        self.lines.append("  " * self.depth + s)

    def _gid(self):
        """GIDVar lets, guards and the symbolic bounds check (codegen/lower.go:194-466)."""
        dims = [[], [], []]
        has_sym = any(s == "N" for _, s in self.out)
        k = 0
        for name, size in reversed(self.out):
            dims[0 if has_sym else k % 3].append((name, size))
            k += 1
        self.ws = [1, 1, 1]
        self.wc = [1, 1, 1]
        self.dim1_used = False
        for d in range(3):
            stride = 1
            for name, size in dims[d]:
                if name is None:
                    continue
                base = "flat_gid_" + "xyz"[d]
                if size == "N":
                    e = f"i32({base})" if stride == 1 else f"i32({base} / {stride}u)"
                    self.emit(f"let {name}: i32 = {e};")
                else:
                    e = f"i32({base} % {size}u)" if stride == 1 else f"i32(({base} / {stride}u) % {size}u)"
                    self.emit(f"let {name}: i32 = {e};")
                    if size > 1:
                        self.emit(f"if ({name} >= {size}) {{ return; }}")
                    stride *= size
                if d > 0:
                    self.dim1_used = True
            if d == 0 and any(n is not None for n, _ in dims[0]):
                self.ws[0] = 64
            total = 1
            for n, s in dims[d]:
                if n is not None:
                    total *= 64 if s == "N" else s
            self.wc[d] = max(1, (total + self.ws[d] - 1) // self.ws[d])
        if has_sym:
            trailing = 1
            seen = False
            for _, s in self.out:
                if s == "N":
                    seen = True
                elif seen:
                    trailing *= s
            self.emit("if (gid_x >= params_n.n0 * %du) { return; }" % trailing if trailing > 1 else
                      "if (gid_x >= params_n.n0) { return; }")

    def let(self, expr, ty="f32"):
        name = f"t{self.t}"
        self.t += 1 + (self.t % 3 == 0)   # arena indices are not consecutive
        self.emit(f"let {name}: {ty} = {expr};")
        return name

    def load(self, buf, idx, ty="f32", widen=False):
        e = f"data{buf}[{idx}]"
        if widen:
            return self.let(f"f32({e})", "f32")
        return self.let(e, ty)

    def idx2(self, a, stride, b):
        """An index as the lowering chains it: (a * stride) then (+ b), each its own i32 let."""
        t = self.let(f"({a} * {stride})", "i32")
        return self.let(f"({t} + {b})", "i32")

    def acc(self, op="+"):
        self.emit("var acc0: f32 = %s;" % ("0.0" if op == "+" else "bitcast<f32>(0xff7fffffu)"))
        self.accop = op

    def loop(self, size):
        name = f"r{self.next_r}"
        self.next_r += 1
        bound = "i32(params_n.n0)" if size == "N" else str(size)
        self.emit(f"for (var {name}: i32 = 0; {name} < {bound}; {name}++) {{")
        self.depth += 1
        return name

    def update(self, v):
        self.emit(f"acc0 = acc0 + {v};" if self.accop == "+" else f"acc0 = max(acc0, {v});")

    def end(self):
        self.depth -= 1
        self.emit("}")

    def store(self, v):
        terms, stride = [], 1
        for name, size in reversed(self.out):
            if name is None:
                continue
            terms.append(f"u32({name})" if stride == 1 else f"(u32({name}) * {stride}u)")
            stride *= 1 if size == "N" else size
        idx = " + ".join(reversed(terms)) if terms else "0u"
        self.emit(f"data0[{idx}] = {v};")

    def source(self):
        types = {F32: "f32", F16: "f16", I32: "i32"}
        src = header([types[d] for _, _, d in self.bufs], self.ws, self.wc, sym_params=True if self.sym else None,
                     f16=self.f16)
        src += main_open(self.ws, self.wc, dim1_used=self.dim1_used)
        return "\n".join(src + self.lines + ["}"])


def mlp_ce_step(B: int, D: int, H: int, C: int, symbolic: bool = False):
    """Linear(D->H) ReLU Linear(H->C), softmax-CE mean loss and its backward, as rendered kernels.
    Returns [(name, wgsl, bufs, ws, wc, plan)] where plan is what ah_wgsl_plan should select ("tmpl:..." with
    the batch written as {B}, "wave" or "thread"), plus the leaf and output uop maps. With symbolic=True
    the batch is bound at run time (NewSymbolicBatchInput) and B only sets the -1/B constant."""
    N = "N" if symbolic else B
    Bk = "sym" if symbolic else str(B)
    a = f32_lit(-1.0 / B)
    leaves = dict(x=1, labels=2, W1=3, b1=4, W2=5, b2=6)
    uZ1, uZ, um, utie, us, uloss, ugls, ugm, udZ, udb2, udW2, udH1, udb1, udW1 = range(10, 24)

    def bshape(*rest):
        return [N if symbolic else B] + list(rest)

    ks = []

    def add(name, k, plan):
        bufs = []
        for uop, shape, dt in k.bufs:
            if symbolic and shape and shape[0] == "N":
                bufs.append((uop, 0, dt, [0] + list(shape[1:])))
            else:
                bufs.append((uop, int(np.prod(shape)), dt, list(shape)))
        ks.append((name, k.source(), bufs, tuple(k.ws), tuple(k.wc), plan))

    # 1. Z1 = x W1^T + b1 (the bias add fused after the reduce)
    k = Kernel([(uZ1, bshape(H), F32), (1, bshape(D), F32), (3, [H, D], F32), (4, [H], F32)], [N, H], symbolic)
    k.acc()
    r2 = k.loop(D)
    tx = k.load(1, k.idx2("r0", D, r2))
    tw = k.load(2, f"(r1 * {D}) + {r2}")
    k.update(k.let(f"({tx} * {tw})"))
    k.end()
    k.store(k.let(f"(acc0 + {k.load(3, 'r1')})"))
    add("fc1", k, f"tmpl:gemm;dtype=f32;epi=bias;ta=0;tb=0;M={Bk};N={H};K={D}")

    # 2. Z = relu(Z1) W2^T + b2: the ReLU inlined into the loop (W2 bound first)
    k = Kernel([(uZ, bshape(C), F32), (5, [C, H], F32), (uZ1, bshape(H), F32), (6, [C], F32)], [N, C], symbolic)
    k.acc()
    r2 = k.loop(H)
    tz = k.load(2, f"(r0 * {H}) + {r2}")
    tr = k.let(f"max({tz}, 0.0)")
    tw = k.load(1, k.idx2("r1", H, r2))
    k.update(k.let(f"({tr} * {tw})"))
    k.end()
    k.store(k.let(f"({k.load(3, 'r1')} + acc0)"))
    add("fc2", k, f"tmpl:gemm;dtype=f32;epi=bias;ta=0;tb=0;M={Bk};N={C};K={H};pa=relu;swap_ab=1")

    # 3. m = Max(z, [1], keepdim)
    k = Kernel([(um, bshape(1), F32), (uZ, bshape(C), F32)], [N, None], symbolic)
    k.acc("max")
    r1 = k.loop(C)
    k.update(k.load(1, f"(r0 * {C}) + {r1}"))
    k.end()
    k.store("acc0")
    add("rowmax", k, f"tmpl:reduce;op=max;axis=1;M={Bk};N={C}")

    def zs(k, zbuf, mbuf, r1):
        tz = k.load(zbuf, f"(r0 * {C}) + {r1}")
        tm = k.load(mbuf, "r0")
        return tz, tm, k.let(f"({tz} - {tm})")

    def onehot(k, lbuf, r1):
        tl = k.load(lbuf, "r0", "i32")
        return k.let(f"select(0.0, 1.0, {k.let(f'({tl} == {r1})', 'bool')})")

    def gzs(k, zbuf, mbuf, sbuf, gbuf, lbuf, r1):
        tz, tm, d = zs(k, zbuf, mbuf, r1)
        e = k.let(f"exp2({k.let(f'({d} * {LOG2E})')})")
        g1 = k.let(f"({k.load(gbuf, 'r0')} * {LN2})")
        rs = k.let(f"(1.0 / {k.let(f'({k.load(sbuf, R0)} * {LN2})')})")
        gs = k.let(f"({g1} * {rs})")
        gv = k.let(f"({k.let(f'({gs} * {e})')} * {LN2})")
        g2 = k.let(f"({gv} * {LOG2E})")
        gl = k.let(f"({a} * {onehot(k, lbuf, r1)})")
        return tz, tm, k.let(f"({gl} + {g2})")

    # 4. tie count: Sum(Cast(z == m)) (the max rule's tie split, tensor/gradient_ruleset.go:307-320)
    k = Kernel([(utie, bshape(1), F32), (um, bshape(1), F32), (uZ, bshape(C), F32)], [N, None], symbolic)
    k.acc()
    r1 = k.loop(C)
    tz = k.load(2, f"(r0 * {C}) + {r1}")
    eq = k.let(f"({tz} == {k.load(1, 'r0')})", "bool")
    k.update(k.let(f"select(0.0, 1.0, {eq})"))
    k.end()
    k.store("acc0")
    add("tie", k, "wave")

    # 5. s = Sum(Exp2((z - m) * 1/ln2))
    k = Kernel([(us, bshape(1), F32), (uZ, bshape(C), F32), (um, bshape(1), F32)], [N, None], symbolic)
    k.acc()
    r1 = k.loop(C)
    _, _, d = zs(k, 1, 2, r1)
    k.update(k.let(f"exp2({k.let(f'({d} * {LOG2E})')})"))
    k.end()
    k.store("acc0")
    add("sumexp", k, "wave")

    # 6. loss = Sum((zs - Log2(s) * ln2) * onehot) * (-1/B), over both axes
    k = Kernel([(uloss, [1], F32), (2, bshape(), I32), (uZ, bshape(C), F32), (um, bshape(1), F32),
                (us, bshape(1), F32)], [], symbolic)
    k.acc()
    k.loop(N)
    r1 = k.loop(C)
    _, _, d = zs(k, 2, 3, r1)
    ls = k.let(f"({k.let(f'log2({k.load(4, R0)})')} * {LN2})")
    lp = k.let(f"({d} - {ls})")
    k.update(k.let(f"({lp} * {onehot(k, 1, r1)})"))
    k.end()
    k.end()
    k.store(k.let(f"(acc0 * {a})"))
    add("loss", k, "wave")

    # 7. gls = Sum(-(a * onehot)) (Sub's src1 -> Neg, expanded and summed back)
    k = Kernel([(ugls, bshape(1), F32), (2, bshape(), I32)], [N, None], symbolic)
    k.acc()
    r1 = k.loop(C)
    k.update(k.let(f"(-{k.let(f'({a} * {onehot(k, 1, r1)})')})"))
    k.end()
    k.store("acc0")
    add("gls", k, "wave")

    # 8. gm = Sum(-gzs): the adjoint of the row max
    k = Kernel([(ugm, bshape(1), F32), (uZ, bshape(C), F32), (um, bshape(1), F32), (us, bshape(1), F32),
                (ugls, bshape(1), F32), (2, bshape(), I32)], [N, None], symbolic)
    k.acc()
    r1 = k.loop(C)
    _, _, g = gzs(k, 1, 2, 3, 4, 5, r1)
    k.update(k.let(f"(-{g})"))
    k.end()
    k.store("acc0")
    add("gmax", k, "wave")

    # 9. dZ = gzs + Where(z == m, gm / tie, 0): elementwise, materialised for its three readers
    k = Kernel([(udZ, bshape(C), F32), (uZ, bshape(C), F32), (um, bshape(1), F32), (us, bshape(1), F32),
                (ugls, bshape(1), F32), (2, bshape(), I32), (ugm, bshape(1), F32), (utie, bshape(1), F32)], [N, C], symbolic)
    tz, tm, g = gzs(k, 1, 2, 3, 4, 5, "r1")
    share = k.let(f"({k.load(6, 'r0')} * {k.let(f'(1.0 / {k.load(7, R0)})')})")
    sel = k.let(f"select(0.0, {share}, {k.let(f'({tz} == {tm})', 'bool')})")
    k.store(k.let(f"({g} + {sel})"))
    add("dZ", k, "thread")

    # 10. db2 = Sum(dZ, [0])
    k = Kernel([(udb2, [C], F32), (udZ, bshape(C), F32)], [C], symbolic)
    k.acc()
    r1 = k.loop(N)
    k.update(k.load(1, k.idx2(r1, C, "r0")))
    k.end()
    k.store("acc0")
    add("db2", k, f"tmpl:reduce;op=sum;axis=0;M={Bk};N={C}")

    # 11. dW2 = dZ^T relu(Z1): the ReLU inlined into the batch loop (Z1 bound first)
    k = Kernel([(udW2, [C, H], F32), (uZ1, bshape(H), F32), (udZ, bshape(C), F32)], [C, H], symbolic)
    k.acc()
    r2 = k.loop(N)
    tdz = k.load(2, k.idx2(r2, C, "r0"))
    tz = k.load(1, f"({r2} * {H}) + r1")
    k.update(k.let(f"({tdz} * {k.let(f'max({tz}, 0.0)')})"))
    k.end()
    k.store("acc0")
    add("dW2", k, f"tmpl:gemm;dtype=f32;epi=store;ta=1;tb=1;M={C};N={H};K={Bk};pb=relu;swap_ab=1")

    # 12. dH1 = dZ W2
    k = Kernel([(udH1, bshape(H), F32), (udZ, bshape(C), F32), (5, [C, H], F32)], [N, H], symbolic)
    k.acc()
    r2 = k.loop(C)
    tdz = k.load(1, f"(r0 * {C}) + {r2}")
    tw = k.load(2, k.idx2(r2, H, "r1"))
    k.update(k.let(f"({tdz} * {tw})"))
    k.end()
    k.store("acc0")
    add("dH1", k, f"tmpl:gemm;dtype=f32;epi=store;ta=0;tb=1;M={Bk};N={H};K={C}")

    def masked(k, zbuf, abuf, r):
        tz = k.load(zbuf, f"({r} * {H}) + r0")
        eq = k.let(f"({tz} == {k.let(f'max({tz}, 0.0)')})", "bool")
        return k.let(f"select(0.0, {k.load(abuf, k.idx2(r, H, 'r0'))}, {eq})")

    # 13. db1 = Sum(Where(Z1 == relu(Z1), dH1, 0), [0])
    k = Kernel([(udb1, [H], F32), (uZ1, bshape(H), F32), (udH1, bshape(H), F32)], [H], symbolic)
    k.acc()
    r1 = k.loop(N)
    k.update(masked(k, 1, 2, r1))
    k.end()
    k.store("acc0")
    add("db1", k, f"tmpl:reduce;op=sum;axis=0;M={Bk};N={H};pa=mask;in_a=2;za=1")

    # 14. dW1 = Where(Z1 == relu(Z1), dH1, 0)^T x
    k = Kernel([(udW1, [H, D], F32), (udH1, bshape(H), F32), (uZ1, bshape(H), F32), (1, bshape(D), F32)], [H, D], symbolic)
    k.acc()
    r2 = k.loop(N)
    m = masked(k, 2, 1, r2)
    tx = k.load(3, f"({r2} * {D}) + r1")
    k.update(k.let(f"({m} * {tx})"))
    k.end()
    k.store("acc0")
    add("dW1", k, f"tmpl:gemm;dtype=f32;epi=store;ta=1;tb=1;M={H};N={D};K={Bk};pa=mask;in_a=1;in_b=3;za=2")

    outs = dict(loss=uloss, dW1=udW1, db1=udb1, dW2=udW2, db2=udb2)
    return ks, leaves, outs


def f16_linear(M: int, N: int, K: int, bias: bool = True, relu_a: bool = False, relu_out: bool = False):
    """An f16 Linear forward as the lowering renders an f16 reduce: loads widened to f32 inside the loop,
    f32 accumulation, f16(acc) after it (codegen/lower.go:667-716), the bias add in f16; relu_a applies
    the ReLU of the previous layer to the loaded input (the consumer-side form), relu_out applies it to
    this layer's output (max(f16(acc) + b, 0.0h), the producer-side form). Returns (wgsl, bufs, ws, wc,
    expected key)."""
    k = Kernel([(30, [M, N], F16), (1, [M, K], F16), (2, [N, K], F16)] + ([(3, [N], F16)] if bias else []),
               [M, N], f16=True)
    k.acc()
    r2 = k.loop(K)
    tx = k.load(1, k.idx2("r0", K, r2), widen=True)
    if relu_a:
        tx = k.let(f"max({tx}, 0.0)")
    tw = k.load(2, f"(r1 * {K}) + {r2}", widen=True)
    k.update(k.let(f"({tx} * {tw})"))
    k.end()
    if bias:
        t = k.let(f"(f16(acc0) + {k.load(3, 'r1', 'f16')})", "f16")
        k.store(k.let(f"max({t}, 0.0h)", "f16") if relu_out else t)
    else:
        k.store("f16(acc0)")
    epi = ("bias_relu" if relu_out else "bias") if bias else "store"
    key = f"tmpl:gemm;dtype=f16;epi={epi};ta=0;tb=0;M={M};N={N};K={K}" + (";pa=relu" if relu_a else "")
    bufs = [(u, int(np.prod(s)), d, list(s)) for u, s, d in k.bufs]
    return k.source(), bufs, tuple(k.ws), tuple(k.wc), key


def mlp3_step(B: int, D0: int, D1: int, D2: int, D3: int):
    """Config 3's step (three f16 Linear layers with ReLU, MSE mean loss, f32 backward) as rendered
    kernels, following the graph the oracle restates (ora_mlp3_f16_step, oracle/anneal_oracle.c): each
    forward layer an f16 reduce (widened loads, f32 accumulation, f16(acc)) with the f16 bias add fused
    after it and the previous layer's ReLU inlined into its loop; loss = f16(Sum((P - t)^2)) * (1/(B*D3))
    as one f16 reduce over both axes; the loss adjoint gP = s*d + s*d with d = f16(P - t), materialised
    for its three readers; the backward contractions in f32 (an f32 adjoint times an f16 weight or
    activation promotes to f32, tensor/ops.go:74-79), the ReLU masks Where(z == max(z, 0), adj, 0)
    inlined into the contractions and column sums that read the adjoint. Returns (kernels, leaves,
    outputs) like mlp_ce_step. The mixed f32 x f16 contractions select the f32 template with their f16
    operands (and mask sources) widened by a prologue (wa / wb / wza keys)."""
    s = f32_lit(1.0 / (B * D3))
    leaves = dict(x=1, t=2, W1=3, b1=4, W2=5, b2=6, W3=7, b3=8)
    uZ1, uZ2, uP, uloss, ugP, udb3, udW3, udH2, udb2, udW2, udH1, udb1, udW1 = range(10, 23)
    ks = []

    def add(name, k, plan):
        ks.append((name, k.source(), [(u, int(np.prod(sh)), dt, list(sh)) for u, sh, dt in k.bufs], tuple(k.ws),
                   tuple(k.wc), plan))

    def linear(name, out, xin, xdim, w, b, n, relu_in):
        k = Kernel([(out, [B, n], F16), (xin, [B, xdim], F16), (w, [n, xdim], F16), (b, [n], F16)], [B, n], f16=True)
        k.acc()
        r2 = k.loop(xdim)
        tx = k.load(1, k.idx2("r0", xdim, r2), widen=True)
        if relu_in:
            tx = k.let(f"max({tx}, 0.0)")
        tw = k.load(2, f"(r1 * {xdim}) + {r2}", widen=True)
        k.update(k.let(f"({tx} * {tw})"))
        k.end()
        k.store(k.let(f"(f16(acc0) + {k.load(3, 'r1', 'f16')})", "f16"))
        add(name, k, f"tmpl:gemm;dtype=f16;epi=bias;ta=0;tb=0;M={B};N={n};K={xdim}" + (";pa=relu" if relu_in else ""))

    linear("fc1", uZ1, 1, D0, 3, 4, D1, False)
    linear("fc2", uZ2, uZ1, D1, 5, 6, D2, True)
    linear("fc3", uP, uZ2, D2, 7, 8, D3, True)

    # loss = f16(Sum((P - t)^2)) * s: an f16 reduce over both axes, the f32 constant promoting after it
    k = Kernel([(uloss, [1], F32), (uP, [B, D3], F16), (2, [B, D3], F16)], [], f16=True)
    k.acc()
    r0 = k.loop(B)
    r1 = k.loop(D3)
    tp = k.load(1, k.idx2(r0, D3, r1), widen=True)
    tt = k.load(2, k.idx2(r0, D3, r1), widen=True)
    d = k.let(f"({tp} - {tt})")
    k.update(k.let(f"({d} * {d})"))
    k.end()
    k.end()
    k.store(k.let(f"(f32({k.let('f16(acc0)', 'f16')}) * {s})"))
    add("loss", k, "wave")

    # gP = s*d + s*d, d = f16(P - t): elementwise, materialised for db3, dW3 and dH2
    k = Kernel([(ugP, [B, D3], F32), (uP, [B, D3], F16), (2, [B, D3], F16)], [B, D3], f16=True)
    i = k.idx2("r0", D3, "r1")
    d = k.let(f"({k.load(1, i, 'f16')} - {k.load(2, i, 'f16')})", "f16")
    sd = k.let(f"(f32({d}) * {s})")
    k.store(k.let(f"({sd} + {sd})"))
    add("gP", k, "thread")

    def colsum(name, out, n, adj, zbuf=None):
        # Sum over the batch of the adjoint, masked by the ReLU of z when given
        bufs = [(out, [n], F32), (adj, [B, n], F32)] + ([(zbuf, [B, n], F16)] if zbuf else [])
        k = Kernel(bufs, [n], f16=zbuf is not None)
        k.acc()
        r1 = k.loop(B)
        a = k.load(1, k.idx2(r1, n, "r0"))
        if zbuf:
            z = k.load(2, f"({r1} * {n}) + r0", widen=True)
            eq = k.let(f"({z} == {k.let(f'max({z}, 0.0)')})", "bool")
            a = k.let(f"select(0.0, {a}, {eq})")
        k.update(a)
        k.end()
        k.store("acc0")
        add(name, k, f"tmpl:reduce;op=sum;axis=0;M={B};N={n}" + ("" if zbuf is None else ";pa=mask;in_a=1;za=2;wza=1"))

    def masked_adj(k, adj, zbuf, r, n, col):
        # Where(z == max(z, 0), adj, 0) at (r, col) of [B, n], z an f16 activation widened
        z = k.load(zbuf, f"({r} * {n}) + {col}", widen=True)
        eq = k.let(f"({z} == {k.let(f'max({z}, 0.0)')})", "bool")
        return k.let(f"select(0.0, {k.load(adj, k.idx2(r, n, col))}, {eq})")

    def dweight(name, out, m, n, adj, zmask, act, relu_act):
        # dW[m, n] = Sum_b adj'[b, m] * act'[b, n]: adj' the (masked) f32 adjoint, act' the f16 input (ReLU'd)
        bufs = [(out, [m, n], F32), (adj, [B, m], F32), (act, [B, n], F16)] + ([(zmask, [B, m], F16)] if zmask else [])
        k = Kernel(bufs, [m, n], f16=True)
        k.acc()
        r2 = k.loop(B)
        a = masked_adj(k, 1, 3, r2, m, "r0") if zmask else k.load(1, k.idx2(r2, m, "r0"))
        x = k.load(2, f"({r2} * {n}) + r1", widen=True)
        if relu_act:
            x = k.let(f"max({x}, 0.0)")
        k.update(k.let(f"({a} * {x})"))
        k.end()
        k.store("acc0")
        key = f"tmpl:gemm;dtype=f32;epi=store;ta=1;tb=1;M={m};N={n};K={B}"
        key += (";pa=mask" if zmask else "") + (";pb=relu" if relu_act else "") + ";wb=1"
        add(name, k, key + (";wza=1;in_a=1;in_b=2;za=3" if zmask else ""))

    def dinput(name, out, n, m, adj, zmask, w):
        # dX[b, n] = Sum_j adj'[b, j] * W[j, n]: the f32 adjoint (masked) times the f16 weight
        bufs = [(out, [B, n], F32), (adj, [B, m], F32), (w, [m, n], F16)] + ([(zmask, [B, m], F16)] if zmask else [])
        k = Kernel(bufs, [B, n], f16=True)
        k.acc()
        r2 = k.loop(m)
        if zmask:
            z = k.load(3, f"(r0 * {m}) + {r2}", widen=True)
            eq = k.let(f"({z} == {k.let(f'max({z}, 0.0)')})", "bool")
            a = k.let(f"select(0.0, {k.load(1, k.idx2('r0', m, r2))}, {eq})")
        else:
            a = k.load(1, k.idx2("r0", m, r2))
        wv = k.load(2, k.idx2(r2, n, "r1"), widen=True)
        k.update(k.let(f"({a} * {wv})"))
        k.end()
        k.store("acc0")
        key = f"tmpl:gemm;dtype=f32;epi=store;ta=0;tb=1;M={B};N={n};K={m}" + (";pa=mask" if zmask else "") + ";wb=1"
        add(name, k, key + (";wza=1;in_a=1;in_b=2;za=3" if zmask else ""))

    colsum("db3", udb3, D3, ugP)
    dweight("dW3", udW3, D3, D2, ugP, None, uZ2, True)
    dinput("dH2", udH2, D2, D3, ugP, None, 7)
    colsum("db2", udb2, D2, udH2, uZ2)
    dweight("dW2", udW2, D2, D1, udH2, uZ2, uZ1, True)
    dinput("dH1", udH1, D1, D2, udH2, uZ2, 5)
    colsum("db1", udb1, D1, udH1, uZ1)
    dweight("dW1", udW1, D1, D0, udH1, uZ1, 1, False)
    outs = dict(loss=uloss, dW1=udW1, db1=udb1, dW2=udW2, db2=udb2, dW3=udW3, db3=udb3)
    return ks, leaves, outs


def chain_step(R: int, Cc: int):
    """Config 5's step (Y = Shrink(Pad(Permute(X))) with one element of padding on every side, per-row
    softmax S = e / s with e = Exp2((y - m) / ln2), r = 1 / Sqrt(Mean(S^2) + 1e-6), out = S * r * g,
    loss = Sum(out), and its backward) as rendered kernels, following the graph the oracle restates
    (ora_chain_step, oracle/anneal_oracle.c). Every reduce is materialised (m, the tie count, s, Sum(S^2),
    the loss, dg, and the backward's gR, gRs, gm); the elementwise chains, the per-row scalars r and the
    rule-by-rule backward factors are recomputed inline by each kernel that reads them; dX is one
    elementwise kernel. The movement chain is index arithmetic inside every load of Y
    (schedule/index.go:30-225): the shrink's +1 offsets, the pad's validity Where (bounds 0 < i + 1 < Cc + 1
    and 0 < j + 1 < R + 1, fill the enclosing reduce's identity: -FLT_MAX under the max, 0 elsewhere), the
    pad's -1, and the permute's swapped indices into X[R, Cc]; dX runs the inverse chain (the Pad of the
    adjoint that Shrink's rule gives, the Shrink that Pad's rule gives, the inverse Permute).
    Returns (kernels, leaves, outputs) like mlp_ce_step."""
    leaves = dict(X=1, g=2)
    um, utie, us, usq, uloss, udg, ugR, ugRs, ugm, udX = range(10, 20)
    ks = []
    rR, eps = f32_lit(1.0 / R), f32_lit(1e-6)
    NEG = "bitcast<f32>(0xff7fffffu)"

    def add(name, k, plan):
        ks.append((name, k.source(), [(u, int(np.prod(sh)), dt, list(sh)) for u, sh, dt in k.bufs], tuple(k.ws),
                   tuple(k.wc), plan))

    def y(k, i, j, fill):
        # element (i, j) of Y: shrink offsets, pad validity and -1, permute into X[R, Cc] (data1)
        a = k.let(f"({i} + 1)", "i32")
        b = k.let(f"({j} + 1)", "i32")
        c = k.let(f"(0 < {a})", "bool")
        c = k.let(f"({c} && {k.let(f'({a} < {Cc + 1})', 'bool')})", "bool")
        c = k.let(f"({c} && {k.let(f'(0 < {b})', 'bool')})", "bool")
        c = k.let(f"({c} && {k.let(f'({b} < {R + 1})', 'bool')})", "bool")
        sj = k.let(f"({b} - 1)", "i32")
        si = k.let(f"({a} - 1)", "i32")
        x = k.load(1, k.idx2(sj, Cc, si))
        return k.let(f"select({fill}, {x}, {c})")

    def row_kernel(out, extra):
        """A reduce over the row j of Y for each row i (r0): data1 = X, then the per-row inputs `extra`
        [(uop, name)] as data2.. . Returns (kernel, loop var, {name: data index})."""
        bufs = [(out, [Cc], F32), (1, [R, Cc], F32)] + [(u, [Cc], F32) for u, _ in extra]
        k = Kernel(bufs, [Cc])
        idx = {nm: 2 + n for n, (_, nm) in enumerate(extra)}
        return k, idx

    def scalars(k, idx, need):
        """Per-row values the kernel reads (loaded once, before the loop, as the lowering hoists them)."""
        v = {nm: k.load(idx[nm], "r0") for nm in need if nm in idx}
        if "rs" in need:
            v["rs"] = k.let(f"(1.0 / {v['s']})")
        if "r" in need:
            q = k.let(f"({v['sq']} * {rR})")
            v["T"] = k.let(f"sqrt(({q} + {eps}))")
            v["r"] = k.let(f"(1.0 / {v['T']})")
        if "gsq" in need:
            gT = k.let(f"((-{v['gR']} * {v['r']}) * {v['r']})")
            gu = k.let(f"({gT} * (1.0 / (2.0 * {v['T']})))")
            v["gsq"] = k.let(f"({gu} * {rR})")
        if "gs" in need:
            v["gs"] = k.let(f"((-{v['gRs']} * {v['rs']}) * {v['rs']})")
        return v

    def elem(k, v, yv, want):
        """Per-element values of row r0 at the loop's j from y: e, S, A, gS, gzs."""
        zs = k.let(f"({yv} - {v['m']})")
        e = k.let(f"exp2(({zs} * {LOG2E}))")
        out = {"e": e}
        if "S" in want or "A" in want or "gS" in want or "gzs" in want:
            out["S"] = k.let(f"({e} * {v['rs']})")
        if "A" in want:
            out["A"] = k.let(f"({out['S']} * {v['r']})")
        if "gS" in want or "gzs" in want:
            t2 = k.let(f"({v['gsq']} * {out['S']})")
            out["gS"] = k.let(f"((({v['g']} * {v['r']}) + {t2}) + {t2})")
        if "gzs" in want:
            ge = k.let(f"(({out['gS']} * {v['rs']}) + {v['gs']})")
            gv = k.let(f"(({ge} * {e}) * {LN2})")
            out["gzs"] = k.let(f"({gv} * {LOG2E})")
        return out

    # 1. m = Max over the row (pad fill -FLT_MAX)
    k, idx = row_kernel(um, [])
    k.acc("M")
    r1 = k.loop(R)
    k.update(y(k, "r0", r1, NEG))
    k.end()
    k.store("acc0")
    add("max", k, "wave")

    # 2. the tie count Sum(Cast(y == m)) (the max rule's mask, tensor/gradient_ruleset.go:307-320)
    k, idx = row_kernel(utie, [(um, "m")])
    m = k.load(idx["m"], "r0")
    k.acc()
    r1 = k.loop(R)
    yv = y(k, "r0", r1, "0.0")
    k.update(k.let(f"select(0.0, 1.0, {k.let(f'({yv} == {m})', 'bool')})"))
    k.end()
    k.store("acc0")
    add("tie", k, "wave")

    # 3. s = Sum(e)
    k, idx = row_kernel(us, [(um, "m")])
    v = scalars(k, idx, ["m"])
    k.acc()
    r1 = k.loop(R)
    k.update(elem(k, v, y(k, "r0", r1, "0.0"), [])["e"])
    k.end()
    k.store("acc0")
    add("sumexp", k, "wave")

    # 4. Sum(S^2)
    k, idx = row_kernel(usq, [(um, "m"), (us, "s")])
    v = scalars(k, idx, ["m", "s", "rs"])
    k.acc()
    r1 = k.loop(R)
    S = elem(k, v, y(k, "r0", r1, "0.0"), ["S"])["S"]
    k.update(k.let(f"({S} * {S})"))
    k.end()
    k.store("acc0")
    add("sumsq", k, "wave")

    # 5. loss = Sum over both axes of A * g (row-major)
    k = Kernel([(uloss, [1], F32), (1, [R, Cc], F32), (um, [Cc], F32), (us, [Cc], F32), (usq, [Cc], F32),
                (2, [Cc], F32)], [])
    k.acc()
    i = k.loop(Cc)
    v = {"m": k.load(2, i), "s": k.load(3, i), "sq": k.load(4, i), "g": k.load(5, i)}
    v["rs"] = k.let(f"(1.0 / {v['s']})")
    q = k.let(f"({v['sq']} * {rR})")
    v["T"] = k.let(f"sqrt(({q} + {eps}))")
    v["r"] = k.let(f"(1.0 / {v['T']})")
    j = k.loop(R)
    A = elem(k, v, y(k, i, j, "0.0"), ["A"])["A"]
    k.update(k.let(f"({A} * {v['g']})"))
    k.end()
    k.end()
    k.store("acc0")
    add("loss", k, "wave")

    # 6. dg = Sum(A) (the Expand rule over the row of out = A * g)
    k, idx = row_kernel(udg, [(um, "m"), (us, "s"), (usq, "sq")])
    v = scalars(k, idx, ["m", "s", "sq", "rs", "r"])
    k.acc()
    r1 = k.loop(R)
    k.update(elem(k, v, y(k, "r0", r1, "0.0"), ["A"])["A"])
    k.end()
    k.store("acc0")
    add("dg", k, "wave")

    # 7. gR = Sum(g * S)
    k, idx = row_kernel(ugR, [(um, "m"), (us, "s"), (2, "g")])
    v = scalars(k, idx, ["m", "s", "g", "rs"])
    k.acc()
    r1 = k.loop(R)
    S = elem(k, v, y(k, "r0", r1, "0.0"), ["S"])["S"]
    k.update(k.let(f"({v['g']} * {S})"))
    k.end()
    k.store("acc0")
    add("gR", k, "wave")

    # 8. gRs = Sum(gS * e)
    k, idx = row_kernel(ugRs, [(um, "m"), (us, "s"), (usq, "sq"), (ugR, "gR"), (2, "g")])
    v = scalars(k, idx, ["m", "s", "sq", "gR", "g", "rs", "r", "gsq"])
    k.acc()
    r1 = k.loop(R)
    el = elem(k, v, y(k, "r0", r1, "0.0"), ["gS"])
    k.update(k.let(f"({el['gS']} * {el['e']})"))
    k.end()
    k.store("acc0")
    add("gRs", k, "wave")

    # 9. gm = Sum(-gzs)
    k, idx = row_kernel(ugm, [(um, "m"), (us, "s"), (usq, "sq"), (ugR, "gR"), (ugRs, "gRs"), (2, "g")])
    v = scalars(k, idx, ["m", "s", "sq", "gR", "gRs", "g", "rs", "r", "gsq", "gs"])
    k.acc()
    r1 = k.loop(R)
    gz = elem(k, v, y(k, "r0", r1, "0.0"), ["gzs"])["gzs"]
    k.update(k.let(f"-{gz}"))
    k.end()
    k.store("acc0")
    add("gm", k, "wave")

    # 10. dX[j, i] = gzs + Where(y == m, gm * (1 / tie), 0) through the inverse chain
    bufs = [(udX, [R, Cc], F32), (1, [R, Cc], F32)] + [(u, [Cc], F32) for u in (um, us, usq, ugR, ugRs, ugm, utie, 2)]
    k = Kernel(bufs, [R, Cc])
    # output (j, i) = (r0, r1); the inverse Permute gives adjoint index (i, j), the Shrink of the padded
    # adjoint adds 1 to each, the Pad's validity guards them (fill 0) and its -1 returns to (i, j)
    a = k.let("(r1 + 1)", "i32")
    b = k.let("(r0 + 1)", "i32")
    c = k.let(f"(0 < {a})", "bool")
    c = k.let(f"({c} && {k.let(f'({a} < {Cc + 1})', 'bool')})", "bool")
    c = k.let(f"({c} && {k.let(f'(0 < {b})', 'bool')})", "bool")
    c = k.let(f"({c} && {k.let(f'({b} < {R + 1})', 'bool')})", "bool")
    i = k.let(f"({a} - 1)", "i32")
    j = k.let(f"({b} - 1)", "i32")
    names = ["m", "s", "sq", "gR", "gRs", "gm", "tie", "g"]
    v = {nm: k.load(2 + n, i) for n, nm in enumerate(names)}
    v["rs"] = k.let(f"(1.0 / {v['s']})")
    q = k.let(f"({v['sq']} * {rR})")
    v["T"] = k.let(f"sqrt(({q} + {eps}))")
    v["r"] = k.let(f"(1.0 / {v['T']})")
    gT = k.let(f"((-{v['gR']} * {v['r']}) * {v['r']})")
    gu = k.let(f"({gT} * (1.0 / (2.0 * {v['T']})))")
    v["gsq"] = k.let(f"({gu} * {rR})")
    v["gs"] = k.let(f"((-{v['gRs']} * {v['rs']}) * {v['rs']})")
    yv = y(k, i, j, "0.0")
    gz = elem(k, v, yv, ["gzs"])["gzs"]
    share = k.let(f"({v['gm']} * (1.0 / {v['tie']}))")
    tie = k.let(f"({yv} == {v['m']})", "bool")
    dy = k.let(f"({gz} + select(0.0, {share}, {tie}))")
    k.store(k.let(f"select(0.0, {dy}, {c})"))
    add("dX", k, "thread")
    outs = dict(loss=uloss, dX=udX, dg=udg)
    return ks, leaves, outs
