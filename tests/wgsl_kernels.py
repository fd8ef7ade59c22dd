"""WGSL kernels in the exact shape anneal's codegen renders them (codegen/wgsl.go:41-238), with inputs
and numpy expectations, for the WGSL->HIP rendering path of ah_module_get / ah_run.

Each entry: name -> (wgsl, bufs, local_size, workgroup_count, inputs, expected, sym) where bufs lists
(uop_idx, n_elems, dtype code[, shape]) in binding order (binding 0 = output; n_elems 0 and a shape
with a 0 leading dim for the symbolic batch), inputs maps uop_idx -> array and
expected is the output (data0) as numpy. The header block (bindings, `@compute`, the `fn main` builtin
list and the flat_* / gid_x lets) is the fixed preamble renderInstrs writes for every kernel; bodies use
the instruction forms of codegen/lower.go (InstrGIDVar axis guards, InstrAccInit/AccUpdate, InstrLet
`tN`, InstrStore) and the ALU/constant renderings of codegen/wgsl.go:253-386.
"""
import numpy as np

F32, F16, I32 = 0, 1, 3


def header(bindings, ws, wc, sym_params=None, f16=False):
    """The module preamble renderInstrs emits (bindings, optional params_n, workgroup size, main)."""
    out = ["enable f16;", ""] if f16 else []
    for i, t in enumerate(bindings):
        access = "read_write" if i == 0 else "read"
        out.append(f"@group(0) @binding({i}) var<storage, {access}> data{i}: array<{t}>;")
    if sym_params is not None:
        out.append("struct ParamsN { n0: u32, n1: u32, n2: u32, n3: u32 };")
        out.append(f"@group(0) @binding({len(bindings)}) var<uniform> params_n: ParamsN;")
    out.append("")
    out.append(f"@compute @workgroup_size({ws[0]}, {ws[1]}, {ws[2]})")
    return out


def main_open(ws, wc, dim1_used=False):
    dimx, dimy = wc[0] * ws[0], wc[1] * ws[1]
    out = ["fn main(", "  @builtin(global_invocation_id) gid: vec3<u32>,", "  @builtin(workgroup_id) wid: vec3<u32>,",
           "  @builtin(local_invocation_id) lid: vec3<u32>", ") {"]
    if not dim1_used:
        out.append(f"  let flat_gid_x = gid.x + (gid.y * {dimx}u) + (gid.z * {dimx * dimy}u);")
        out.append(f"  let flat_wid_x = wid.x + (wid.y * {wc[0]}u) + (wid.z * {wc[0] * wc[1]}u);")
    else:
        out.append("  let flat_gid_x = gid.x;")
        out.append("  let flat_wid_x = wid.x;")
    out += ["  let flat_gid_y = gid.y;", "  let flat_wid_y = wid.y;", "  let flat_gid_z = gid.z;", "  let flat_wid_z = wid.z;",
            f"  let gid_x = gid.x + (gid.y * {dimx}u) + (gid.z * {dimx * dimy}u);"]
    return out


def kernels():
    rng = np.random.default_rng(7)
    ks = {}

    # 1. Elementwise Exp (tensor/ops.go:56-65: exp2(x * f32(1/ln2))), 32 elements, workgroup (64,1,1)
    x = rng.standard_normal(32).astype(np.float32)
    ws, wc = (64, 1, 1), (1, 1, 1)
    src = header(["f32", "f32"], ws, wc) + main_open(ws, wc) + [
        "  let r0: i32 = i32(flat_gid_x % 32u);",
        "  if (r0 >= 32) { return; }",
        "  let t3: f32 = data1[r0];",
        "  let t4: f32 = (t3 * 1.442695);",
        "  let t5: f32 = exp2(t4);",
        "  data0[r0] = t5;",
        "}"]
    want = np.exp2(x * np.float32(1.442695)).astype(np.float32)
    ks["exp2_elementwise"] = ("\n".join(src), [(10, 32, F32), (1, 32, F32)], ws, wc, {1: x}, want, None)

    # 2. Matmul [2,3]@[3,2] as REDUCE(ADD, MUL(INDEX, INDEX)) with the unsimplified index chains of
    #    schedule/index.go (webgpu_test.go:224-253 known answer [58, 64, 139, 154])
    A = np.array([1, 2, 3, 4, 5, 6], np.float32)
    B = np.array([7, 8, 9, 10, 11, 12], np.float32)
    src = header(["f32", "f32", "f32"], ws, wc) + main_open(ws, wc) + [
        "  let r0: i32 = i32((flat_gid_x / 2u) % 2u);",
        "  if (r0 >= 2) { return; }",
        "  let r1: i32 = i32(flat_gid_x % 2u);",
        "  if (r1 >= 2) { return; }",
        "  var acc0: f32 = 0.0;",
        "  for (var r2: i32 = 0; r2 < 3; r2++) {",
        "    let t9: f32 = data1[((((r0 * 3) + r2) / 3) % 2) * 3 + (((r0 * 3) + r2) % 3)];",
        "    let t12: f32 = data2[((((r2 * 2) + r1) / 2) % 3) * 2 + (((r2 * 2) + r1) % 2)];",
        "    acc0 = acc0 + (t9 * t12);",
        "  }",
        "  data0[((r0 * 2) + r1)] = acc0;",
        "}"]
    ks["matmul_known_answer"] = ("\n".join(src), [(20, 4, F32), (1, 6, F32), (2, 6, F32)], ws, wc, {1: A, 2: B},
                                 np.array([58, 64, 139, 154], np.float32), None)

    # 3. Row max with the -FLT_MAX identity (codegen/wgsl.go:376-386), rows of 10, and a Where over the
    #    tie mask (select(f, t, cond), codegen/wgsl.go:298-299)
    X = rng.standard_normal((4, 10)).astype(np.float32)
    X[2, 3] = X[2, 7] = X[2].max() + 1.0
    src = header(["f32", "f32"], ws, wc) + main_open(ws, wc) + [
        "  let r0: i32 = i32(flat_gid_x % 40u);",
        "  if (r0 >= 40) { return; }",
        "  var acc0: f32 = bitcast<f32>(0xff7fffffu);",
        "  for (var r1: i32 = 0; r1 < 10; r1++) {",
        "    let t4: f32 = data1[((r0 / 10) * 10) + r1];",
        "    acc0 = max(acc0, t4);",
        "  }",
        "  let t6: f32 = data1[r0];",
        "  let t7: bool = (t6 == acc0);",
        "  let t8: f32 = select(0.0, 1.0, t7);",
        "  data0[r0] = t8;",
        "}"]
    want = (X == X.max(1, keepdims=True)).astype(np.float32).ravel()
    ks["max_tie_mask"] = ("\n".join(src), [(30, 40, F32), (1, 40, F32)], ws, wc, {1: X.ravel()}, want, None)

    # 4. Symbolic batch (tensor.NewSymbolicBatchInput): bounds check on params_n.n0 * trailing and a
    #    loop bound i32(params_n.n0): out[n, j] = sum_i x[i, j] * (1/n)... here out[b, j] = x[b, j] + colsum
    n, J = 7, 4
    xs = rng.standard_normal((n, J)).astype(np.float32)
    ws4, wc4 = (64, 1, 1), (1, 1, 1)
    src = header(["f32", "f32"], ws4, wc4, sym_params=True) + main_open(ws4, wc4) + [
        "  if (gid_x >= params_n.n0 * 4u) { return; }",
        "  let r0: i32 = i32(flat_gid_x / 4u);",
        "  let r1: i32 = i32(flat_gid_x % 4u);",
        "  if (r1 >= 4) { return; }",
        "  var acc0: f32 = 0.0;",
        "  for (var r2: i32 = 0; r2 < i32(params_n.n0); r2++) {",
        "    let t3: f32 = data1[(r2 * 4) + r1];",
        "    acc0 = acc0 + t3;",
        "  }",
        "  let t5: f32 = data1[(r0 * 4) + r1];",
        "  let t6: f32 = (t5 + (acc0 * (1.0 / f32(params_n.n0))));",
        "  data0[(r0 * 4) + r1] = t6;",
        "}"]
    want = (xs + xs.sum(0, dtype=np.float32) * np.float32(1.0 / n)).astype(np.float32).ravel()
    ks["symbolic_batch"] = ("\n".join(src), [(40, 0, F32, [0, J]), (1, 0, F32, [0, J])], ws4, wc4, {1: xs.ravel()}, want, n)

    # 5. LOCAL/GROUP reduction through a workgroup array (Opt seam, codegen/lower.go DefineLocal +
    #    Barrier): 4 rows of 256, one workgroup of 64 per row, strided partials then a serial fold
    R, Cn = 4, 256
    Xr = rng.standard_normal((R, Cn)).astype(np.float32)
    ws5, wc5 = (64, 1, 1), (4, 1, 1)
    src = header(["f32", "f32"], ws5, wc5)
    src += ["var<workgroup> temp0: array<f32, 64>;"]
    src += main_open(ws5, wc5) + [
        "  let r0: i32 = i32(flat_wid_x % 4u);",
        "  if (r0 >= 4) { return; }",
        "  let r1: i32 = i32(lid.x % 64u);",
        "  var acc0: f32 = 0.0;",
        "  for (var r2: i32 = 0; r2 < 4; r2++) {",
        "    let t3: f32 = data1[(r0 * 256) + ((r2 * 64) + r1)];",
        "    acc0 = acc0 + t3;",
        "  }",
        "  temp0[r1] = acc0;",
        "  workgroupBarrier();",
        "  if ((r1 == 0)) {",
        "    var acc1: f32 = 0.0;",
        "    for (var r3: i32 = 0; r3 < 64; r3++) {",
        "      acc1 = acc1 + temp0[r3];",
        "    }",
        "    data0[r0] = acc1;",
        "  }",
        "}"]
    want = Xr.sum(1, dtype=np.float64).astype(np.float32)
    ks["group_reduce_lds"] = ("\n".join(src), [(50, R, F32), (1, R * Cn, F32)], ws5, wc5, {1: Xr.ravel()}, want, None)

    # 6. f16 storage: f16 elementwise math and an f32 accumulator over f16 products narrowed at the
    #    end with f16(acc) (codegen/lower.go:667-716), plus the f16 -FLT_MAX literal form
    a16 = (rng.standard_normal((3, 16)) * 2).astype(np.float16)
    b16 = (rng.standard_normal(16) * 2).astype(np.float16)
    src = header(["f16", "f16", "f16"], ws, wc, f16=True) + main_open(ws, wc) + [
        "  let r0: i32 = i32(flat_gid_x % 3u);",
        "  if (r0 >= 3) { return; }",
        "  var acc0: f32 = 0.0;",
        "  for (var r1: i32 = 0; r1 < 16; r1++) {",
        "    let t2: f16 = data1[(r0 * 16) + r1];",
        "    let t3: f16 = data2[r1];",
        "    let t4: f16 = (t2 * t3);",
        "    acc0 = acc0 + f32(t4);",
        "  }",
        "  let t5: f16 = max(f16(acc0), bitcast<f16>(0xFBFFu));",
        "  data0[r0] = (t5 * f16(0.5));",
        "}"]
    prod = (a16.astype(np.float32) * b16.astype(np.float32)).astype(np.float16).astype(np.float32)
    acc = np.zeros(3, np.float32)
    for k in range(16):
        acc = (acc + prod[:, k]).astype(np.float32)
    want = (np.maximum(acc.astype(np.float16), np.float16(-65504)).astype(np.float32) * 0.5).astype(np.float16)
    ks["f16_accumulate"] = ("\n".join(src), [(60, 3, F16), (1, 48, F16), (2, 16, F16)], ws, wc,
                            {1: a16.astype(np.float32).ravel(), 2: b16.astype(np.float32)}, want.astype(np.float32), None)

    # 7. vec4 accumulators of the vectorized Opt path (codegen/lower.go:865-941): 4 outputs per thread
    xv = rng.standard_normal(128).astype(np.float32)
    wv = rng.standard_normal(8).astype(np.float32)
    ws7, wc7 = (4, 1, 1), (1, 1, 1)
    src = header(["f32", "f32", "f32"], ws7, wc7) + main_open(ws7, wc7) + [
        "  let r0: i32 = i32(flat_gid_x % 4u);",
        "  if (r0 >= 4) { return; }",
        "  var acc0: vec4<f32> = vec4<f32>(0.0);",
        "  for (var r1: i32 = 0; r1 < 8; r1++) {",
        "    let rA0: f32 = data2[r1];",
        "    let rB0: vec4<f32> = vec4<f32>(data1[(r1 * 16) + (r0 * 4) + 0], data1[(r1 * 16) + (r0 * 4) + 1], "
        "data1[(r1 * 16) + (r0 * 4) + 2], data1[(r1 * 16) + (r0 * 4) + 3]);",
        "    acc0 = acc0 + (rA0 * rB0);",
        "  }",
        "  data0[(r0 * 4) + 0] = acc0.x;",
        "  data0[(r0 * 4) + 1] = acc0.y;",
        "  data0[(r0 * 4) + 2] = acc0.z;",
        "  data0[(r0 * 4) + 3] = acc0.w;",
        "}"]
    Xv = xv.reshape(8, 16)
    want = np.zeros(16, np.float32)
    for k in range(8):
        want = (want + (wv[k] * Xv[k]).astype(np.float32)).astype(np.float32)
    ks["vec4_accumulators"] = ("\n".join(src), [(70, 16, F32), (1, 128, F32), (2, 8, F32)], ws7, wc7,
                               {1: xv, 2: wv}, want, None)

    # 8. The reference's own hand-written probe shader (backend/webgpu/diag_test.go:84-101): untyped
    #    lets/vars, explicit `f` / `u` suffixes, a u32 loop
    probe = """
@group(0) @binding(0) var<storage, read_write> out: array<f32>;
@group(0) @binding(1) var<storage, read>       inp: array<f32>;

@compute @workgroup_size(256, 1, 1)
fn main(@builtin(global_invocation_id) gid: vec3<u32>) {
    let idx  = gid.x;
    let seed = inp[0u] + f32(idx % 7u) * 0.001f;
    var a0   = seed;
    var a1   = seed + 1.0f;
    var a2   = seed + 2.0f;
    var a3   = seed + 3.0f;
    let c    = 1.00001f;
    let d    = 0.00001f;
    for (var i: u32 = 0u; i < 256u; i++) {
        a0 = a0 * c + d;
        a1 = a1 * c + d;
        a2 = a2 * c + d;
        a3 = a3 * c + d;
    }
    out[idx] = a0 + a1 + a2 + a3;
}
"""
    inp = np.array([0.5], np.float32)
    seeds = (np.float32(0.5) + (np.arange(256) % 7).astype(np.float32) * np.float32(0.001)).astype(np.float32)
    accs = [seeds + np.float32(j) for j in range(4)]
    accs = [a.astype(np.float32) for a in accs]
    for _ in range(256):
        accs = [(a * np.float32(1.00001)).astype(np.float32) + np.float32(0.00001) for a in accs]
        accs = [a.astype(np.float32) for a in accs]
    want = (((accs[0] + accs[1]).astype(np.float32) + accs[2]).astype(np.float32) + accs[3]).astype(np.float32)
    ks["diag_fma_probe"] = (probe, [(80, 256, F32), (1, 1, F32)], (256, 1, 1), (1, 1, 1), {1: inp}, want, None)
    return ks


def matmul_wgsl(M, N, K, ta=False, tb=True, b_first=False, offset=0, bias=None):
    """A contraction as the reference's codegen renders it (codegen/lower.go REDUCE(ADD, MUL(INDEX, INDEX))
    with the unsimplified index chains of schedule/index.go): out[m, n] = sum_k A(m, k) * B(k, n), A read
    from data1 ([M,K], or [K,M] with ta), B from data2 ([K,N] with tb, else [N,K]); with b_first the B load
    is emitted first. offset shifts A's index (no longer a zero-offset contraction). bias adds data3[n]
    after the loop (Linear's forward epilogue, the add rendered "(a + b)" by codegen/wgsl.go:270):
    "let" (a let of the sum), "inline" (the sum in the store), "let_rev" (bias first), "rows" (data3[m],
    not a bias of the columns). Returns (wgsl, local_size, workgroup_count) for ExecItem."""
    ws = (64, 1, 1)
    wc = ((M * N + 63) // 64, 1, 1)
    if ta:   # A(m, k) at k*M + m, through a chain over the flat [K, M] view
        ia = f"((((r2 * {M}) + r0) / {M}) % {K}) * {M} + (((r2 * {M}) + r0) % {M})"
    else:
        ia = f"((((r0 * {K}) + r2) / {K}) % {M}) * {K} + (((r0 * {K}) + r2) % {K})"
    if offset:
        ia = f"({ia}) + {offset}"
    if tb:   # B(k, n) at k*N + n
        ib = f"((((r2 * {N}) + r1) / {N}) % {K}) * {N} + (((r2 * {N}) + r1) % {N})"
    else:
        ib = f"((((r1 * {K}) + r2) / {K}) % {N}) * {K} + (((r1 * {K}) + r2) % {K})"
    loads = [f"    let t9: f32 = data1[{ia}];", f"    let t12: f32 = data2[{ib}];"]
    if b_first:
        loads.reverse()
    post, store = [], "acc0"
    if bias:
        bi = f"(((r0 * {N}) + r1) / {N}) % {M}" if bias == "rows" else f"(((r0 * {N}) + r1) % {N})"
        post = [f"  let t14: f32 = data3[{bi}];"]
        add = "(t14 + acc0)" if bias == "let_rev" else "(acc0 + t14)"
        if bias == "inline":
            store = add
        else:
            post.append(f"  let t15: f32 = {add};")
            store = "t15"
    src = header(["f32", "f32", "f32"] + (["f32"] if bias else []), ws, wc) + main_open(ws, wc) + [
        f"  let r0: i32 = i32((flat_gid_x / {N}u) % {M}u);",
        f"  if (r0 >= {M}) {{ return; }}",
        f"  let r1: i32 = i32(flat_gid_x % {N}u);",
        f"  if (r1 >= {N}) {{ return; }}",
        "  var acc0: f32 = 0.0;",
        f"  for (var r2: i32 = 0; r2 < {K}; r2++) {{"] + loads + [
        "    acc0 = acc0 + (t9 * t12);",
        "  }"] + post + [
        f"  data0[((r0 * {N}) + r1)] = {store};",
        "}"]
    return "\n".join(src), ws, wc
