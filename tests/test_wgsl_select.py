"""Template selection for rendered WGSL (host side): a kernel that is a plain contraction of three f32
buffers is recognised from its evaluated index expressions and runs the MFMA contraction template
(tmpl:gemm) instead of its rendering; everything else keeps the rendering. The GPU side of the same
kernels is tests/test_gpu_wgsl.py."""
import pytest

import wgsl_kernels as W
from anneal_amd import _lib as L


def test_reference_matmul_known_answer_is_selected():
    # webgpu_test.go:224-253's [2,3] @ [3,2]: A [M,K] K-contiguous, B [K,N] (tb=1)
    assert L.wgsl_template_key(W.kernels()["matmul_known_answer"][0]) == \
        "tmpl:gemm;dtype=f32;epi=store;ta=0;tb=1;M=2;N=2;K=3"


@pytest.mark.parametrize("ta,tb,b_first", [(False, True, False), (True, True, False), (False, False, True),
                                           (True, False, True)])
def test_layouts_and_load_order(ta, tb, b_first):
    M, N, K = 96, 80, 64
    src, _, _ = W.matmul_wgsl(M, N, K, ta=ta, tb=tb, b_first=b_first)
    want = f"tmpl:gemm;dtype=f32;epi=store;ta={int(ta)};tb={int(tb)};M={M};N={N};K={K}"
    assert L.wgsl_template_key(src) == want      # the load order does not change the binding roles


@pytest.mark.parametrize("name", ["exp2_elementwise", "max_tie_mask", "symbolic_batch", "f16_accumulate",
                                  "vec4_accumulators", "group_reduce_lds", "diag_fma_probe"])
def test_other_kernels_keep_their_rendering(name):
    ks = W.kernels()
    if name not in ks:
        pytest.skip(f"no kernel {name}")
    assert L.wgsl_template_key(ks[name][0]) == ""


def test_offset_index_is_not_a_contraction():
    src, _, _ = W.matmul_wgsl(16, 16, 16, offset=1)
    assert L.wgsl_template_key(src) == ""


def test_swapped_bindings_select_swap_ab():
    # B bound first (data1 holds B): the same contraction with the operand PARAMs swapped
    src, _, _ = W.matmul_wgsl(32, 48, 16)
    src = src.replace("data1[", "dataX[").replace("data2[", "data1[").replace("dataX[", "data2[")
    assert L.wgsl_template_key(src) == "tmpl:gemm;dtype=f32;epi=store;ta=0;tb=1;M=32;N=48;K=16;swap_ab=1"


@pytest.mark.parametrize("mutate", [
    lambda s: s.replace("var acc0: f32 = 0.0;", "var acc0 = 0.0;"),            # no type: not the emitted form
    lambda s: s.replace("acc0 = acc0 + (t9 * t12);", "acc0 = acc0 + (t9 + t12);"),
    lambda s: s.replace("data0[((r0 * 2) + r1)] = acc0;", "data0[((r0 * 2) + r1)] = (acc0 - 2.0);"),
    lambda s: s.replace("let t9: f32 = data1[", "let t9: f32 = data1[((("),   # unbalanced parentheses
    lambda s: s[: len(s) // 2],                                                  # truncated
    lambda s: "",
])
def test_malformed_or_other_forms_are_not_selected(mutate):
    assert L.wgsl_template_key(mutate(W.kernels()["matmul_known_answer"][0])) == ""


def test_huge_axis_is_left_to_the_rendering():
    src, _, _ = W.matmul_wgsl(16, 16, 1 << 20)
    assert L.wgsl_template_key(src) == ""


@pytest.mark.parametrize("form", ["let", "inline", "let_rev"])
def test_bias_epilogue_is_selected(form):
    src, _, _ = W.matmul_wgsl(64, 48, 32, bias=form)
    assert L.wgsl_template_key(src) == "tmpl:gemm;dtype=f32;epi=bias;ta=0;tb=1;M=64;N=48;K=32"


def test_bias_over_rows_is_not_a_column_bias():
    src, _, _ = W.matmul_wgsl(64, 48, 32, bias="rows")
    assert L.wgsl_template_key(src) == ""


def test_scaled_store_is_selected_with_its_scale():
    # acc * c (a constant scale, e.g. a mean's 1/B) is the store epilogue's scale, spelled exactly
    src = W.kernels()["matmul_known_answer"][0].replace("data0[((r0 * 2) + r1)] = acc0;",
                                                       "data0[((r0 * 2) + r1)] = (acc0 * 2.0);")
    assert L.wgsl_template_key(src) == "tmpl:gemm;dtype=f32;epi=store;ta=0;tb=1;M=2;N=2;K=3;scale=0x1p+1"


# ── the configs-1/4 step as rendered kernels (tests/wgsl_lower.py) ──────────────────────────────────

import wgsl_lower as WL  # noqa: E402


@pytest.mark.parametrize("symbolic", [False, True])
@pytest.mark.parametrize("shape", [(64, 784, 128, 10), (256, 512, 2048, 512)])
def test_rendered_mlp_ce_step_selects_a_template_or_the_wave_rendering(shape, symbolic):
    """Every kernel of the rendered step is run by a hand-written template (the contractions with their
    ReLU and mask prologues and bias epilogues, the plain row max and column sum, the masked column sum
    db1) or, for the softmax-CE reductions with elementwise prologues, by the wave-per-output rendering;
    only the elementwise dZ kernel keeps the one-thread-per-output rendering."""
    B, D, H, C = shape
    ks, _, _ = WL.mlp_ce_step(B, D, H, C, symbolic=symbolic)
    plans = {name: L.wgsl_plan(src) for name, src, *_ in ks}
    for name, src, bufs, ws, wc, want in ks:
        assert plans[name] == want, (name, plans[name], want)
    assert sum(p.startswith("tmpl:gemm") for p in plans.values()) == 5
    assert sum(p.startswith("tmpl:reduce") for p in plans.values()) == 3
    assert sorted(n for n, p in plans.items() if p == "wave") == ["gls", "gmax", "loss", "sumexp", "tie"]
    assert [n for n, p in plans.items() if p == "thread"] == ["dZ"]


@pytest.mark.parametrize("bias,relu,relu_out", [(True, False, False), (False, False, False), (True, True, False),
                                               (True, False, True), (True, True, True)])
def test_f16_contraction_with_narrowing_is_selected(bias, relu, relu_out):
    """An f16 reduce (loads widened to f32 in the loop, f16(acc) after it) selects the f16 MFMA template,
    with the ReLU as the input's prologue, as the output's epilogue, or both."""
    src, _, _, _, key = WL.f16_linear(256, 128, 192, bias=bias, relu_a=relu, relu_out=relu_out)
    assert L.wgsl_template_key(src) == key


def test_masked_column_sum_needs_the_same_index_for_z_and_the_adjoint():
    """The masked column sum (a ReLU layer's bias gradient) selects the reduce template only when z is read
    at the adjoint's element; shifted, it keeps the wave rendering."""
    ks, _, _ = WL.mlp_ce_step(64, 784, 128, 10)
    src = dict((n, s) for n, s, *_ in ks)["db1"]
    assert L.wgsl_plan(src) == "tmpl:reduce;op=sum;axis=0;M=64;N=128;pa=mask;in_a=2;za=1"
    bad = src.replace("data1[(r1 * 128) + r0]", "data1[(r1 * 128) + ((r0 + 1) % 128)]")
    assert bad != src and L.wgsl_plan(bad) == "wave"


def test_mask_prologue_needs_the_same_index_for_z_and_the_adjoint():
    """Where(z == max(z, 0), adj, 0) is the ReLU backward only when z is read where adj is."""
    ks, _, _ = WL.mlp_ce_step(64, 784, 128, 10)
    src = dict((n, s) for n, s, *_ in ks)["dW1"]
    assert "pa=mask" in L.wgsl_template_key(src)
    bad = src.replace("let t5: f32 = data2[(r2 * 128) + r0];", "let t5: f32 = data2[(r2 * 128) + ((r0 + 1) % 128)];")
    assert bad != src
    assert L.wgsl_template_key(bad) == ""


def test_reduce_with_scale_and_scalar_output():
    """Sum over a whole 1-D buffer times a constant (a mean) is tmpl:reduce with M=1 and the scale."""
    k = WL.Kernel([(20, [1], L.AH_F32), (1, [300], L.AH_F32)], [])
    k.acc()
    r = k.loop(300)
    k.update(k.load(1, r))
    k.end()
    k.store(k.let("(acc0 * 0.5)"))
    assert L.wgsl_template_key(k.source()) == "tmpl:reduce;op=sum;axis=1;M=1;N=300;scale=0x1p-1"


def test_rendered_mlp3_step_selects_templates():
    """Config 3's rendered step: the three f16 layers select the f16 contraction template (ReLU prologue on
    the second and third); the five f32 x f16 backward contractions the f32 template with their f16
    operands and mask sources widened (wa/wb/wza); the output bias gradient the column-sum template and the
    masked ones (db2, db1) the column-sum template with the mask prologue on their f16 pre-activations;
    the loss keeps the wave rendering, the loss adjoint the thread one."""
    ks, _, _ = WL.mlp3_step(256, 128, 256, 256, 128)
    plans = {name: L.wgsl_plan(src) for name, src, *_ in ks}
    for name, src, _, _, _, plan in ks:
        assert plans[name] == plan, name
    assert [n for n, p in plans.items() if p.startswith("tmpl:gemm;dtype=f16")] == ["fc1", "fc2", "fc3"]
    assert [n for n, p in plans.items() if p.startswith("tmpl:gemm;dtype=f32")] == ["dW3", "dH2", "dW2", "dH1", "dW1"]
    assert plans["db3"].startswith("tmpl:reduce") and plans["gP"] == "thread"
    assert plans["db2"].endswith(";pa=mask;in_a=1;za=2;wza=1") and plans["db1"].endswith(";pa=mask;in_a=1;za=2;wza=1")
    assert [n for n, p in plans.items() if p == "wave"] == ["loss"]


def test_mixed_type_contraction_needs_widened_f16_loads():
    """An f32 x f16 contraction selects the f32 template only when the f16 operand is widened in the loop
    (f32(load)), as the lowering writes every f16 load inside an f32 reduce."""
    ks, _, _ = WL.mlp3_step(64, 32, 48, 40, 24)
    src = dict((n, s) for n, s, *_ in ks)["dH2"]
    assert L.wgsl_template_key(src).endswith(";wb=1")
    raw = src.replace("f32(data2[", "(data2[")
    assert raw != src and L.wgsl_template_key(raw) == ""


def test_rendered_chain_step_renders_the_movement_chain():
    """Config 5's rendered step (tests/wgsl_lower.py chain_step): every kernel parses in the lowering's
    form, the movement chain (shrink offsets, the pad's validity select with the reduce identity as fill,
    the permute's swapped indices) included; the per-row reductions take the wave rendering (their
    reduced values are elementwise chains, not plain loads), dX the thread one."""
    ks, _, _ = WL.chain_step(64, 48)
    plans = {name: L.wgsl_plan(src) for name, src, *_ in ks}
    for name, src, _, _, _, plan in ks:
        assert plans[name] == plan, name
    assert [n for n, p in plans.items() if p == "thread"] == ["dX"]
    src = dict((n, s) for n, s, *_ in ks)["max"]
    assert "select(bitcast<f32>(0xff7fffffu)" in src and "(t5 < 49)" in src
