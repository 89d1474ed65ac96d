"""Host-side tests of the plugin runtime (no GPU): the StableHLO reader, the
planner's kernel routing, compile-time rejection of unsupported programs,
and the event/error object model.

The compile path mirrors the reference's PJRT_Client_Compile: unsupported
ops fail at compile with a message listing them
(src/pjrt_plugin/api/pjrt_client.cc:211-220); events follow
src/pjrt_plugin/api/pjrt_event.cc (error before ready is
FAILED_PRECONDITION, :32-44; on_ready runs inline when already ready,
:81-98) and the await timeout of core/completion_event.h.
"""

import re

import pytest

from mi355x import programs as P
from mi355x import runtime as rt


def plan(text):
    t, n = rt.compile_check(text)
    steps = [l for l in t.strip().splitlines() if l]
    assert len(steps) == n
    return steps


# Every workload function of the benchmark plans to exactly one kernel step
# at its full size.
@pytest.mark.parametrize("text,step", [
    (P.int4_g64_matmul(16, 4096, 14336), "int4_g64_matmul M=16 K=4096 N=14336 -> bf16"),
    (P.int4_g64_matmul(1, 4096, 14336), "int4_g64_matmul M=1 K=4096 N=14336 -> bf16"),
    (P.int8_pc_matmul(16, 4096, 14336), "int8_pc_matmul M=16 K=4096 N=14336 -> bf16"),
    (P.matmul(4096, 4096, 4096), "gemm_bf16 batch=1 M=4096 N=4096 K=4096 -> bf16"),
    (P.matmul(4096, 4096, 4096, preferred_f32=True), "gemm_bf16 batch=1 M=4096 N=4096 K=4096 -> f32"),
    (P.matmul(2048, 128, 2048, batch=16), "gemm_bf16 batch=16 M=2048 N=2048 K=128 -> bf16"),
    (P.matmul(2048, 2048, 2048, dt="f32"), "gemm_f32 batch=1 M=2048 N=2048 K=2048 -> f32"),
    (P.softmax(8192, 8192), "softmax rows=8192 cols=8192 f32"),
    (P.softmax(8192, 8192, "bf16"), "softmax rows=8192 cols=8192 bf16"),
    (P.rmsnorm(8192, 8192), "rmsnorm rows=8192 cols=8192 eps=1e-06 f32"),
    (P.argmax(8192, 8192), "argmax rows=8192 cols=8192 f32 -> i32"),
    (P.argmax(8192, 8192, "bf16"), "argmax rows=8192 cols=8192 bf16 -> i32"),
    (P.reduce(8192, 8192, "sum"), "reduce_sum rows=8192 cols=8192 f32"),
    (P.reduce(8192, 8192, "sum", "bf16"), "reduce_sum rows=8192 cols=8192 bf16"),
    (P.reduce(8192, 8192, "max", "bf16"), "reduce_max rows=8192 cols=8192 bf16"),
    (P.chain6(8192, 8192), "elementwise 11 instr, 1 inputs, n=67108864 f32"),
    (P.chain6(8192, 8192, "bf16"), "elementwise 11 instr, 1 inputs, n=67108864 bf16"),
])
def test_workload_plans_to_one_kernel(text, step):
    assert plan(text) == [step]


def test_rmsnorm_bf16_keeps_the_bf16_epsilon():
    # 1e-6 printed as a bf16 constant is the bf16 value nearest 1e-6.
    (s,) = plan(P.rmsnorm(64, 128, "bf16"))
    eps = float(re.search(r"eps=([0-9.e+-]+)", s).group(1))
    assert s.startswith("rmsnorm rows=64 cols=128") and s.endswith("bf16")
    assert abs(eps - 9.98377799987793e-07) < 1e-12


def test_plumbing_chain_plans_three_steps():
    assert plan(P.plumbing()) == [
        "gemm_f32 batch=1 M=1024 N=1024 K=1024 -> f32",
        "elementwise 2 instr, 1 inputs, n=1048576 f32",
        "reduce_sum rows=1024 cols=1024 f32",
    ]


def _wrap(args, rets, body):
    a = ", ".join(f"%arg{i}: {t}" for i, t in enumerate(args))
    r = ", ".join(rets)
    return ("module @jit_f {\n  func.func public @main(" + a + ") -> (" + r + ") {\n" +
            "".join("    " + l + "\n" for l in body) + "  }\n}\n")


def test_private_function_is_inlined():
    inner = P.softmax(8, 16).replace("func.func public @main", "func.func private @_softmax")
    inner = inner.split("\n", 1)[1].rsplit("}", 1)[0]  # the func.func only
    text = ("module @jit_f {\n  func.func public @main(%arg0: tensor<8x16xf32>) -> (tensor<8x16xf32>) {\n"
            "    %0 = call @_softmax(%arg0) : (tensor<8x16xf32>) -> tensor<8x16xf32>\n"
            "    return %0 : tensor<8x16xf32>\n  }\n" + inner + "}\n")
    assert plan(text) == ["softmax rows=8 cols=16 f32"]


GENERIC_ARGMAX = """module @jit_argmax {
  func.func public @main(%arg0: tensor<4x8xf32>) -> tensor<4xi32> {
    %0 = "stablehlo.iota"() {iota_dimension = 1 : i64} : () -> tensor<4x8xi32>
    %1 = "stablehlo.constant"() {value = dense<0xFF800000> : tensor<f32>} : () -> tensor<f32>
    %2 = "stablehlo.constant"() {value = dense<0> : tensor<i32>} : () -> tensor<i32>
    %3:2 = "stablehlo.reduce"(%arg0, %0, %1, %2) ({
    ^bb0(%a: tensor<f32>, %b: tensor<i32>, %c: tensor<f32>, %d: tensor<i32>):
      %4 = "stablehlo.compare"(%a, %c) {comparison_direction = #stablehlo<comparison_direction GT>} : (tensor<f32>, tensor<f32>) -> tensor<i1>
      %5 = "stablehlo.compare"(%a, %a) {comparison_direction = #stablehlo<comparison_direction NE>} : (tensor<f32>, tensor<f32>) -> tensor<i1>
      %6 = "stablehlo.or"(%4, %5) : (tensor<i1>, tensor<i1>) -> tensor<i1>
      %7 = "stablehlo.select"(%6, %a, %c) : (tensor<i1>, tensor<f32>, tensor<f32>) -> tensor<f32>
      %8 = "stablehlo.select"(%6, %b, %d) : (tensor<i1>, tensor<i32>, tensor<i32>) -> tensor<i32>
      "stablehlo.return"(%7, %8) : (tensor<f32>, tensor<i32>) -> ()
    }) {dimensions = array<i64: 1>} : (tensor<4x8xf32>, tensor<4x8xi32>, tensor<f32>, tensor<i32>) -> (tensor<4xf32>, tensor<4xi32>)
    "func.return"(%3#1) : (tensor<4xi32>) -> ()
  }
}
"""


def test_generic_form_argmax():
    assert plan(GENERIC_ARGMAX) == ["argmax rows=4 cols=8 f32 -> i32"]


def test_generic_form_reduce_and_broadcast():
    text = _wrap(["tensor<4x8xf32>"], ["tensor<4xf32>"], [
        '%0 = "stablehlo.constant"() {value = dense<0.000000e+00> : tensor<f32>} : () -> tensor<f32>',
        '%1 = "stablehlo.reduce"(%arg0, %0) ({',
        '^bb0(%a: tensor<f32>, %b: tensor<f32>):',
        '  %2 = "stablehlo.add"(%a, %b) : (tensor<f32>, tensor<f32>) -> tensor<f32>',
        '  "stablehlo.return"(%2) : (tensor<f32>) -> ()',
        '}) {dimensions = array<i64: 1>} : (tensor<4x8xf32>, tensor<f32>) -> tensor<4xf32>',
        '"func.return"(%1) : (tensor<4xf32>) -> ()',
    ])
    assert plan(text) == ["reduce_sum rows=4 cols=8 f32"]


def test_returning_an_argument_copies_it():
    text = _wrap(["tensor<4x8xf32>"], ["tensor<4x8xf32>", "tensor<4x8xf32>"], [
        "%0 = stablehlo.exponential %arg0 : tensor<4x8xf32>",
        "return %arg0, %0 : tensor<4x8xf32>, tensor<4x8xf32>",
    ])
    assert plan(text) == ["copy tensor<4x8xf32>", "elementwise 2 instr, 1 inputs, n=32 f32"]


def test_same_value_returned_twice_gets_two_buffers():
    text = _wrap(["tensor<4x8xf32>"], ["tensor<4x8xf32>", "tensor<4x8xf32>"], [
        "%0 = stablehlo.tanh %arg0 : tensor<4x8xf32>",
        "return %0, %0 : tensor<4x8xf32>, tensor<4x8xf32>",
    ])
    assert plan(text) == ["elementwise 2 instr, 1 inputs, n=32 f32", "copy tensor<4x8xf32>"]


def test_reshape_is_a_view():
    text = _wrap(["tensor<4x8xf32>"], ["tensor<32xf32>"], [
        "%0 = stablehlo.reshape %arg0 : (tensor<4x8xf32>) -> tensor<32xf32>",
        "%1 = stablehlo.negate %0 : tensor<32xf32>",
        "%2 = stablehlo.reshape %1 : (tensor<32xf32>) -> tensor<4x8xf32>",
        "%3 = stablehlo.reshape %2 : (tensor<4x8xf32>) -> tensor<32xf32>",
        "return %3 : tensor<32xf32>",
    ])
    assert plan(text) == ["elementwise 2 instr, 1 inputs, n=32 f32"]


def test_long_elementwise_chain_is_split():
    body = ["%0 = stablehlo.tanh %arg0 : tensor<64xf32>"]
    for i in range(1, 50):
        body.append(f"%{i} = stablehlo.add %{i - 1}, %arg{i % 3} : tensor<64xf32>")
    body.append("return %49 : tensor<64xf32>")
    steps = plan(_wrap(["tensor<64xf32>"] * 3, ["tensor<64xf32>"], body))
    assert len(steps) >= 2
    assert all(s.startswith("elementwise") for s in steps)
    assert all(int(re.search(r"(\d+) instr", s).group(1)) <= 32 for s in steps)


def test_five_inputs_are_split_to_four_per_program():
    body = ["%0 = stablehlo.add %arg0, %arg1 : tensor<64xf32>"]
    for i in range(2, 5):
        body.append(f"%{i - 1} = stablehlo.multiply %{i - 2}, %arg{i} : tensor<64xf32>")
    body.append("return %3 : tensor<64xf32>")
    steps = plan(_wrap(["tensor<64xf32>"] * 5, ["tensor<64xf32>"], body))
    assert len(steps) == 2
    assert all(int(re.search(r"(\d+) inputs", s).group(1)) <= 4 for s in steps)


def test_bf16_typed_node_in_f32_program_rounds():
    # x.astype(bf16).astype(f32) * 2 rounds once to bf16 inside an f32
    # program: load, round, constant, multiply (3 without the rounding).
    text = _wrap(["tensor<64xf32>"], ["tensor<64xf32>"], [
        "%0 = stablehlo.convert %arg0 : (tensor<64xf32>) -> tensor<64xbf16>",
        "%1 = stablehlo.convert %0 : (tensor<64xbf16>) -> tensor<64xf32>",
        "%cst = stablehlo.constant dense<2.000000e+00> : tensor<f32>",
        "%2 = stablehlo.broadcast_in_dim %cst, dims = [] : (tensor<f32>) -> tensor<64xf32>",
        "%3 = stablehlo.multiply %1, %2 : tensor<64xf32>",
        "return %3 : tensor<64xf32>",
    ])
    assert plan(text) == ["elementwise 4 instr, 1 inputs, n=64 f32"]


def _unsupported(text):
    with pytest.raises(rt.PluginError) as ei:
        rt.compile_check(text)
    assert ei.value.code == rt.UNIMPLEMENTED, ei.value
    return ei.value.message


def test_unsupported_ops_fail_at_compile_with_a_list():
    text = _wrap(["tensor<4x8xf32>", "tensor<8x4xf32>"], ["tensor<8x4xf32>", "tensor<4x8xf32>"], [
        "%0 = stablehlo.remainder %arg1, %arg1 : tensor<8x4xf32>",
        "%1 = stablehlo.cosine %arg1 : tensor<8x4xf32>",
        "%2 = stablehlo.add %0, %1 : tensor<8x4xf32>",
        "%3 = stablehlo.sine %arg0 : tensor<4x8xf32>",
        "return %2, %3 : tensor<8x4xf32>, tensor<4x8xf32>",
    ])
    msg = _unsupported(text)
    for op in ("stablehlo.remainder", "stablehlo.cosine", "stablehlo.sine"):
        assert op in msg, msg


def test_non_canonical_dot_takes_the_general_kernel():
    # x @ w.T as a contraction over both last dims: not the [M,K] x [K,N]
    # form, so the strided general kernel reads w in place.
    text = _wrap(["tensor<16x64xbf16>", "tensor<32x64xbf16>"], ["tensor<16x32xbf16>"], [
        "%0 = stablehlo.dot_general %arg0, %arg1, contracting_dims = [1] x [1] : "
        "(tensor<16x64xbf16>, tensor<32x64xbf16>) -> tensor<16x32xbf16>",
        "return %0 : tensor<16x32xbf16>",
    ])
    plan, n = rt.compile_check(text)
    assert plan.strip() == "dot_general bf16 batch=1 M=16 N=32 K=64 -> bf16" and n == 1


def test_several_contracting_dims_plan():
    """Contracting dims that collapse by strides need no copy; others are
    copied to [batch, K, N] / [batch, M, K] first; none at all is K = 1."""
    text = _wrap(["tensor<4x8x8xf32>", "tensor<8x8x3xf32>"], ["tensor<4x3xf32>"], [
        "%0 = stablehlo.dot_general %arg0, %arg1, contracting_dims = [1, 2] x [0, 1] : "
        "(tensor<4x8x8xf32>, tensor<8x8x3xf32>) -> tensor<4x3xf32>",
        "return %0 : tensor<4x3xf32>",
    ])
    assert plan(text) == ["dot_general f32 batch=1 M=4 N=3 K=64 -> f32"]
    assert plan(P.dot_general_dims((4, 6, 8), (8, 6, 5), "float32", (1, 2), (1, 0))) == [
        "dot operand b to [6,8,5]", "dot_general f32 batch=1 M=4 N=5 K=48 (strided) -> f32"]
    assert plan(P.dot_general_dims((3, 4), (5, 6), "float32", (), ())) == [
        "dot_general f32 batch=1 M=12 N=30 K=1 -> f32"]
    # batch dims not leading: (a3, a0) x (b0, b1), result [2, 5, 7, 9]
    assert plan(P.dot_general_dims((5, 7, 3, 2), (2, 5, 3, 9), "float32", (2,), (2,), (3, 0), (0, 1))) == [
        "dot operand a to [2,5,7,3]", "dot_general f32 batch=10 M=7 N=9 K=3 (strided) -> f32"]
    # large enough for the tiled GEMM: K = 32 x 16 collapses in place
    assert plan(P.dot_general_dims((64, 32, 16), (32, 16, 128), "bfloat16", (1, 2), (0, 1))) == [
        "gemm_bf16 batch=1 M=64 N=128 K=512 -> bf16"]


def test_rhs_contracting_last_plans_the_nt_gemm(monkeypatch):
    """x @ W.T and q @ k^T (rhs contracting its last dim) read the rhs in
    place on 256-aligned bf16 shapes; other shapes, f32 and
    MK_PLAN_GEMM_NT=0 copy it to [batch, K, N] first."""
    assert plan(P.dot_general_dims((512, 256), (768, 256), "bfloat16", (1,), (1,))) == [
        "gemm_bf16_nt batch=1 M=512 N=768 K=256 -> bf16"]
    assert plan(P.dot_general_dims((2, 256, 64), (2, 512, 64), "bfloat16", (2,), (2,), (0,), (0,))) == [
        "gemm_bf16_nt batch=2 M=256 N=512 K=64 -> bf16"]
    assert plan(P.dot_general_dims((500, 256), (768, 256), "bfloat16", (1,), (1,))) == [
        "gemm operand b to [1,256,768]", "gemm_bf16 batch=1 M=500 N=768 K=256 -> bf16"]
    assert plan(P.dot_general_dims((512, 256), (768, 256), "float32", (1,), (1,))) == [
        "gemm operand b to [1,256,768]", "gemm_f32 batch=1 M=512 N=768 K=256 -> f32"]
    monkeypatch.setenv("MK_PLAN_GEMM_NT", "0")
    assert plan(P.dot_general_dims((512, 256), (768, 256), "bfloat16", (1,), (1,))) == [
        "gemm operand b to [1,256,768]", "gemm_bf16 batch=1 M=512 N=768 K=256 -> bf16"]


def test_dot_with_mismatched_dimension_sizes_is_rejected():
    text = _wrap(["tensor<4x8x8xf32>", "tensor<8x6x3xf32>"], ["tensor<4x3xf32>"], [
        "%0 = stablehlo.dot_general %arg0, %arg1, contracting_dims = [1, 2] x [0, 1] : "
        "(tensor<4x8x8xf32>, tensor<8x6x3xf32>) -> tensor<4x3xf32>",
        "return %0 : tensor<4x3xf32>",
    ])
    assert "stablehlo.dot_general" in _unsupported(text)


def test_unaligned_gemm_takes_the_general_kernel():
    plan, _ = rt.compile_check(P.matmul(16, 60, 32))
    assert plan.strip() == "dot_general bf16 batch=1 M=16 N=32 K=60 -> bf16"


def test_broken_softmax_is_not_fused():
    # The max is taken over another tensor: not a softmax.  It runs op by
    # op: the reductions, the row broadcasts as layout copies, elementwise.
    text = P.softmax(8, 16).replace(
        "%0 = stablehlo.reduce(%arg0 init: %cst)", "%0 = stablehlo.reduce(%arg1 init: %cst)").replace(
        "@main(%arg0: tensor<8x16xf32>)", "@main(%arg0: tensor<8x16xf32>, %arg1: tensor<8x16xf32>)")
    steps = plan(text)
    assert not any(s.startswith("softmax") for s in steps), steps
    assert "reduce_max rows=8 cols=16 f32" in steps and "reduce_sum rows=8 cols=16 f32" in steps
    assert any(s.startswith("broadcast [8,1] -> f32 [8,16]") for s in steps), steps


def test_f32_arithmetic_inside_a_bf16_program():
    # (x.astype(f32) * y + 1).astype(bf16), y f32: one bf16 program that
    # loads y as f32, keeps the product and sum in f32 and rounds once.
    text = _wrap(["tensor<64xbf16>", "tensor<64xf32>"], ["tensor<64xbf16>"], [
        "%0 = stablehlo.convert %arg0 : (tensor<64xbf16>) -> tensor<64xf32>",
        "%1 = stablehlo.multiply %0, %arg1 : tensor<64xf32>",
        "%cst = stablehlo.constant dense<1.000000e+00> : tensor<f32>",
        "%2 = stablehlo.broadcast_in_dim %cst, dims = [] : (tensor<f32>) -> tensor<64xf32>",
        "%3 = stablehlo.add %1, %2 : tensor<64xf32>",
        "%4 = stablehlo.convert %3 : (tensor<64xf32>) -> tensor<64xbf16>",
        "return %4 : tensor<64xbf16>",
    ])
    assert plan(text) == ["elementwise 6 instr, 2 inputs, n=64 bf16"]


def test_residual_add_keeps_the_dequant_matmul():
    # x + int4mm(h): the elementwise add loads the matmul's bf16 output; it
    # does not pull the matmul's f32 product into its program.
    t = P.int4_g64_matmul(16, 128, 256)
    t = t.replace("-> (tensor<16x256xbf16>", "-> (tensor<16x256xbf16>").replace(
        "    return %21 : tensor<16x256xbf16>",
        "    %22 = stablehlo.add %21, %21 : tensor<16x256xbf16>\n    return %22 : tensor<16x256xbf16>")
    assert plan(t) == ["int4_g64_matmul M=16 K=128 N=256 -> bf16", "elementwise 2 instr, 1 inputs, n=4096 bf16"]


@pytest.mark.parametrize("fmt", ["int4", "int8"])
def test_residual_and_swiglu_fold_into_the_dequant_matmul(fmt, monkeypatch):
    name = "int4_g64_matmul" if fmt == "int4" else "int8_pc_matmul"
    assert plan(P.qmm_epilogue(256, 128, 256, fmt, "add")) == [f"{name} M=256 K=128 N=256 -> bf16 + add epilogue"]
    assert plan(P.qmm_epilogue(256, 128, 256, fmt, "swiglu")) == [f"{name} M=256 K=128 N=256 -> bf16",
                                                                   "elementwise 5 instr, 2 inputs, n=65536 bf16"]
    monkeypatch.setenv("MK_PLAN_EPILOGUES", "all")
    assert plan(P.qmm_epilogue(256, 128, 256, fmt, "swiglu")) == [f"{name} M=256 K=128 N=256 -> bf16 + swiglu epilogue"]
    monkeypatch.setenv("MK_PLAN_EPILOGUES", "0")
    assert plan(P.qmm_epilogue(256, 128, 256, fmt, "add")) == [f"{name} M=256 K=128 N=256 -> bf16",
                                               "elementwise 3 instr, 2 inputs, n=65536 bf16"]


@pytest.mark.parametrize("fmt", ["int4", "int8"])
def test_swiglu_pair_plans_one_step_on_the_many_row_route(fmt, monkeypatch):
    name = "int4_g64" if fmt == "int4" else "int8_pc"
    assert plan(P.swiglu_mlp(1024, 256, 512, fmt)) == [f"{name} swiglu pair matmul M=1024 K=256 N=512 -> bf16"]
    # below the dequantise-then-GEMM route (and with pairing off) the two
    # products and the SwiGLU program stay apart
    mm = "int4_g64_matmul" if fmt == "int4" else "int8_pc_matmul"
    apart = [f"{mm} M=256 K=256 N=512 -> bf16"] * 2 + ["elementwise 5 instr, 2 inputs, n=131072 bf16"]
    assert plan(P.swiglu_mlp(256, 256, 512, fmt)) == apart
    monkeypatch.setenv("MK_PLAN_PAIRS", "0")
    assert plan(P.swiglu_mlp(1024, 256, 512, fmt)) == [s.replace("M=256", "M=1024").replace("131072", "524288")
                                                       for s in apart]


def test_decoder_layer_pairs_gate_and_up_at_many_rows():
    steps = plan(P.decoder_layer(4, 256, 256, 2, 128, 512))
    assert "int4_g64 swiglu pair matmul M=1024 K=256 N=512 -> bf16" in steps
    assert not any(s.startswith("elementwise") for s in steps) and len(steps) == 8


def test_decoder_layer_plans_onto_the_kernels():
    """The Llama layer's StableHLO: projections on the dequant-matmul, norms
    and softmax on their row kernels, the two attention products on the bf16
    GEMM, everything else as layout copies and elementwise programs."""
    steps = plan(P.decoder_layer(2, 64, 128, 2, 64, 256))
    kinds = [s.split()[0] for s in steps]
    assert kinds.count("int4_g64_matmul") == 5 and kinds.count("rmsnorm") == 2
    assert kinds.count("softmax") == 1 and kinds.count("gemm_bf16") == 2
    assert set(kinds) <= {"int4_g64_matmul", "rmsnorm", "softmax", "gemm_bf16", "gemm", "dot", "elementwise", "slice",
                          "broadcast", "concatenate", "transpose"}, set(kinds)
    assert "softmax rows=256 cols=64 bf16" in steps
    # the causal mask is folded at compile time into the select's program
    assert not any(s.startswith("iota") for s in steps)


def test_decoder_layer_routes_rope_and_attention_to_the_decoder_kernels(monkeypatch):
    """With head_dim 128 and S % 128 == 0 the RoPE chain becomes one
    rope/split step and the masked-softmax attention one fused step writing
    the merged [B, S, H, D] layout; MK_PLAN_DECODER_FUSION=0 keeps the
    op-by-op plan."""
    text = P.decoder_layer(2, 128, 256, 2, 128, 512)
    assert plan(text) == [
        "rmsnorm rows=256 cols=256 eps=9.98378e-07 bf16",
        "int4_g64_matmul M=256 K=256 N=768 -> bf16",
        "rope_qkv_split B=2 S=128 H=2 D=128 bf16",
        "attention_causal B=2 H=2 S=128 D=128 scale=0.0883789 bf16",
        "int4_g64_matmul M=256 K=256 N=256 -> bf16 + add epilogue",
        "rmsnorm rows=256 cols=256 eps=9.98378e-07 bf16",
        "int4_g64_matmul M=256 K=256 N=512 -> bf16",
        "int4_g64_matmul M=256 K=256 N=512 -> bf16",
        "elementwise 5 instr, 2 inputs, n=131072 bf16",
        "int4_g64_matmul M=256 K=512 N=256 -> bf16 + add epilogue",
    ]
    monkeypatch.setenv("MK_PLAN_EPILOGUES", "all")
    assert plan(text)[7] == "int4_g64_matmul M=256 K=256 N=512 -> bf16 + swiglu epilogue"
    monkeypatch.setenv("MK_PLAN_EPILOGUES", "0")
    steps = plan(text)
    assert not any("epilogue" in s for s in steps) and len(steps) == 12
    monkeypatch.setenv("MK_PLAN_DECODER_FUSION", "0")
    kinds = [s.split()[0] for s in plan(text)]
    assert "attention_causal" not in kinds and "rope_qkv_split" not in kinds
    assert kinds.count("softmax") == 1 and kinds.count("gemm_bf16") == 2


def test_attention_route_needs_a_positive_scale():
    text = P.causal_attention(1, 2, 128, 128)
    const = f"{128 ** -0.5:.6e}"
    assert const in text
    neg = text.replace(const, f"{-(128 ** -0.5):.6e}")
    steps = plan(neg)
    assert not any(s.startswith("attention_causal") for s in steps) and any(s.startswith("softmax") for s in steps)


def test_attention_route_needs_the_causal_mask():
    want = ["attention_causal B=1 H=2 S=128 D=128 scale=0.0883789 bf16"]
    assert plan(P.causal_attention(1, 2, 128, 128)) == want
    # k contracted on its last axis (einsum 'bhqd,bhkd->bhqk'), no transpose
    assert plan(P.causal_attention(1, 2, 128, 128, transpose_k=False)) == want
    # an anti-causal or strict mask is not this kernel's: op by op
    for op in ("LE", "GT"):
        steps = plan(P.causal_attention(1, 2, 128, 128, mask=op))
        assert not any(s.startswith("attention_causal") for s in steps), (op, steps)
        assert any(s.startswith("softmax") for s in steps)


def test_argmax_values_result_is_rejected():
    text = P.argmax(4, 8).replace("return %1#1 : tensor<4xi32>", "return %1#0 : tensor<4xf32>").replace(
        "-> (tensor<4xi32> {", "-> (tensor<4xf32> {")
    assert "argmax" in _unsupported(text)


@pytest.mark.parametrize("text", [
    "this is not stablehlo",
    "module @m {\n  func.func public @main(%arg0: tensor<4xf32>) -> tensor<4xf32> {\n"
    "    %0 = stablehlo.add %arg0, %undefined : tensor<4xf32>\n    return %0 : tensor<4xf32>\n  }\n}\n",
    "module @m {\n  func.func public @main(%arg0: tensor<4xq7>) -> tensor<4xf32> {\n"
    "    return %arg0 : tensor<4xf32>\n  }\n}\n",
])
def test_malformed_text_is_invalid_argument(text):
    with pytest.raises(rt.PluginError) as ei:
        rt.compile_check(text)
    assert ei.value.code == rt.INVALID_ARGUMENT


def test_truncated_bytecode_is_invalid_argument():
    # The bytecode magic routes to the MLIR-bytecode reader (tests in
    # test_bytecode_cpu.py); a file cut inside its version is malformed.
    with pytest.raises(rt.PluginError) as ei:
        rt.compile_check(b"ML\xefR\x00\x01\x02")
    assert ei.value.code == rt.INVALID_ARGUMENT
    assert "bytecode" in ei.value.message


def test_client_without_device_is_unavailable():
    try:
        c = rt.Client()
    except rt.PluginError as e:
        assert e.code == rt.UNAVAILABLE
        return
    c.close()
    pytest.skip("a HIP device is visible")


def test_event_lifecycle():
    e = rt.Event.create()
    assert not e.is_ready()
    with pytest.raises(rt.PluginError) as ei:
        e.error()
    assert ei.value.code == rt.FAILED_PRECONDITION
    with pytest.raises(rt.PluginError) as ei:
        e.wait(20)
    assert ei.value.code == rt.DEADLINE_EXCEEDED
    seen = []
    e.on_ready(seen.append)
    assert seen == []
    e.set()
    assert seen == [None] and e.is_ready()
    e.error()
    e.wait(0)
    late = []
    e.on_ready(late.append)  # already ready: runs inline
    assert late == [None]


def test_event_error_reaches_waiters_and_callbacks():
    e = rt.Event.create()
    seen = []
    e.on_ready(seen.append)
    e.set(rt.INTERNAL, "device lost")
    assert seen[0].code == rt.INTERNAL and seen[0].message == "device lost"
    for call in (lambda: e.wait(10), e.error):
        with pytest.raises(rt.PluginError) as ei:
            call()
        assert ei.value.code == rt.INTERNAL and ei.value.message == "device lost"


def test_event_timeout_from_environment(monkeypatch):
    monkeypatch.setenv("MK_COMPLETION_TIMEOUT_MS", "30")
    e = rt.Event.create()
    with pytest.raises(rt.PluginError) as ei:
        e.wait()  # negative timeout: the environment value
    assert ei.value.code == rt.DEADLINE_EXCEEDED
    assert "30 ms" in ei.value.message


def test_interleave_gate_up_column_map():
    """Column 32q + c of the interleaved weight is gate column 16q + c and
    column 32q + 16 + c is up column 16q + c, for every per-column array."""
    import torch
    from mi355x import ops
    g = torch.arange(3 * 64, dtype=torch.int32).reshape(3, 64)
    u = -1 - g
    w = ops.interleave_gate_up(g, u)
    assert w.shape == (3, 128)
    for q in range(4):
        assert torch.equal(w[:, 32 * q:32 * q + 16], g[:, 16 * q:16 * q + 16])
        assert torch.equal(w[:, 32 * q + 16:32 * q + 32], u[:, 16 * q:16 * q + 16])


@pytest.mark.parametrize("args,kw,expect", [
    (((5, 7), (7, 3), "int8"), {}, "dot_general i8 batch=1 M=5 N=3 K=7 -> i8"),
    (((7,), (7, 3), "int16"), {}, "dot_general i16 batch=1 M=1 N=3 K=7 -> i16"),
    (((2, 3, 4, 5), (2, 3, 5, 6), "uint32"), {"batch": 2}, "dot_general ui32 batch=6 M=4 N=6 K=5 -> ui32"),
    (((5, 7), None, "int8"), {"self_transpose": True}, "dot_general i8 batch=1 M=5 N=5 K=7 (strided) -> i8"),
    (((5, 7), (7, 3), "int8"), {"out_dt": "int32"}, "dot_general i8 batch=1 M=5 N=3 K=7 -> i32"),
    (((4, 1), (1, 3), "float32"), {}, "dot_general f32 batch=1 M=4 N=3 K=1 -> f32"),
    (((64, 64), (64, 64), "bfloat16"), {}, "gemm_bf16 batch=1 M=64 N=64 K=64 -> bf16"),
    (((6, 0), (0, 3), "float32"), {}, "zero tensor<6x3xf32> (empty contraction)"),
])
def test_dot_general_routes(args, kw, expect):
    """Integer dots, K = 1, K or N off the multiple of 8, vectors and
    transposed operands take the general dot_general kernel; canonical
    bf16 / f32 shapes keep the tiled GEMMs (the reference's routing of
    HandleDotGeneral, src/pjrt_plugin/ops/binary_ops.mm:644-1100)."""
    from mi355x import programs as P
    plan, n = rt.compile_check(P.dot_general(*args, **kw))
    assert plan.strip() == expect and n == 1, plan


@pytest.mark.parametrize("args,expect", [
    (((8, 16), 1, "min"), ["reduce_min rows=8 cols=16 f32"]),
    (((4, 5, 6), 2, "sum"), ["reduce_sum rows=4 cols=30 f32"]),
    (((4, 5, 6), 2, "max", "bf16"), ["reduce_max rows=4 cols=30 bf16"]),
    (((8, 16), 1, "mean"), ["reduce_sum rows=8 cols=16 f32", "elementwise 3 instr, 1 inputs, n=8 f32"]),
    (((8, 16), 1, "sum", "f32", 2.5), ["reduce_sum rows=8 cols=16 f32",
                                       "elementwise 3 instr, 1 inputs, n=8 f32 (reduce init)"]),
])
def test_reduce_routes(args, expect):
    """min, several trailing axes, mean (sum then an elementwise divide) and a
    non-neutral init (combined once after the reduction, as the reference's
    mps_executable.mm:955-975 does)."""
    assert plan(P.reduce_trailing(*args)) == expect
