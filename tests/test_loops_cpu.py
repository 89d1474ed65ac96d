"""Counted stablehlo.while loops unrolled at compile (the reference unrolls
short counted loops before planning, core/stablehlo_parser.mm:462-519), the
lax.scan form of the decoder stack, dynamic_slice with constant starts, and
contiguous slices of arguments planned as views.  Plans only (no device)."""

import numpy as np
import pytest

from mi355x import programs as P
from mi355x import runtime as rt

import _bytecode as Bc

INVALID_ARGUMENT = 3


@pytest.mark.parametrize("trips", [0, 1, 4, 16])
def test_counted_loop_unrolls(trips):
    plan, steps = rt.compile_check(P.counted_loop(trips))
    assert "while" not in plan
    # trips == 0 returns the argument itself: one copy step (results own memory)
    assert steps >= 1
    if trips == 0:
        assert plan.startswith("copy")
    else:
        assert "elementwise" in plan


@pytest.mark.parametrize("kw,why", [
    (dict(trips=17), "more than 16 trips"),
    (dict(trips=4, step=0), "more than 16 trips"),          # never ends
    (dict(trips=4, cond="NE", step=3), "more than 16 trips"),  # steps over the limit
])
def test_loops_beyond_the_limit_are_rejected(kw, why):
    with pytest.raises(rt.PluginError) as e:
        rt.compile_check(P.counted_loop(**kw))
    assert e.value.code == INVALID_ARGUMENT and why in str(e.value)


DATA_DEPENDENT = """module @jit_f {
  func.func public @main(%arg0: tensor<8xf32>) -> (tensor<8xf32>) {
    %0 = stablehlo.constant dense<0.000000e+00> : tensor<f32>
    %1:2 = stablehlo.while(%iterArg = %0, %iterArg_0 = %arg0) : tensor<f32>, tensor<8xf32>
    cond {
      %2 = stablehlo.constant dense<1.000000e+01> : tensor<f32>
      %3 = stablehlo.reduce(%iterArg_0 init: %iterArg) applies stablehlo.add across dimensions = [0] : (tensor<8xf32>, tensor<f32>) -> tensor<f32>
      %4 = stablehlo.compare  LT, %3, %2,  FLOAT : (tensor<f32>, tensor<f32>) -> tensor<i1>
      stablehlo.return %4 : tensor<i1>
    } do {
      %5 = stablehlo.add %iterArg_0, %iterArg_0 : tensor<8xf32>
      stablehlo.return %iterArg, %5 : tensor<f32>, tensor<8xf32>
    }
    return %1#1 : tensor<8xf32>
  }
}
"""


def test_data_dependent_loop_is_rejected():
    with pytest.raises(rt.PluginError) as e:
        rt.compile_check(DATA_DEPENDENT)
    assert e.value.code == INVALID_ARGUMENT and "does not fold to a constant" in str(e.value)


def test_counted_loop_equals_its_unrolled_form():
    """fori_loop(0, 3, x * 2 + i) plans exactly like the three bodies written
    out (x * 2 + 0, then + 1, then + 2)."""
    e = P._Body()
    t = P._t([8], "f32")
    x = "%arg0"
    for i in range(3):
        x = e.bin("add", e.bin("multiply", x, e.splat("2.000000e+00", "f32", [8]), t),
                  e.splat(f"{float(i):.6e}", "f32", [8]), t)
    unrolled = P._module("jit_loop", [t], [t], e.lines + [f"return {x} : {t}"])
    assert rt.compile_check(P.counted_loop(3)) == rt.compile_check(unrolled)


@pytest.mark.parametrize("cfg", [(2, 1, 64, 128, 2, 64, 256), (3, 2, 128, 256, 2, 128, 512),
                                 (4, 4, 2048, 2048, 16, 128, 8192)])
def test_scan_decoder_plans_like_the_inline_stack(cfg):
    """The lax.scan form (weights stacked over layers, taken by dynamic_slice
    on the counter) plans the same kernel steps as the stack written out
    layer by layer: the per-layer weight slices are views, not copies."""
    scan = rt.compile_check(P.decoder_stack_scan(*cfg))
    inline = rt.compile_check(P.decoder_stack(*cfg))
    assert scan == inline
    assert "slice [" + str(cfg[0]) not in scan[0]  # no copy of a stacked weight


@pytest.mark.parametrize("text", [P.counted_loop(5), P.decoder_stack_scan(2, 1, 64, 128, 2, 64, 256)],
                         ids=["counted_loop", "scan_decoder"])
def test_loops_through_bytecode(text):
    """The vhlo bytecode of a loop (decoded to the generic op form, with
    ^bb0 block arguments in both regions) plans like its text."""
    assert rt.compile_check(Bc.to_bytecode(text)) == rt.compile_check(text)


def _slice_program(src_shape, start, limit):
    e = P._Body()
    ts = P._t(src_shape, "f32")
    out = [b - a for a, b in zip(start, limit)]
    to = P._t(out, "f32")
    sl = e.slice("%arg0", ts, list(zip(start, limit)), to)
    y = e.un("exponential", sl, to)
    return P._module("jit_s", [ts], [to], e.lines + [f"return {y} : {to}"])


@pytest.mark.parametrize("src,start,limit,view", [
    ([4, 8, 8], [2, 0, 0], [3, 8, 8], True),    # one leading index
    ([4, 8, 8], [1, 2, 0], [2, 5, 8], True),    # rows 2..4 of matrix 1
    ([1, 4, 8], [0, 2, 0], [1, 3, 8], True),    # a leading dimension of extent 1
    ([4, 8, 8], [1, 0, 0], [3, 8, 8], True),    # two whole leading entries
    ([4, 8, 8], [1, 2, 0], [3, 4, 8], False),   # two matrices, partial rows: strided
    ([4, 8, 8], [0, 0, 2], [4, 8, 4], False),   # inner columns: strided
])
def test_contiguous_slices_of_arguments_are_views(src, start, limit, view):
    plan, _ = rt.compile_check(_slice_program(src, start, limit))
    assert ("slice" not in plan) == view, plan


def test_dynamic_slice_with_constant_starts_is_a_slice():
    """dynamic_slice with constant start indices plans like the static
    slice, with StableHLO's clamp of each start to [0, dim - size]."""
    def prog(starts):
        e = P._Body()
        ts, to = P._t([4, 8], "f32"), P._t([1, 8], "f32")
        cs = [e.const(s_, "i32") for s_ in starts]
        ti = P._t([], "i32")
        ds = e(f"stablehlo.dynamic_slice %arg0, {', '.join(cs)}, sizes = [1, 8] : ({ts}, {ti}, {ti}) -> {to}")
        y = e.un("exponential", ds, to)
        return P._module("jit_d", [ts], [to], e.lines + [f"return {y} : {to}"])
    for starts, eff in (([2, 0], [2, 0]), ([9, 3], [3, 0]), ([-5, 0], [0, 0])):
        static = _slice_program([4, 8], eff, [eff[0] + 1, 8])
        assert rt.compile_check(prog(starts)) == rt.compile_check(static), starts
