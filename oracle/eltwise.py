"""Fused elementwise oracle (test infrastructure only).

An elementwise program is a list of steps ``(op, args)`` where each arg is
either a step index (an earlier value; index 0 is the first input, inputs
occupy the first ``n_inputs`` slots) or a Python float (a scalar constant
splat).  Ops follow StableHLO names.

Rounding: every float result of a bf16 program is rounded to bf16, which is
what XLA:CPU does for bf16 ops (``src/pjrt_plugin/ops/registry.h:273-287``,
"JAX_METALLIB_BF16_STRICT_ROUNDING=1 rounds every bf16 op result, which is
what XLA:CPU does for bf16").  f32 programs are evaluated in float64 and
rounded to f32 per op.

``CHAIN6`` is the workload's 6-op chain (mul, add, exp, log1p, max, select;
the select's predicate is a compare against 0):

    a = x * 1.5; b = a + 0.5; c = exp(b); d = log1p(c); e = max(d, x)
    y = select(x > 0, e, b)
"""

import numpy as np

from .bf16 import round_bf16

CHAIN6 = [
    ("multiply", (0, 1.5)),
    ("add", (1, 0.5)),
    ("exponential", (2,)),
    ("log_plus_one", (3,)),
    ("maximum", (4, 0)),
    ("compare_GT", (0, 0.0)),
    ("select", (6, 5, 2)),
]


def _max(a, b):
    # NaN-propagating maximum with -0 < +0 (stablehlo.maximum).
    out = np.maximum(a, b)
    both_zero = (a == 0) & (b == 0)
    if np.any(both_zero):
        pos = both_zero & (~np.signbit(a) | ~np.signbit(b))
        out = np.where(pos, 0.0, out)
        out = np.where(both_zero & ~pos, -0.0, out)
    return out


def _min(a, b):
    out = np.minimum(a, b)
    both_zero = (a == 0) & (b == 0)
    if np.any(both_zero):
        neg = both_zero & (np.signbit(a) | np.signbit(b))
        out = np.where(neg, -0.0, out)
        out = np.where(both_zero & ~neg, 0.0, out)
    return out


_UNARY = {
    "exponential": np.exp,
    "log": np.log,
    "log_plus_one": np.log1p,
    "tanh": np.tanh,
    "rsqrt": lambda v: 1.0 / np.sqrt(v),
    "sqrt": np.sqrt,
    "negate": np.negative,
    "abs": np.abs,
    "logistic": lambda v: 1.0 / (1.0 + np.exp(-v)),
}
_BINARY = {
    "add": np.add,
    "subtract": np.subtract,
    "multiply": np.multiply,
    "divide": np.divide,
    "maximum": _max,
    "minimum": _min,
}
_COMPARE = {
    "GT": np.greater, "GE": np.greater_equal, "LT": np.less,
    "LE": np.less_equal, "EQ": np.equal, "NE": np.not_equal,
}


def evaluate(program, inputs, dtype="f32"):
    """Evaluate ``program`` on float32 ``inputs``; returns the last value.

    ``dtype`` is "f32" or "bf16": the rounding applied to each float result.
    Predicates (compare results) are bool arrays.
    """
    rnd = round_bf16 if dtype == "bf16" else (lambda v: np.asarray(v, dtype=np.float32))
    vals = [np.asarray(v, dtype=np.float32) for v in inputs]

    def get(a):
        return np.float64(a) if isinstance(a, float) else vals[a]

    with np.errstate(all="ignore"):
        for op, args in program:
            if op in _UNARY:
                v = rnd(_UNARY[op](get(args[0]).astype(np.float64)))
            elif op in _BINARY:
                v = rnd(_BINARY[op](np.asarray(get(args[0]), np.float64),
                                    np.asarray(get(args[1]), np.float64)))
            elif op.startswith("compare_"):
                v = _COMPARE[op[8:]](get(args[0]), get(args[1]))
            elif op == "select":
                v = np.where(get(args[0]), get(args[1]), get(args[2])).astype(np.float32)
            else:
                raise ValueError(f"unknown elementwise op {op}")
            vals.append(v)
    return vals[-1]
