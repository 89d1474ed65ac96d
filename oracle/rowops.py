"""Row (last-axis) reduction oracles (test infrastructure only).

softmax   jax.nn.softmax: exp(x - max) / sum(exp(x - max)); the reference
          matches reduce_max -> sub -> exp -> reduce_sum -> div
          (``src/pjrt_plugin/core/mps_executable.mm:1922-2089``).  A row whose
          max is NaN or +-inf gives an all-NaN row (inf - inf = NaN), the
          behaviour ``tests/test_native_softmax.py:26-35`` pins.  For bf16 the
          XLA:CPU rounding points are restated after the reference's f16
          emulation (``src/pjrt_plugin/runtime/metal_kernels.mm:1742-1819``):
          d = r(x - m), e = r(exp d), s = r(sum_f32 e), y = r(e / s).
rmsnorm   x * rsqrt(mean(x^2) + eps) * g (the workload's definition; the
          reference has no RMSNorm fusion, its nearest is LayerNorm at
          ``mps_executable.mm:1457-1820``).
argmax    index of the first NaN in the row, else of the first maximum, with
          -0 == +0 (``src/pjrt_plugin/ops/reduction_ops.mm:1478-1536``;
          ``tests/test_argreduce_nan.py:8-11``).  int32 output.
reduce    sum (float64 accumulate) and max (NaN propagates; -0 < +0, the
          reference's order key, ``runtime/metal_kernels.mm:830-857``).
"""

import numpy as np

from .bf16 import bf16_bits_to_f32, f32_to_bf16_bits, round_bf16


def softmax(x):
    """float64 softmax over the last axis of a float array."""
    x = np.asarray(x, dtype=np.float64)
    with np.errstate(invalid="ignore", over="ignore"):
        m = np.max(x, axis=-1, keepdims=True)
        e = np.exp(x - m)
        return e / np.sum(e, axis=-1, keepdims=True)


def softmax_bf16(x_bits):
    """bf16 softmax with XLA:CPU's per-op rounding points -> bf16 bits."""
    x = bf16_bits_to_f32(x_bits)
    with np.errstate(invalid="ignore", over="ignore"):
        m = np.max(x, axis=-1, keepdims=True)
        d = round_bf16(x - m)
        e = round_bf16(np.exp(d))
        s = round_bf16(np.sum(e.astype(np.float32), axis=-1, keepdims=True, dtype=np.float32))
        y = round_bf16(e / s)
    return f32_to_bf16_bits(y)


def rmsnorm(x, g, eps=1e-6):
    """float64 RMSNorm over the last axis."""
    x = np.asarray(x, dtype=np.float64)
    g = np.asarray(g, dtype=np.float64)
    ms = np.mean(x * x, axis=-1, keepdims=True)
    return x / np.sqrt(ms + eps) * g


def argmax(x):
    """First-NaN-else-first-max index along the last axis (int32).

    Works for float and integer arrays.  -0.0 and +0.0 compare equal, so the
    earlier one wins a tie.
    """
    x = np.asarray(x)
    if np.issubdtype(x.dtype, np.floating):
        nan = np.isnan(x)
        has_nan = nan.any(axis=-1)
        first_nan = np.argmax(nan, axis=-1)
        filled = np.where(nan, -np.inf, x)
        # np.argmax returns the first occurrence and treats -0 == +0.
        first_max = np.argmax(filled, axis=-1)
        return np.where(has_nan, first_nan, first_max).astype(np.int32)
    return np.argmax(x, axis=-1).astype(np.int32)


def reduce_sum(x):
    """float64 sum over the last axis."""
    return np.sum(np.asarray(x, dtype=np.float64), axis=-1)


def reduce_max(x):
    """NaN-propagating max over the last axis with -0 < +0."""
    x = np.asarray(x, dtype=np.float64)
    with np.errstate(invalid="ignore"):
        m = np.max(x, axis=-1)
    # np.max keeps whichever zero it met first; XLA's order puts +0 above -0.
    zero_row = (m == 0)
    if zero_row.any():
        pos = np.any((x == 0) & ~np.signbit(x), axis=-1)
        m = np.where(zero_row & pos, 0.0, m)
        m = np.where(zero_row & ~pos, -0.0, m)
    return m


def brute_argmax_row(row):
    """Pure-Python loop argmax for one row (a pin for ``argmax``)."""
    best = None
    for i, v in enumerate(row):
        v = float(v)
        if v != v:
            return i
        if best is None or v > row[best]:
            best = i
    return 0 if best is None else best
