"""bfloat16 helpers for the oracle (test infrastructure only).

numpy has no bfloat16 dtype here (``ml_dtypes`` is not installed), so bf16
tensors are carried as ``uint16`` bit patterns.  Rounding is IEEE
round-to-nearest-even from float32, which is what XLA:CPU's ``convert`` to
bf16 does and what the reference relies on when it states that XLA:CPU
rounds every bf16 op result (``src/pjrt_plugin/ops/registry.h:273-287``).
"""

import numpy as np


def f32_to_bf16_bits(x):
    """float32 array -> uint16 bf16 bit patterns, round-to-nearest-even.

    NaN stays NaN (quiet bit forced, sign kept); +-inf stay inf; values that
    round past the largest finite bf16 become inf, as in IEEE RNE.
    """
    x = np.asarray(x, dtype=np.float32)
    shape = x.shape
    x = np.ascontiguousarray(x).reshape(-1)
    u = x.view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    rounded = ((u + 0x7FFF + lsb) >> 16).astype(np.uint32)
    nan = np.isnan(x)
    out = rounded.astype(np.uint16)
    if nan.any():
        out = out.copy()
        out[nan] = ((u[nan] >> 16) | 0x0040).astype(np.uint16)
    return out.reshape(shape)


def bf16_bits_to_f32(b):
    """uint16 bf16 bit patterns -> float32 (exact widening)."""
    b = np.asarray(b, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32).reshape(b.shape)


def round_bf16(x):
    """Round float values to the nearest bf16 and return them as float32."""
    return bf16_bits_to_f32(f32_to_bf16_bits(np.asarray(x, dtype=np.float32)))


def randn_bf16(rng, shape, scale=1.0):
    """Draw N(0, scale^2) float32 values and round them to bf16 bits."""
    return f32_to_bf16_bits((rng.standard_normal(shape) * scale).astype(np.float32))
