"""dot_general oracle (test infrastructure only).

Semantics restated from the reference's ``HandleDotGeneral``
(``src/pjrt_plugin/ops/binary_ops.mm:644-1100``):

* result element type: the dot's declared result type; bf16 x bf16 with
  ``preferred_element_type=f32`` widens and returns f32 (``:775-782``);
* integer dots are exact (``:806-809``);
* a contracting size of 1 is a broadcast multiply, which keeps XLA's signed
  zero: (-0) * 1 = -0, where a sum seeded with +0 would give +0
  (``:904-1004``);
* zero-sized dims give zeros (``:832-845``).

Products are accumulated in float64 and rounded once to the result type, so
the oracle is at least as accurate as XLA:CPU's f32 accumulation; tests use
the workload's tolerances (f32 rel 1e-5, bf16 rel 2e-2).
"""

import numpy as np

from .bf16 import bf16_bits_to_f32, f32_to_bf16_bits


def dot_general(a, b, lhs_batch=(), rhs_batch=(), lhs_contract=(1,), rhs_contract=(0,)):
    """float64 dot_general on float arrays.

    Result dims follow StableHLO: batch dims, then lhs free dims, then rhs
    free dims.
    """
    a = np.asarray(a)
    b = np.asarray(b)
    la = [d for d in range(a.ndim) if d not in lhs_batch and d not in lhs_contract]
    rb = [d for d in range(b.ndim) if d not in rhs_batch and d not in rhs_contract]
    at = np.transpose(a, list(lhs_batch) + la + list(lhs_contract))
    bt = np.transpose(b, list(rhs_batch) + list(rhs_contract) + rb)
    nb = len(lhs_batch)
    bshape = at.shape[:nb]
    fa = at.shape[nb:nb + len(la)]
    fb = bt.shape[nb + len(rhs_contract):]
    K = int(np.prod(at.shape[nb + len(la):], dtype=np.int64))
    A = at.reshape(bshape + (int(np.prod(fa, dtype=np.int64)), K)).astype(np.float64)
    B = bt.reshape(bshape + (K, int(np.prod(fb, dtype=np.int64)))).astype(np.float64)
    if K == 1:
        # Broadcast multiply: keeps the sign of zero products.
        C = A * B
    elif K == 0:
        C = np.zeros(bshape + (A.shape[-2], B.shape[-1]), dtype=np.float64)
    else:
        C = np.matmul(A, B)
    return C.reshape(bshape + fa + fb)


def matmul_bf16(a_bits, b_bits, out="f32"):
    """[.., M, K] x [.., K, N] bf16 matmul with f32 accumulation semantics.

    Returns (c_f64, c_out) where c_out is float32 (``out="f32"``, the
    preferred_element_type=f32 case) or bf16 bits (``out="bf16"``).
    """
    a = bf16_bits_to_f32(a_bits).astype(np.float64)
    b = bf16_bits_to_f32(b_bits).astype(np.float64)
    c = np.matmul(a, b)
    if out == "f32":
        return c, c.astype(np.float32)
    return c, f32_to_bf16_bits(c.astype(np.float32))


def matmul_f32(a, b):
    """f32 matmul: (c_f64, c_f32)."""
    c = np.matmul(np.asarray(a, np.float64), np.asarray(b, np.float64))
    return c, c.astype(np.float32)


def rel_err(out, ref):
    """max|out - ref| / max|ref| -- the reference's GEMM error measure
    (``tests/test_f32_gemm_precision.py:25-27``)."""
    out = np.asarray(out, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    denom = np.max(np.abs(ref))
    return float(np.max(np.abs(out - ref)) / (denom if denom > 0 else 1.0))
