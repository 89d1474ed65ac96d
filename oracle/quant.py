"""Quantized-matmul oracle (test infrastructure only).

Two layouts are restated here.

1. The hot-path format this plugin accelerates (the workload's int4 and int8
   cases), written as the jnp program a user jits:

     int4 g64:  X bf16 [M, K]; W uint4 packed two nibbles per uint8 along K,
                [K/2, N], low nibble = even k (the reference's nibble order,
                ``src/jax_plugins/silicon/quantized.py:189-190``); per-group
                (64 along K) bf16 scale s [K/64, N] and uint4 zero-point z
                [K/64, N] held in uint8.  Y = X @ ((W - z) * s) -> bf16.
     int8 pc:   X bf16 [M, K]; W int8 [K, N]; f32 per-output-channel scale
                s [N].  Y = X @ (W * s) -> bf16.

   XLA:CPU evaluates the bf16 dequant expression op by op and rounds each
   bf16 result (``src/pjrt_plugin/ops/registry.h:273-287``): (W - z) is exact
   in bf16 (|W - z| <= 15) and the product with s is rounded to bf16.  The
   dot then accumulates bf16 x bf16 products in f32 and rounds the output
   to bf16 (``src/pjrt_plugin/ops/binary_ops.mm:775-782`` for the bf16 dot
   dtype rule).  This oracle accumulates in float64 and rounds once, so it is
   at least as accurate as XLA:CPU; tests compare at bf16 rel 2e-2.

2. The reference's own affine quantizer, ``affine_quantize`` /
   ``affine_dequantize`` (``quantized.py:276-482``): W [N, K], 8 nibbles per
   uint32 low-first (``:354-365``), w = scale * q + bias per (row, K/group)
   (``:326-339``, ``:473-478``).  It is restated so the reference tests' known
   answers (``tests/test_quantized.py:418-541``) pin this module, and so a
   reference-format weight can be carried into the hot-path format
   (``affine_to_int4_g64``) when its bias is an integer multiple of its scale.
"""

import numpy as np

from .bf16 import bf16_bits_to_f32, f32_to_bf16_bits, round_bf16

GROUP = 64


# ---------------------------------------------------------------------------
# hot-path format: nibble packing along K
# ---------------------------------------------------------------------------

def pack_int4_k(q):
    """q uint8 [K, N] with values 0..15 -> packed uint8 [K/2, N].

    packed[kp, n] = q[2kp, n] | (q[2kp+1, n] << 4): low nibble holds the even
    k, as in the reference's ``byte = q[i] | (q[i + 1] << 4)``
    (``quantized.py:189-190``).
    """
    q = np.asarray(q, dtype=np.uint8)
    if q.shape[0] % 2:
        raise ValueError("K must be even to pack two nibbles per byte")
    if (q > 15).any():
        raise ValueError("int4 values must lie in 0..15")
    return (q[0::2] | (q[1::2] << 4)).astype(np.uint8)


def unpack_int4_k(packed):
    """packed uint8 [K/2, N] -> q uint8 [K, N] (inverse of ``pack_int4_k``)."""
    p = np.asarray(packed, dtype=np.uint8)
    q = np.empty((p.shape[0] * 2,) + p.shape[1:], dtype=np.uint8)
    q[0::2] = p & 0x0F
    q[1::2] = p >> 4
    return q


def int4_g64_dequant(packed, s_bits, z, group=GROUP, round_to_bf16=True):
    """Dequantized weight W' = (q - z) * s as float32 [K, N].

    With ``round_to_bf16`` the product is rounded to bf16, as XLA:CPU does
    for the bf16 multiply; without it the exact value is returned.
    """
    q = unpack_int4_k(packed).astype(np.float32)
    K = q.shape[0]
    if K % group:
        raise ValueError("K must be a multiple of the group size")
    s = bf16_bits_to_f32(s_bits)
    zf = np.asarray(z, dtype=np.float32)
    if s.shape != (K // group,) + q.shape[1:] or zf.shape != s.shape:
        raise ValueError("scale/zero-point must be [K/group, N]")
    s_full = np.repeat(s, group, axis=0)
    z_full = np.repeat(zf, group, axis=0)
    w = (q - z_full) * s_full
    return round_bf16(w) if round_to_bf16 else w


def int4_g64_matmul(x_bits, packed, s_bits, z, group=GROUP, round_w=True):
    """Y = X @ ((W - z) * s): returns (y_f64 [M, N], y_bf16_bits [M, N])."""
    x = bf16_bits_to_f32(x_bits).astype(np.float64)
    w = int4_g64_dequant(packed, s_bits, z, group, round_to_bf16=round_w).astype(np.float64)
    if x.shape[1] != w.shape[0]:
        raise ValueError("X and W disagree on K")
    y = x @ w
    return y, f32_to_bf16_bits(y.astype(np.float32))


def int8_pc_matmul(x_bits, w_i8, s_f32):
    """Y = X @ (W * s) with per-output-channel f32 scale: (y_f64, y_bf16_bits).

    s factors out of the K sum: Y[m, n] = s[n] * sum_k X[m, k] W[k, n].
    """
    x = bf16_bits_to_f32(x_bits).astype(np.float64)
    w = np.asarray(w_i8, dtype=np.int8).astype(np.float64)
    s = np.asarray(s_f32, dtype=np.float32).astype(np.float64)
    if x.shape[1] != w.shape[0] or s.shape != (w.shape[1],):
        raise ValueError("shape mismatch in int8 dequant-matmul")
    y = (x @ w) * s[None, :]
    return y, f32_to_bf16_bits(y.astype(np.float32))


def make_int4_case(rng, M, K, N, group=GROUP):
    """Seeded synthetic inputs in the workload's draw order: X, W, s, z.

    X ~ N(0,1) bf16; q ~ U{0..15}; s ~ U(1e-3, 1e-2) bf16; z ~ U{0..15}.
    """
    x = f32_to_bf16_bits(rng.standard_normal((M, K)).astype(np.float32))
    q = rng.integers(0, 16, size=(K, N), dtype=np.uint8)
    s = f32_to_bf16_bits(rng.uniform(1e-3, 1e-2, size=(K // group, N)).astype(np.float32))
    z = rng.integers(0, 16, size=(K // group, N), dtype=np.uint8)
    return x, pack_int4_k(q), s, z


def make_int8_case(rng, M, K, N):
    """X ~ N(0,1) bf16; W ~ U{-127..127} int8; s ~ U(1e-3, 1e-2) f32."""
    x = f32_to_bf16_bits(rng.standard_normal((M, K)).astype(np.float32))
    w = rng.integers(-127, 128, size=(K, N), dtype=np.int16).astype(np.int8)
    s = rng.uniform(1e-3, 1e-2, size=(N,)).astype(np.float32)
    return x, w, s


# ---------------------------------------------------------------------------
# the reference's affine quantizer (quantized.py:276-482), bits 4 and 8
# ---------------------------------------------------------------------------

def affine_quantize(w, bits=4, group_size=64):
    """Restates ``affine_quantize`` (``quantized.py:276-405``) for 4/8 bits.

    Per (row, group): scale = (max - min) / (2^bits - 1), or 1.0 when the
    group is constant (``:326-327``); bias = min (``:328``);
    q = clip(round((w - bias) / scale), 0, 2^bits - 1) with numpy's
    round-half-to-even (``:334-336``).  4-bit values are packed eight per
    uint32, value j at bits 4j (``:354-365``).
    """
    if bits not in (4, 8):
        raise ValueError("only 4- and 8-bit affine codes are on this path")
    w = np.asarray(w, dtype=np.float32)
    K = w.shape[-1]
    if K % group_size:
        raise ValueError("last dimension must be divisible by group_size")
    flat = w.reshape(-1, K)
    g = flat.reshape(flat.shape[0], K // group_size, group_size)
    wmin = g.min(axis=2)
    wmax = g.max(axis=2)
    n_bins = (1 << bits) - 1
    # float() in the reference promotes min/max to Python floats (float64).
    scale64 = np.where(wmax != wmin, (wmax.astype(np.float64) - wmin.astype(np.float64)) / n_bins, 1.0)
    scale = scale64.astype(np.float32)
    bias = wmin.astype(np.float32)
    # (group - bias) / scale: float32 array op float Python scalar -> float32
    # arithmetic in numpy, as in the reference's per-group loop.
    qf = (g - bias[..., None]) / scale[..., None]
    q = np.clip(np.round(qf).astype(np.int32), 0, n_bins).reshape(flat.shape)
    if bits == 8:
        packed = q.astype(np.uint8)
    else:
        q8 = q.reshape(flat.shape[0], K // 8, 8).astype(np.uint32)
        shifts = (np.arange(8, dtype=np.uint32) * 4)[None, None, :]
        packed = np.bitwise_or.reduce((q8 & 0xF) << shifts, axis=2).astype(np.uint32)
    lead = w.shape[:-1]
    packed = packed.reshape(lead + (packed.shape[-1],))
    return packed, scale.reshape(lead + (K // group_size,)), bias.reshape(lead + (K // group_size,))


def affine_unpack(packed, bits, K):
    """Quantized integers [rows, K] from the reference's packing (``:430-448``)."""
    p = np.asarray(packed)
    flat = p.reshape(-1, p.shape[-1])
    if bits == 8:
        return flat[:, :K].astype(np.int32)
    words = flat.astype(np.uint32)
    shifts = (np.arange(8, dtype=np.uint32) * 4)[None, None, :]
    q = (words[:, :, None] >> shifts) & 0xF
    return q.reshape(flat.shape[0], -1)[:, :K].astype(np.int32)


def affine_dequantize(packed, scales, biases, bits=4, group_size=64, shape=None):
    """Restates ``affine_dequantize`` (``quantized.py:408-482``) for 4/8 bits."""
    scales = np.asarray(scales, dtype=np.float32)
    biases = np.asarray(biases, dtype=np.float32)
    if bits != 8 and shape is None:
        raise ValueError("shape is required for sub-byte dequantization")
    K = shape[-1] if shape is not None else np.asarray(packed).shape[-1]
    q = affine_unpack(packed, bits, K).astype(np.float32)
    G = K // group_size
    sc = scales.reshape(-1, G)
    bi = biases.reshape(-1, G)
    out = np.repeat(sc, group_size, axis=1) * q + np.repeat(bi, group_size, axis=1)
    return out.reshape(shape) if shape is not None else out


def affine_to_int4_g64(packed_u32, scales, biases, K, group_size=64):
    """Carry a reference-format 4-bit weight W [N, K] into the hot-path format.

    The reference stores w = scale*q + bias; the hot path stores
    w = (q' - z) * s.  With c = bias/scale an integer, q' = q + max(c, 0)
    and z = max(-c, 0) give the same w whenever q' <= 15 and scale is a bf16
    value.  Returns (packed [K/2, N], s_bits [K/64, N], z [K/64, N]) or
    raises ValueError when the weight is not representable.
    """
    if group_size != GROUP:
        raise ValueError("the hot-path format uses group size 64")
    q = affine_unpack(packed_u32, 4, K)               # [N, K]
    sc = np.asarray(scales, dtype=np.float32).reshape(q.shape[0], -1)
    bi = np.asarray(biases, dtype=np.float32).reshape(q.shape[0], -1)
    c = bi / sc
    if not np.all(c == np.round(c)):
        raise ValueError("bias is not an integer multiple of scale")
    c = c.astype(np.int64)
    s_bits = f32_to_bf16_bits(sc)
    if not np.array_equal(bf16_bits_to_f32(s_bits), sc):
        raise ValueError("scale is not exactly representable in bf16")
    shift = np.maximum(c, 0)
    z = np.maximum(-c, 0)
    qq = q + np.repeat(shift, group_size, axis=1)
    if (qq > 15).any() or (z > 15).any():
        raise ValueError("shifted codes leave the uint4 range")
    return pack_int4_k(qq.T.astype(np.uint8)), s_bits.T.copy(), z.T.astype(np.uint8).copy()
