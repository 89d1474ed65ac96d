"""Seeded synthetic inputs of the workload's quantized shapes, for the
benchmark and profiling runs (there is no dataset or checkpoint on this
path; the weights are random draws of the right format).

Formats (the ones ``ops.int4_g64_matmul`` / ``ops.int8_pc_matmul`` take):
  int4 g64: x bf16 [M, K]; W packed uint8 [K/2, N], byte (i, n) holding
            k = 2i in its low nibble and k = 2i + 1 in its high nibble;
            scale bf16 [K/64, N]; zero point uint8 [K/64, N] (0..15).
  int8 pc:  x bf16 [M, K]; W int8 [K, N]; scale f32 [N].

Draws, in this order from one ``numpy.random.Generator``:
  x ~ N(0, 1); q ~ U{0..15}; s ~ U(1e-3, 1e-2); z ~ U{0..15}   (int4)
  x ~ N(0, 1); W ~ U{-127..127}; s ~ U(1e-3, 1e-2)              (int8)
bf16 values are the round-to-nearest-even bf16 of the f32 draw, returned as
uint16 bit patterns.
"""

import numpy as np

GROUP = 64


def bf16_bits(x):
    """float32 array -> uint16 bf16 bit patterns, round to nearest even
    (finite inputs: every draw here is finite)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def pack_nibbles(q):
    """uint8 [K, N] values 0..15 -> uint8 [K/2, N], even k in the low nibble."""
    q = np.asarray(q, dtype=np.uint8)
    return (q[0::2] | (q[1::2] << 4)).astype(np.uint8)


def int4_case(rng, M, K, N):
    """(x bf16 bits [M, K], W packed [K/2, N], scale bf16 bits [K/64, N],
    zero uint8 [K/64, N])."""
    x = bf16_bits(rng.standard_normal((M, K)).astype(np.float32))
    q = rng.integers(0, 16, size=(K, N), dtype=np.uint8)
    s = bf16_bits(rng.uniform(1e-3, 1e-2, size=(K // GROUP, N)).astype(np.float32))
    z = rng.integers(0, 16, size=(K // GROUP, N), dtype=np.uint8)
    return x, pack_nibbles(q), s, z


def int8_case(rng, M, K, N):
    """(x bf16 bits [M, K], W int8 [K, N], scale f32 [N])."""
    x = bf16_bits(rng.standard_normal((M, K)).astype(np.float32))
    w = rng.integers(-127, 128, size=(K, N), dtype=np.int16).astype(np.int8)
    s = rng.uniform(1e-3, 1e-2, size=(N,)).astype(np.float32)
    return x, w, s


def decoder_stack_case(rng, layers, B, S, hidden, heads, head_dim, ffn, rope_base=10000.0):
    """decoder_layer_case for `layers` layers: (x, [weights per layer], cos, sin)."""
    x, w, cos, sin = decoder_layer_case(rng, B, S, hidden, heads, head_dim, ffn, rope_base)
    ws = [w] + [decoder_layer_case(rng, 1, 1, hidden, heads, head_dim, ffn, rope_base, weights_only=True)
                for _ in range(layers - 1)]
    return x, ws, cos, sin


def decoder_stack_arguments(x, ws, cos, sin):
    """The arguments of programs.decoder_stack in order, as (array, is_bf16)."""
    args = [(x, True)]
    for w in ws:
        args += decoder_layer_arguments(None, w, None, None)[1:-2]
    return args + [(cos, False), (sin, False)]


def decoder_stack_scan_arguments(x, ws, cos, sin):
    """The arguments of programs.decoder_stack_scan in order, as (array,
    is_bf16): each of a layer's 17 weight arrays stacked over the layers."""
    per = [decoder_layer_arguments(None, w, None, None)[1:-2] for w in ws]
    args = [(x, True)]
    for k in range(len(per[0])):
        args.append((np.ascontiguousarray(np.stack([p[k][0] for p in per])), per[0][k][1]))
    return args + [(cos, False), (sin, False)]


def decoder_layer_case(rng, B, S, hidden, heads, head_dim, ffn, rope_base=10000.0, weights_only=False):
    """One random-init layer of the Llama-style decoder and its input:
    (x bf16 bits [B*S, hidden], weights, cos, sin).  weights holds g_attn,
    g_mlp (bf16 bits, U(0.5, 1.5)) and w_qkv, w_o, w_gate, w_up, w_down as
    int4 g64 (packed, scale bf16 bits, zero) with s ~ U(0.004, 0.006), scales
    that keep a random layer's activations O(1); cos / sin f32 [S, head_dim/2]
    of positions 0..S-1 at frequencies rope_base^(-2i/head_dim)."""
    A = heads * head_dim

    def weight(K, N):
        q = rng.integers(0, 16, size=(K, N), dtype=np.uint8)
        s = bf16_bits(rng.uniform(0.004, 0.006, size=(K // GROUP, N)).astype(np.float32))
        z = rng.integers(0, 16, size=(K // GROUP, N), dtype=np.uint8)
        return pack_nibbles(q), s, z

    x = None if weights_only else bf16_bits(rng.standard_normal((B * S, hidden)).astype(np.float32))
    g1 = bf16_bits(rng.uniform(0.5, 1.5, size=hidden).astype(np.float32))
    g2 = bf16_bits(rng.uniform(0.5, 1.5, size=hidden).astype(np.float32))
    w = {"g_attn": g1, "g_mlp": g2, "w_qkv": weight(hidden, 3 * A), "w_o": weight(A, hidden),
         "w_gate": weight(hidden, ffn), "w_up": weight(hidden, ffn), "w_down": weight(ffn, hidden)}
    if weights_only:
        return w
    half = head_dim // 2
    inv = rope_base ** (-np.arange(half, dtype=np.float64) * 2.0 / head_dim)
    ang = np.arange(S, dtype=np.float64)[:, None] * inv[None, :]
    return x, w, np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def decoder_layer_arguments(x, w, cos, sin):
    """The arguments of programs.decoder_layer in order, as (array, is_bf16)."""
    args = [(x, True), (w["g_attn"], True)]
    for name in ("w_qkv", "w_o"):
        p, s, z = w[name]
        args += [(p, False), (s, True), (z, False)]
    args.append((w["g_mlp"], True))
    for name in ("w_gate", "w_up", "w_down"):
        p, s, z = w[name]
        args += [(p, False), (s, True), (z, False)]
    return args + [(cos, False), (sin, False)]
