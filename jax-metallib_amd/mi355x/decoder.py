"""Llama-style decoder forward on the plugin's kernels (the workload's
decoder config: layers x [RMSNorm, fused QKV projection, RoPE, causal
softmax attention, output projection, residual, RMSNorm, SwiGLU MLP,
residual], int4 group-64 weights, bf16 activations).

The layer follows the reference's transformer-layer benchmark
(benchmarks/vs_cpu.py:603-626: qkv = xn @ wqkv reshaped (B, T, 3, H, Dh);
logits = q @ swapaxes(k) * Dh**-0.5; softmax; @ v; transpose back; x + out
@ wo; MLP; residual), with the Llama choices of the workload: RMSNorm
(eps 1e-6) instead of LayerNorm, rotary embedding on q and k, a causal mask,
SwiGLU (silu(h @ Wg) * (h @ Wu)) @ Wd, and every projection an int4 g64
dequant-matmul.

Every step is one C-ABI call on the current stream (no allocation inside
`forward` when the Buffers are reused), so a whole forward can be captured
in one HIP graph:

    h    = rmsnorm(x, g_attn)                      mk_rmsnorm_lastdim
    qkv  = h @ Wqkv                                mk_int4g64_matmul_bf16
    q, k, v = split + rope(qkv)                    mk_rope_qkv_split_bf16
    a    = causal_attention(q, k, v), heads merged mk_attention_causal_bf16
    x    = x + a @ Wo     (add in the GEMM store)  mk_int4g64_matmul_epilogue_bf16
    h    = rmsnorm(x, g_mlp)
    act  = silu(h @ Wg) * (h @ Wu)                 mk_int4g64_matmul_epilogue_bf16,
           one product against [Wg | Wu] with        MK_EPI_SWIGLU_PAIRS (with
           16-column blocks interleaved              fewer tokens than the
                                                     many-row route takes: g,
                                                     then MK_EPI_SWIGLU)
    x    = x + act @ Wd   (add in the GEMM store)  mk_int4g64_matmul_epilogue_bf16

fuse_epilogues=False runs the gate and up projections as two products and
the residual adds and silu(g) * u as separate elementwise programs
(mk_elementwise); the results are bit-identical.

attention="composed" runs the attention as the reference's layer writes it,
one op at a time: s = q @ k^T (mk_gemm_bf16 on kT), p = causal softmax of
s * Dh**-0.5 in place (mk_softmax_causal_bf16), o = p @ v (mk_gemm_bf16),
merge heads (mk_merge_heads_bf16).  It materialises the [B*H, S, S] scores.
"""

import math
from dataclasses import dataclass

import numpy as np
import torch

from . import ops

GROUP = 64


@dataclass(frozen=True)
class DecoderConfig:
    layers: int = 4
    hidden: int = 2048
    heads: int = 16
    head_dim: int = 128
    ffn: int = 8192
    batch: int = 4
    seq: int = 2048
    rope_base: float = 10000.0
    eps: float = 1e-6

    @property
    def tokens(self):
        return self.batch * self.seq

    def matmul_flops(self, causal=True):
        """FLOPs of one forward: the projections plus the two attention
        products (q @ k^T, p @ v), the latter over the causal half
        (S (S + 1) / 2 score entries per head) unless causal=False."""
        T, Hd, A = self.tokens, self.hidden, self.heads * self.head_dim
        proj = 2 * T * (Hd * 3 * A + A * Hd + 2 * Hd * self.ffn + self.ffn * Hd)
        pairs = self.seq * (self.seq + 1) // 2 if causal else self.seq * self.seq
        attn = 2 * 2 * self.batch * self.heads * pairs * self.head_dim
        return self.layers * (proj + attn)


@dataclass
class Int4Weight:
    """int4 g64 weight W [K, N]: packed uint8 [K/2, N] (low nibble = even k),
    bf16 scale [K/64, N], uint8 zero [K/64, N]."""
    packed: torch.Tensor
    scale: torch.Tensor
    zero: torch.Tensor

    @property
    def shape(self):
        return (self.packed.shape[0] * 2, self.packed.shape[1])


def random_int4(rng, K, N, device, scale_lo=0.004, scale_hi=0.006):
    """Random int4 g64 weight: q, z ~ U{0..15}, s ~ U(scale_lo, scale_hi)."""
    q = rng.integers(0, 16, size=(K, N), dtype=np.uint8)
    packed = (q[0::2] | (q[1::2] << 4)).astype(np.uint8)
    s = rng.uniform(scale_lo, scale_hi, size=(K // GROUP, N)).astype(np.float32)
    z = rng.integers(0, 16, size=(K // GROUP, N), dtype=np.uint8)
    return Int4Weight(torch.from_numpy(packed).to(device),
                      torch.from_numpy(s).to(torch.bfloat16).to(device),
                      torch.from_numpy(z).to(device))


@dataclass
class LayerWeights:
    g_attn: torch.Tensor
    w_qkv: Int4Weight
    w_o: Int4Weight
    g_mlp: torch.Tensor
    w_gate: Int4Weight
    w_up: Int4Weight
    w_down: Int4Weight
    w_gateup: Int4Weight = None  # w_gate and w_up, 16-column blocks interleaved


def interleave_int4(a: Int4Weight, b: Int4Weight) -> Int4Weight:
    """[Wa | Wb] with 16-column blocks alternating (int4 g64 packs along K,
    so every array of the weight is interleaved by column alike)."""
    return Int4Weight(ops.interleave_gate_up(a.packed, b.packed), ops.interleave_gate_up(a.scale, b.scale),
                      ops.interleave_gate_up(a.zero, b.zero))


def init_weights(cfg: DecoderConfig, seed=0, device="cuda"):
    """Random-init weights of every layer (the workload uses random init)."""
    rng = np.random.default_rng(seed)
    A = cfg.heads * cfg.head_dim
    layers = []
    for _ in range(cfg.layers):
        g1 = torch.from_numpy(rng.uniform(0.5, 1.5, size=cfg.hidden).astype(np.float32)).to(torch.bfloat16)
        g2 = torch.from_numpy(rng.uniform(0.5, 1.5, size=cfg.hidden).astype(np.float32)).to(torch.bfloat16)
        layers.append(LayerWeights(
            g_attn=g1.to(device), w_qkv=random_int4(rng, cfg.hidden, 3 * A, device),
            w_o=random_int4(rng, A, cfg.hidden, device), g_mlp=g2.to(device),
            w_gate=random_int4(rng, cfg.hidden, cfg.ffn, device),
            w_up=random_int4(rng, cfg.hidden, cfg.ffn, device),
            w_down=random_int4(rng, cfg.ffn, cfg.hidden, device)))
        layers[-1].w_gateup = interleave_int4(layers[-1].w_gate, layers[-1].w_up)
    return layers


def rope_tables(cfg: DecoderConfig, device="cuda"):
    """cos / sin [seq, head_dim/2] (f32) of positions 0..seq-1 and
    frequencies base^(-2i/head_dim), computed in float64."""
    half = cfg.head_dim // 2
    inv = cfg.rope_base ** (-np.arange(half, dtype=np.float64) * 2.0 / cfg.head_dim)
    ang = np.arange(cfg.seq, dtype=np.float64)[:, None] * inv[None, :]
    return (torch.from_numpy(np.cos(ang).astype(np.float32)).to(device),
            torch.from_numpy(np.sin(ang).astype(np.float32)).to(device))


# silu(g) * u as a bf16 register program: slots 0 = g, 1 = u.
SWIGLU_PROGRAM = [
    ("LOAD", 0, 0, 0, 0, 0.0), ("LOAD", 1, 1, 0, 0, 0.0),
    ("LOGISTIC", 2, 0, 0, 0, 0.0), ("MUL", 3, 0, 2, 0, 0.0), ("MUL", 4, 3, 1, 0, 0.0),
]
RESIDUAL_PROGRAM = [("LOAD", 0, 0, 0, 0, 0.0), ("LOAD", 1, 1, 0, 0, 0.0), ("ADD", 2, 0, 1, 0, 0.0)]


class Buffers:
    """Every activation of one forward, allocated once (the score matrix only
    for the composed attention)."""

    def __init__(self, cfg: DecoderConfig, device="cuda", attention="fused", fuse_epilogues=True):
        T, A, BH = cfg.tokens, cfg.heads * cfg.head_dim, cfg.batch * cfg.heads
        bf = dict(dtype=torch.bfloat16, device=device)
        self.x = torch.empty((T, cfg.hidden), **bf)
        self.h = torch.empty((T, cfg.hidden), **bf)
        self.qkv = torch.empty((T, 3 * A), **bf)
        self.attention = attention
        self.fuse = fuse_epilogues
        self.q = torch.empty((BH, cfg.seq, cfg.head_dim), **bf)
        kshape = (BH, cfg.head_dim, cfg.seq) if attention == "composed" else (BH, cfg.seq, cfg.head_dim)
        self.k = torch.empty(kshape, **bf)
        self.v = torch.empty((BH, cfg.seq, cfg.head_dim), **bf)
        if attention == "composed":
            self.s = torch.empty((BH, cfg.seq, cfg.seq), **bf)
            self.o = torch.empty((BH, cfg.seq, cfg.head_dim), **bf)
        self.attn = torch.empty((T, A), **bf)
        self.proj = torch.empty((T, cfg.hidden), **bf)
        self.gate = torch.empty((T, cfg.ffn), **bf)
        self.up = torch.empty((T, cfg.ffn), **bf)
        self.act = torch.empty((T, cfg.ffn), **bf)


def _qmm(x, w: Int4Weight, out, epilogue=None, aux=None):
    return ops.int4_g64_matmul(x, w.packed, w.scale, w.zero, out=out, epilogue=epilogue, aux=aux)


def layer_forward(cfg: DecoderConfig, lw: LayerWeights, buf: Buffers, cos, sin, taps=None):
    """One decoder layer on buf.x, in place.  With a dict `taps`, copies of
    the attention output ("attn"), the residual stream after the attention
    block ("x1") and the SwiGLU activation ("act") are stored in it (for
    stage-by-stage checks; the copies allocate, so leave taps None under
    graph capture)."""
    B, S, H, D = cfg.batch, cfg.seq, cfg.heads, cfg.head_dim
    ops.rmsnorm(buf.x, lw.g_attn, eps=cfg.eps, out=buf.h)
    _qmm(buf.h, lw.w_qkv, buf.qkv)
    composed = buf.attention == "composed"
    ops.rope_qkv_split(buf.qkv, cos, sin, B, S, H, D, q=buf.q, k=buf.k, v=buf.v, k_transposed=composed)
    if composed:
        ops.gemm_bf16(buf.q, buf.k, out=buf.s)
        ops.softmax_causal(buf.s, 1.0 / math.sqrt(D), out=buf.s)
        ops.gemm_bf16(buf.s, buf.v, out=buf.o)
        ops.merge_heads(buf.o, B, H, out=buf.attn)
    else:
        ops.attention_causal(buf.q, buf.k, buf.v, B, H, 1.0 / math.sqrt(D), out=buf.attn)
    def tap(name, t):
        if taps is not None:
            taps[name] = t.clone()

    tap("attn", buf.attn)
    if buf.fuse:
        # Residual adds and silu(g) * u ride on the projections' stores, and
        # the gate and up projections are one product (bit-identical to the
        # separate products and elementwise programs below).
        _qmm(buf.attn, lw.w_o, buf.x, epilogue="add", aux=buf.x)
        tap("x1", buf.x)
        ops.rmsnorm(buf.x, lw.g_mlp, eps=cfg.eps, out=buf.h)
        if ops.int4_swiglu_pairs_supported(cfg.tokens, cfg.hidden, 2 * cfg.ffn):
            _qmm(buf.h, lw.w_gateup, buf.act, epilogue="swiglu_pairs")
        else:  # too few tokens for the many-row route: two products
            _qmm(buf.h, lw.w_gate, buf.gate)
            _qmm(buf.h, lw.w_up, buf.act, epilogue="swiglu", aux=buf.gate)
        tap("act", buf.act)
        _qmm(buf.act, lw.w_down, buf.x, epilogue="add", aux=buf.x)
        return
    _qmm(buf.attn, lw.w_o, buf.proj)
    ops.elementwise(RESIDUAL_PROGRAM, [buf.x, buf.proj], out_slot=2, out=buf.x)
    tap("x1", buf.x)
    ops.rmsnorm(buf.x, lw.g_mlp, eps=cfg.eps, out=buf.h)
    _qmm(buf.h, lw.w_gate, buf.gate)
    _qmm(buf.h, lw.w_up, buf.up)
    ops.elementwise(SWIGLU_PROGRAM, [buf.gate, buf.up], out_slot=4, out=buf.act)
    tap("act", buf.act)
    _qmm(buf.act, lw.w_down, buf.proj)
    ops.elementwise(RESIDUAL_PROGRAM, [buf.x, buf.proj], out_slot=2, out=buf.x)


def forward(cfg: DecoderConfig, weights, buf: Buffers, cos, sin):
    """All layers on buf.x (bf16 [batch*seq, hidden]), in place."""
    for lw in weights:
        layer_forward(cfg, lw, buf, cos, sin)
    return buf.x
