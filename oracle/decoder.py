"""Llama-style decoder-layer oracle (test infrastructure only).

Restates one layer of the workload's decoder in float64
with a bf16 rounding wherever the plugin's layer writes a bf16 activation,
built from the other oracle modules (``quant.int4_g64_dequant`` for every
projection, ``rowops.rmsnorm``, ``bf16.round_bf16``).  The layer is the
reference's transformer-layer benchmark (``benchmarks/vs_cpu.py:603-626``:
qkv = xn @ wqkv reshaped (B, T, 3, H, Dh); logits = q @ swapaxes(k) * Dh**-0.5;
softmax; @ v; heads merged; x + out @ wo; MLP; residual) with the workload's
Llama choices: RMSNorm (eps 1e-6) for LayerNorm, rotate-half RoPE on q and k,
a causal mask, SwiGLU ``(silu(h @ Wg) * (h @ Wu)) @ Wd`` and int4 g64
projections whose dequantised weight is rounded to bf16 as XLA:CPU rounds the
bf16 ``(q - z) * s`` (``src/pjrt_plugin/ops/registry.h:273-287``), or, with
``exact_weights=True``, used exactly: the form of a program that converts q, z
and s to f32 before the product (``mi355x/programs.py``'s int4 projections),
where ``(q - z) * s`` of a 4-bit difference and a bf16 scale is exact in f32.
Over a 4-layer stack the two conventions alone differ by up to ~4e-2 per row
at the bf16 measure, so each program is checked against its own.

Rounding points (each is one bf16 rounding of a float64 value):
    h    = r(rmsnorm(x) * g)
    qkv  = r(h @ Wqkv)
    q, k = r(rope(q)), r(rope(k));  v = qkv's v block
    a    = r(softmax_causal(q k^T * Dh**-0.5) @ v)     (heads merged)
    x1   = r(x + r(a @ Wo))
    h2   = r(rmsnorm(x1) * g2)
    act  = r(r(g * r(logistic(g))) * u),  g = r(h2 @ Wg), u = r(h2 @ Wu)
    x2   = r(x1 + r(act @ Wd))
Inside the attention the oracle keeps float64 throughout; the plugin's fused
kernel rounds P to bf16 before P @ V, so the two agree at the workload's bf16
tolerance, not bit for bit.

Only the rows of the requested query positions are computed (plus the keys
and values of every earlier position, which causal attention reads), so a
full-size layer is checked on a token subset in seconds.
"""

import numpy as np

from . import quant, rowops
from .bf16 import bf16_bits_to_f32, round_bf16


def rope_tables(seq, head_dim, base=10000.0):
    """cos, sin [seq, head_dim/2] (float64) for positions 0..seq-1 and
    frequencies base^(-2i/head_dim)."""
    half = head_dim // 2
    inv = base ** (-np.arange(half, dtype=np.float64) * 2.0 / head_dim)
    ang = np.arange(seq, dtype=np.float64)[:, None] * inv[None, :]
    return np.cos(ang), np.sin(ang)


def rope(x, cos, sin):
    """Rotate-half RoPE of x [..., D] with per-row tables cos/sin [..., D/2]:
    (x0, x1) -> (x0 cos - x1 sin, x1 cos + x0 sin) for the halves x0, x1."""
    half = x.shape[-1] // 2
    x0, x1 = x[..., :half], x[..., half:]
    return np.concatenate([x0 * cos - x1 * sin, x1 * cos + x0 * sin], axis=-1)


def attention_causal_rows(q_rows, pos, k_all, v_all, scale):
    """Causal attention for query rows q_rows [R, D] at positions pos [R]
    against keys / values k_all, v_all [S, D]: row r attends to keys 0..pos[r]."""
    out = np.empty_like(q_rows, dtype=np.float64)
    for r, p in enumerate(pos):
        s = (k_all[:p + 1] @ q_rows[r]) * scale
        e = np.exp(s - s.max())
        out[r] = (e / e.sum()) @ v_all[:p + 1]
    return out


def _w(weight, exact=False):
    """Dequantised int4 g64 weight [K, N] (float64) from (packed, s_bits, z):
    rounded to bf16, or exact with ``exact``."""
    packed, s_bits, z = weight
    return quant.int4_g64_dequant(packed, s_bits, z, round_to_bf16=not exact).astype(np.float64)


def _logistic(x):
    return 1.0 / (1.0 + np.exp(-x))


def attention_block(x, pos, w, heads, head_dim, eps=1e-6, rope_base=10000.0, exact_weights=False):
    """The attention half of a layer at query positions `pos` of one sequence
    x [S, hidden]: {"attn": heads-merged attention output a, "attn_proj":
    r(a @ Wo), "x1": r(x + r(a @ Wo))} for those rows."""
    x = np.asarray(x, dtype=np.float64)
    pos = np.asarray(pos, dtype=np.int64)
    S, hidden = x.shape
    H, D = heads, head_dim
    A = H * D
    last = int(pos.max()) + 1
    g1 = bf16_bits_to_f32(w["g_attn"]).astype(np.float64)
    cos, sin = rope_tables(S, D, rope_base)
    h = round_bf16(rowops.rmsnorm(x[:last], g1, eps))
    wqkv = _w(w["w_qkv"], exact_weights)
    kv = round_bf16(h @ wqkv[:, A:])                        # k | v of positions 0..last-1
    qr = round_bf16(h[pos] @ wqkv[:, :A])                   # q of the requested rows
    k = kv[:, :A].reshape(last, H, D)
    v = kv[:, A:].reshape(last, H, D)
    k = round_bf16(rope(k, cos[:last, None, :], sin[:last, None, :]))
    q = round_bf16(rope(qr.reshape(len(pos), H, D), cos[pos][:, None, :], sin[pos][:, None, :]))
    scale = 1.0 / np.sqrt(D)
    a = np.empty((len(pos), H, D))
    for hd in range(H):
        a[:, hd] = attention_causal_rows(q[:, hd], pos, k[:, hd], v[:, hd], scale)
    a = round_bf16(a.reshape(len(pos), A))
    return {"attn": a, **output_residual(x[pos], a, w["w_o"], exact_weights)}


def output_residual(x_rows, a_rows, w_o, exact_weights=False):
    """{"attn_proj": r(a @ Wo), "x1": r(x + r(a @ Wo))} for given rows."""
    attn_proj = round_bf16(np.asarray(a_rows, np.float64) @ _w(w_o, exact_weights))
    return {"attn_proj": attn_proj, "x1": round_bf16(np.asarray(x_rows, np.float64) + attn_proj)}


def mlp_act(x1_rows, w, eps=1e-6, exact_weights=False):
    """act = r(r(g * r(logistic(g))) * u) with g = r(h2 @ Wg), u = r(h2 @ Wu),
    h2 = r(rmsnorm(x1) * g_mlp), for rows of x1."""
    g2 = bf16_bits_to_f32(w["g_mlp"]).astype(np.float64)
    h2 = round_bf16(rowops.rmsnorm(np.asarray(x1_rows, np.float64), g2, eps))
    gt = round_bf16(h2 @ _w(w["w_gate"], exact_weights))
    up = round_bf16(h2 @ _w(w["w_up"], exact_weights))
    return round_bf16(round_bf16(gt * round_bf16(_logistic(gt))) * up)


def down_residual(x1_rows, act_rows, w_down, exact_weights=False):
    """{"down": r(act @ Wd), "out": r(x1 + r(act @ Wd))} for given rows."""
    down = round_bf16(np.asarray(act_rows, np.float64) @ _w(w_down, exact_weights))
    return {"down": down, "out": round_bf16(np.asarray(x1_rows, np.float64) + down)}


def layer_rows(x, pos, w, heads, head_dim, eps=1e-6, rope_base=10000.0, parts=False, exact_weights=False):
    """One decoder layer of one sequence, evaluated at query positions `pos`.

    x    float [S, hidden] -- the layer's bf16 input (as float values)
    pos  int [R] -- query positions to return
    w    dict: g_attn, g_mlp (bf16 bits [hidden]); w_qkv, w_o, w_gate, w_up,
         w_down as (packed uint8 [K/2, N], scale bf16 bits [K/64, N],
         zero uint8 [K/64, N])
    exact_weights: use (q - z) * s exactly instead of its bf16 rounding
    Returns the layer output rows [R, hidden] (float64 values of bf16), or
    with ``parts`` a dict of them ("out") and of every intermediate the
    blocks above return ("attn", "attn_proj", "x1", "act", "down").
    """
    att = attention_block(x, pos, w, heads, head_dim, eps, rope_base, exact_weights)
    act = mlp_act(att["x1"], w, eps, exact_weights)
    dr = down_residual(att["x1"], act, w["w_down"], exact_weights)
    if parts:
        return {**att, "act": act, **dr}
    return dr["out"]
