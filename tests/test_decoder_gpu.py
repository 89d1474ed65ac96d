"""GPU parity of the decoder-layer kernels (RoPE + head split, causal
softmax, head merge) and of a whole Llama-style decoder forward
(mi355x/decoder.py) against a float32 torch-CPU reference that rounds to
bf16 at the same points the kernels do (every kernel writes bf16).

These are floating-point kernels with no reference counterpart (jax.jit
lowers them to generic StableHLO), so the checks are the plain float32 /
float64 restatements below, at the workload's bf16 tolerance."""

import math

import numpy as np
import pytest

from _gpu import BF16_RTOL, assert_rel_close, need_gpu, torch

pytestmark = pytest.mark.gpu


def _ops():
    need_gpu()
    from mi355x import ops
    return ops


def _bf(t):
    return t.to(torch.bfloat16).to(torch.float32)


def _rope_ref(x, cos, sin):
    """Rotate-half RoPE on [..., S, D] (f32) with tables [S, D/2]."""
    half = x.shape[-1] // 2
    x0, x1 = x[..., :half], x[..., half:]
    return torch.cat([x0 * cos - x1 * sin, x1 * cos + x0 * sin], dim=-1)


def _tables(S, D, base=10000.0):
    inv = base ** (-np.arange(D // 2, dtype=np.float64) * 2.0 / D)
    ang = np.arange(S, dtype=np.float64)[:, None] * inv[None, :]
    return torch.from_numpy(np.cos(ang).astype(np.float32)), torch.from_numpy(np.sin(ang).astype(np.float32))


@pytest.mark.parametrize("B,S,H", [(1, 64, 1), (2, 128, 3), (3, 192, 2)])
def test_rope_qkv_split(B, S, H):
    ops = _ops()
    D = 128
    g = torch.Generator().manual_seed(B * 100 + S + H)
    qkv = torch.randn((B * S, 3 * H * D), generator=g).to(torch.bfloat16)
    cos, sin = _tables(S, D)
    q, kT, v = ops.rope_qkv_split(qkv.cuda(), cos.cuda(), sin.cuda(), B, S, H, D)
    q2, k2, v2 = ops.rope_qkv_split(qkv.cuda(), cos.cuda(), sin.cuda(), B, S, H, D, k_transposed=False)
    torch.cuda.synchronize()
    assert torch.equal(q2, q) and torch.equal(v2, v) and torch.equal(k2.transpose(1, 2), kT)
    x = qkv.float().reshape(B, S, 3, H, D).permute(2, 0, 3, 1, 4)  # [3, B, H, S, D]
    q_ref = _bf(_rope_ref(x[0], cos, sin)).reshape(B * H, S, D)
    k_ref = _bf(_rope_ref(x[1], cos, sin)).reshape(B * H, S, D)
    v_ref = x[2].reshape(B * H, S, D)
    # One rounding of an f32 FMA-or-not expression: within one bf16 ulp.
    assert torch.allclose(q.float().cpu(), q_ref, rtol=2 ** -7, atol=1e-6)
    assert torch.allclose(kT.float().cpu(), k_ref.transpose(1, 2), rtol=2 ** -7, atol=1e-6)
    assert torch.equal(v.float().cpu(), v_ref)  # v is copied exactly


@pytest.mark.parametrize("batches,S", [(1, 64), (3, 128), (2, 2048), (1, 4096)])
def test_softmax_causal(batches, S):
    ops = _ops()
    g = torch.Generator().manual_seed(S + batches)
    s = (torch.randn((batches, S, S), generator=g) * 4).to(torch.bfloat16)
    scale = 1.0 / math.sqrt(128)
    p = ops.softmax_causal(s.cuda(), scale).float().cpu()
    x = s.double() * scale
    mask = torch.ones((S, S), dtype=torch.bool).tril()
    x = x.masked_fill(~mask, float("-inf"))
    ref = torch.softmax(x, dim=-1)
    assert torch.all(p.masked_select(~mask.expand_as(p)) == 0)
    assert torch.allclose(p.double(), ref, rtol=2 ** -7, atol=1e-7)
    # Rows sum to one within bf16 rounding of each term.
    assert torch.allclose(p.double().sum(-1), torch.ones((batches, S), dtype=torch.float64), atol=2e-2)


def test_softmax_causal_in_place_and_first_row():
    ops = _ops()
    s = torch.randn((2, 64, 64)).to(torch.bfloat16).cuda()
    ref = ops.softmax_causal(s.clone(), 0.5)
    ops.softmax_causal(s, 0.5, out=s)
    torch.cuda.synchronize()
    assert torch.equal(s, ref)
    assert torch.all(s[:, 0, 0].float() == 1.0)  # row 0 keeps only column 0


@pytest.mark.parametrize("B,H,S", [(1, 1, 8), (2, 3, 40), (4, 16, 64)])
def test_merge_heads(B, H, S):
    ops = _ops()
    o = torch.randn((B * H, S, 128)).to(torch.bfloat16)
    y = ops.merge_heads(o.cuda(), B, H).cpu()
    ref = o.reshape(B, H, S, 128).permute(0, 2, 1, 3).reshape(B * S, H * 128)
    assert torch.equal(y, ref)


def _attention_ref(q, k, v, scale):
    """float64 causal attention on bf16 inputs [BH, S, D]; P rounded to bf16
    as the kernel feeds it to P @ V (normalised at the end)."""
    S = q.shape[1]
    s = (q.double() @ k.double().transpose(1, 2)) * scale
    s = s.masked_fill(~torch.ones((S, S), dtype=torch.bool).tril(), float("-inf"))
    return torch.softmax(s, dim=-1) @ v.double()


@pytest.mark.parametrize("B,H,S", [(1, 1, 128), (2, 3, 256), (1, 2, 1024), (1, 2, 384), (2, 2, 2048)])
def test_attention_causal_fused(B, H, S):
    ops = _ops()
    g = torch.Generator().manual_seed(B * 7 + H * 3 + S)
    q = torch.randn((B * H, S, 128), generator=g).to(torch.bfloat16)
    k = torch.randn((B * H, S, 128), generator=g).to(torch.bfloat16)
    v = torch.randn((B * H, S, 128), generator=g).to(torch.bfloat16)
    scale = 1.0 / math.sqrt(128)
    y = ops.attention_causal(q.cuda(), k.cuda(), v.cuda(), B, H, scale).float().cpu()
    ref = _attention_ref(q, k, v, scale).reshape(B, H, S, 128).permute(0, 2, 1, 3).reshape(B * S, H * 128)
    assert_rel_close(y.numpy(), ref.numpy(), BF16_RTOL, f"attention {B}x{H}x{S}")
    # Row 0 of every head attends to key 0 only: exactly v[0] (bf16).
    y0 = y.reshape(B, S, H, 128)[:, 0]
    assert torch.equal(y0, v.reshape(B, H, S, 128)[:, :, 0].float())


@pytest.mark.parametrize("B,H,S", [(2, 2, 512), (1, 4, 2048)])
def test_attention_row_blocks_bit_identical(B, H, S, monkeypatch):
    """32 query rows per wave (S % 256 == 0, the default there) and 16
    (MK_ATTN_RB=1): every row sees the same tiles in the same order, so the
    outputs are the same bits."""
    ops = _ops()
    g = torch.Generator().manual_seed(S + H)
    q, k, v = (torch.randn((B * H, S, 128), generator=g).to(torch.bfloat16).cuda() for _ in range(3))
    scale = 1.0 / math.sqrt(128)
    y2 = ops.attention_causal(q, k, v, B, H, scale)
    monkeypatch.setenv("MK_ATTN_RB", "1")
    y1 = ops.attention_causal(q, k, v, B, H, scale)
    torch.cuda.synchronize()
    assert torch.equal(y1.view(torch.int16), y2.view(torch.int16))


def test_attention_fused_vs_composed_accuracy():
    """The composed path (bf16 scores, GEMM / causal softmax / GEMM) and the
    one-pass kernel (f32 scores on chip) against float64: the composed path
    meets the tolerance norm-wise, and the one-pass kernel is at least as
    accurate (its only bf16 roundings are of P and of the output)."""
    ops = _ops()
    B, H, S = 2, 2, 256
    g = torch.Generator().manual_seed(11)
    q, k, v = (torch.randn((B * H, S, 128), generator=g).to(torch.bfloat16) for _ in range(3))
    scale = 1.0 / math.sqrt(128)
    fused = ops.attention_causal(q.cuda(), k.cuda(), v.cuda(), B, H, scale).double().cpu()
    s = ops.gemm_bf16(q.cuda(), k.transpose(1, 2).contiguous().cuda())
    p = ops.softmax_causal(s, scale)
    comp = ops.merge_heads(ops.gemm_bf16(p, v.cuda()), B, H).double().cpu()
    ref = _attention_ref(q, k, v, scale).reshape(B, H, S, 128).permute(0, 2, 1, 3).reshape(B * S, H * 128)
    err_c = float((comp - ref).abs().max() / ref.abs().max())
    err_f = float((fused - ref).abs().max() / ref.abs().max())
    assert err_c <= BF16_RTOL, err_c
    assert err_f <= err_c, (err_f, err_c)


def test_decoder_kernels_reject_bad_shapes():
    ops = _ops()
    from mi355x._lib import MKError
    qkv = torch.zeros((2 * 96, 3 * 128), dtype=torch.bfloat16, device="cuda")
    cos = torch.zeros((96, 64), dtype=torch.float32, device="cuda")
    with pytest.raises(MKError):
        ops.rope_qkv_split(qkv, cos, cos, 2, 96, 1, 128)  # S % 64 != 0
    with pytest.raises(MKError):
        ops.softmax_causal(torch.zeros((1, 12, 12), dtype=torch.bfloat16, device="cuda"), 1.0)  # S % 8
    z = torch.zeros((1, 192, 128), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(MKError):
        ops.attention_causal(z, z, z, 1, 1, 1.0)  # S % 128 != 0
    z = torch.zeros((1, 128, 128), dtype=torch.bfloat16, device="cuda")
    for bad in (0.0, -0.125, float("inf"), float("nan")):  # the kernel scales after its row max
        with pytest.raises(MKError):
            ops.attention_causal(z, z, z, 1, 1, bad)


# ---------------------------------------------------------------------------
# Whole decoder forward
# ---------------------------------------------------------------------------
def _deq(w):
    """int4 g64 weight -> f32 [K, N], each weight rounded to bf16 once (the
    many-row quantized paths do the same)."""
    p = w.packed.cpu()
    q = torch.empty((p.shape[0] * 2, p.shape[1]), dtype=torch.float32)
    q[0::2] = (p & 15).float()
    q[1::2] = (p >> 4).float()
    s = w.scale.cpu().float().repeat_interleave(64, 0)
    z = w.zero.cpu().float().repeat_interleave(64, 0)
    return _bf((q - z) * s)


def _rms(x, g, eps):
    return x * torch.rsqrt((x * x).mean(-1, keepdim=True) + eps) * g


def reference_forward(cfg, weights, x0, cos, sin):
    B, S, H, D = cfg.batch, cfg.seq, cfg.heads, cfg.head_dim
    x = x0.float()
    mask = torch.ones((S, S), dtype=torch.bool).tril()
    for lw in weights:
        h = _bf(_rms(x, lw.g_attn.cpu().float(), cfg.eps))
        qkv = _bf(h @ _deq(lw.w_qkv)).reshape(B, S, 3, H, D).permute(2, 0, 3, 1, 4)
        q = _bf(_rope_ref(qkv[0], cos, sin))
        k = _bf(_rope_ref(qkv[1], cos, sin))
        v = qkv[2]
        s = _bf(q @ k.transpose(-1, -2))
        p = torch.softmax((s * (1.0 / math.sqrt(D))).masked_fill(~mask, float("-inf")), dim=-1)
        o = _bf(_bf(p) @ v)
        attn = o.permute(0, 2, 1, 3).reshape(B * S, H * D)
        x = _bf(x + _bf(attn @ _deq(lw.w_o)))
        h = _bf(_rms(x, lw.g_mlp.cpu().float(), cfg.eps))
        gt = _bf(h @ _deq(lw.w_gate))
        up = _bf(h @ _deq(lw.w_up))
        act = _bf(_bf(gt * _bf(torch.sigmoid(gt))) * up)
        x = _bf(x + _bf(act @ _deq(lw.w_down)))
    return x


@pytest.mark.parametrize("attention", ["fused", "composed"])
def test_decoder_forward_matches_reference(attention):
    need_gpu()
    from mi355x import decoder
    cfg = decoder.DecoderConfig(layers=2, hidden=256, heads=2, head_dim=128, ffn=512, batch=2, seq=128)
    weights = decoder.init_weights(cfg, seed=3)
    cos, sin = decoder.rope_tables(cfg)
    buf = decoder.Buffers(cfg, attention=attention)
    x0 = torch.randn((cfg.tokens, cfg.hidden), generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    buf.x.copy_(x0.cuda())
    y = decoder.forward(cfg, weights, buf, cos, sin).float().cpu()
    ref = reference_forward(cfg, weights, x0, cos.cpu(), sin.cpu())
    assert torch.isfinite(y).all()
    assert_rel_close(y.numpy(), ref.numpy(), BF16_RTOL, "decoder forward")


@pytest.mark.parametrize("seq", [128, 512])
def test_decoder_fused_epilogues_bit_identical(seq):
    """Residual adds and SwiGLU fused into the projections' stores give the
    same bits as the separate products and elementwise programs.  At 1024
    tokens the gate and up projections are one paired product; at 256 the
    fused form falls back to two."""
    need_gpu()
    from mi355x import decoder, ops
    cfg = decoder.DecoderConfig(layers=2, hidden=256, heads=2, head_dim=128, ffn=512, batch=2, seq=seq)
    assert ops.int4_swiglu_pairs_supported(cfg.tokens, cfg.hidden, 2 * cfg.ffn) == (seq == 512)
    weights = decoder.init_weights(cfg, seed=6)
    cos, sin = decoder.rope_tables(cfg)
    x0 = torch.randn((cfg.tokens, cfg.hidden)).to(torch.bfloat16).cuda()
    outs = []
    for fuse in (True, False):
        buf = decoder.Buffers(cfg, fuse_epilogues=fuse)
        buf.x.copy_(x0)
        outs.append(decoder.forward(cfg, weights, buf, cos, sin).clone())
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])


def test_decoder_forward_graph_replays_match_eager():
    """A captured forward replays to the eager result (fresh input each time)."""
    need_gpu()
    from mi355x import decoder
    cfg = decoder.DecoderConfig(layers=1, hidden=256, heads=2, head_dim=128, ffn=512, batch=1, seq=128)
    weights = decoder.init_weights(cfg, seed=4)
    cos, sin = decoder.rope_tables(cfg)
    buf = decoder.Buffers(cfg)
    x0 = torch.randn((cfg.tokens, cfg.hidden)).to(torch.bfloat16).cuda()
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        buf.x.copy_(x0)
        eager = decoder.forward(cfg, weights, buf, cos, sin).clone()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        decoder.forward(cfg, weights, buf, cos, sin)
    for _ in range(3):
        buf.x.copy_(x0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(buf.x, eager)
