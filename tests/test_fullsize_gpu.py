"""Every form bench.py times, at the full size it times it, against the CPU
oracle.

* quantized matmul: int4 g64 and int8 per-channel at M = 1, 16, 256, 4096
  with K = 4096, N = 14336 (the workload's sweep), through the same C-ABI
  calls the bench makes.  Rows are checked directly against the oracle's C
  port (every row up to M = 256, a row sample at M = 4096), and every row at
  once through a column checksum r^T Y = (r^T X) W' with random signs r.
* bf16 GEMM 4096^3 with bf16 output (the headline GEMM): a row sample against
  float64, the bf16 output equal bit for bit to the f32-output run of the same
  kernel rounded to bf16, and a column checksum over every row.
* softmax / RMSNorm / argmax / the 6-op chain on X [8192, 8192] ~ N(0, 2) in
  f32 and bf16: every element against the oracle (argmax exactly).
* the plumbing program at n = 1024 through the runtime.
* the decoder: one full-size layer (hidden 2048, 16 x 128 heads, SwiGLU 8192,
  batch 4 x seq 2048, int4 g64 weights) against the oracle's layer
  restatement on a token subset, and the 4-layer forward bench.py times
  checked for finiteness and scale.

Tolerances are the workload's: bf16 rel 2e-2, f32 rel 1e-5, indices exact.
"""

import math

import numpy as np
import pytest

from _gpu import (BF16_RTOL, F32_RTOL, assert_rel_close, dev, dev_bf16, f32_sum_bound, host_bf16, host_bf16_bits,
                  need_gpu, torch)
from oracle import bf16 as obf
from oracle import cport, eltwise, quant, rowops

pytestmark = pytest.mark.gpu

K, N = 4096, 14336


def _ops():
    need_gpu()
    from mi355x import ops
    return ops


def _row_sample(M, n=96, seed=0):
    if M <= 256:
        return np.arange(M)
    rows = np.random.default_rng(seed).choice(np.arange(1, M - 1), size=n - 2, replace=False)
    return np.sort(np.concatenate([[0, M - 1], rows]))


def _checksum(y, x_f64, w_f64, seed, what):
    """r^T Y against (r^T X) W' for random signs r: every row of Y enters.
    Each bf16 output carries at most half an ulp (2^-8 relative) of rounding,
    so the difference per column is bounded by 4 * 2^-8 * sqrt(sum_m Y^2)
    (a 7-sigma bound for independent roundings)."""
    r = np.random.default_rng(seed).choice([-1.0, 1.0], size=y.shape[0])
    got = r @ y.astype(np.float64)
    ref = (r @ x_f64) @ w_f64
    noise = 4 * 2.0 ** -8 * np.sqrt(np.sum(y.astype(np.float64) ** 2, axis=0)) + 1e-6 * np.max(np.abs(ref))
    bad = np.abs(got - ref) > noise
    assert not bad.any(), f"{what}: checksum off in {int(bad.sum())} columns, worst {np.max(np.abs(got - ref)):.3e}"


@pytest.mark.parametrize("M", [1, 16, 256, 4096])
def test_int4_full_size(M):
    ops = _ops()
    print(f"[fullsize] int4 M={M} K={K} N={N}", flush=True)
    rng = np.random.default_rng(M)
    x, packed, s, z = quant.make_int4_case(rng, M, K, N)
    y = host_bf16(ops.int4_g64_matmul(dev_bf16(x), dev(packed), dev_bf16(s), dev(z)))
    torch.cuda.synchronize()
    rows = _row_sample(M)
    ref = cport.int4_g64_matmul(x[rows], packed, s, z)
    assert_rel_close(y[rows], ref, BF16_RTOL, f"int4 M={M}")
    if M >= 256:
        w = quant.int4_g64_dequant(packed, s, z, round_to_bf16=True).astype(np.float64)
        _checksum(y, obf.bf16_bits_to_f32(x).astype(np.float64), w, M, f"int4 M={M}")


@pytest.mark.parametrize("M", [1, 16, 256, 4096])
def test_int8_full_size(M):
    ops = _ops()
    print(f"[fullsize] int8 M={M} K={K} N={N}", flush=True)
    rng = np.random.default_rng(M + 1)
    x, w, s = quant.make_int8_case(rng, M, K, N)
    y = host_bf16(ops.int8_pc_matmul(dev_bf16(x), dev(w), dev(s)))
    torch.cuda.synchronize()
    rows = _row_sample(M)
    ref = cport.int8_pc_matmul(x[rows], w, s)
    assert_rel_close(y[rows], ref, BF16_RTOL, f"int8 M={M}")
    if M >= 256:
        wd = w.astype(np.float64) * s.astype(np.float64)[None, :]
        _checksum(y, obf.bf16_bits_to_f32(x).astype(np.float64), wd, M, f"int8 M={M}")


def test_gemm_bf16_4096_bf16_output():
    """The headline GEMM exactly as bench.py runs it (bf16 output)."""
    ops = _ops()
    M = Nn = Kk = 4096
    print("[fullsize] bf16 GEMM 4096^3, bf16 and f32 outputs", flush=True)
    rng = np.random.default_rng(4096)
    sc = 1.0 / np.sqrt(np.sqrt(Kk))
    a = obf.f32_to_bf16_bits((rng.standard_normal((M, Kk)) * sc).astype(np.float32))
    b = obf.f32_to_bf16_bits((rng.standard_normal((Kk, Nn)) * sc).astype(np.float32))
    ad, bd = dev_bf16(a), dev_bf16(b)
    c16 = host_bf16_bits(ops.gemm_bf16(ad, bd))
    c32 = ops.gemm_bf16(ad, bd, out_f32=True).cpu().numpy()
    torch.cuda.synchronize()
    # Same kernel, same accumulation: the bf16 store is the RNE rounding of
    # the f32 accumulator.
    assert np.array_equal(c16, obf.f32_to_bf16_bits(c32)), "bf16 output is not r(f32 output)"
    af = obf.bf16_bits_to_f32(a).astype(np.float64)
    bf = obf.bf16_bits_to_f32(b).astype(np.float64)
    rows = _row_sample(M, 64, seed=1)
    ref = af[rows] @ bf
    c = obf.bf16_bits_to_f32(c16)
    assert_rel_close(c[rows], ref, BF16_RTOL, "gemm 4096^3 bf16 out")
    assert_rel_close(c32[rows], ref, F32_RTOL, "gemm 4096^3 f32 out",
                     elem=f32_sum_bound(np.abs(af[rows]) @ np.abs(bf), Kk))
    _checksum(c, af, bf, 7, "gemm 4096^3 bf16 out")


@pytest.mark.parametrize("K_", [2048, 4096, 4128])
def test_gemm_bf16_pipelined_bf16_output(K_):
    """The pipelined kernel's LDS-staged bf16 store at K = 2048 / 4096 / 4128
    (both loop tails), every element against float64."""
    ops = _ops()
    rng = np.random.default_rng(K_)
    M, Nn = 512, 768
    sc = 1.0 / np.sqrt(np.sqrt(K_))
    a = obf.f32_to_bf16_bits((rng.standard_normal((M, K_)) * sc).astype(np.float32))
    b = obf.f32_to_bf16_bits((rng.standard_normal((K_, Nn)) * sc).astype(np.float32))
    print(f"[fullsize] pipelined GEMM bf16 out K={K_}", flush=True)
    c16 = host_bf16_bits(ops.gemm_bf16(dev_bf16(a), dev_bf16(b)))
    c32 = ops.gemm_bf16(dev_bf16(a), dev_bf16(b), out_f32=True).cpu().numpy()
    torch.cuda.synchronize()
    ref = obf.bf16_bits_to_f32(a).astype(np.float64) @ obf.bf16_bits_to_f32(b).astype(np.float64)
    assert_rel_close(obf.bf16_bits_to_f32(c16), ref, BF16_RTOL, f"pipelined bf16 K={K_}")
    assert np.array_equal(c16, obf.f32_to_bf16_bits(c32))


R = C = 8192


def _x(dt, seed):
    x = (np.random.default_rng(seed).standard_normal((R, C)) * np.sqrt(2.0)).astype(np.float32)
    if dt == "bf16":
        bits = obf.f32_to_bf16_bits(x)
        return bits, obf.bf16_bits_to_f32(bits), dev_bf16(bits)
    return x, x, dev(x)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_softmax_full_size(dt):
    ops = _ops()
    print(f"[fullsize] softmax {dt} 8192x8192", flush=True)
    raw, xf, xd = _x(dt, 11)
    y = ops.softmax(xd)
    torch.cuda.synchronize()
    if dt == "f32":
        assert_rel_close(y.cpu().numpy(), rowops.softmax(xf), F32_RTOL, "softmax f32 8192^2")
    else:
        ref = obf.bf16_bits_to_f32(rowops.softmax_bf16(raw))
        assert_rel_close(host_bf16(y), ref, BF16_RTOL, "softmax bf16 8192^2")


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_rmsnorm_full_size(dt):
    ops = _ops()
    print(f"[fullsize] rmsnorm {dt} 8192x8192", flush=True)
    raw, xf, xd = _x(dt, 12)
    g = np.random.default_rng(13).uniform(0.5, 1.5, C).astype(np.float32)
    if dt == "bf16":
        gb = obf.f32_to_bf16_bits(g)
        g, gd = obf.bf16_bits_to_f32(gb), dev_bf16(gb)
    else:
        gd = dev(g)
    y = ops.rmsnorm(xd, gd)
    torch.cuda.synchronize()
    out = y.cpu().numpy() if dt == "f32" else host_bf16(y)
    assert_rel_close(out, rowops.rmsnorm(xf, g), F32_RTOL if dt == "f32" else BF16_RTOL, f"rmsnorm {dt}")


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_argmax_full_size(dt):
    ops = _ops()
    print(f"[fullsize] argmax {dt} 8192x8192", flush=True)
    raw, xf, xd = _x(dt, 14)
    y = ops.argmax(xd).cpu().numpy()
    np.testing.assert_array_equal(y, rowops.argmax(xf))
    if dt == "f32":
        np.testing.assert_array_equal(y, cport.argmax_f32(xf))


# bench.py's 6-op chain as a register program (slots: 0 = x).
CHAIN6_PROGRAM = [("LOAD", 0, 0, 0, 0, 0.0), ("CONST", 1, 0, 0, 0, 1.5), ("MUL", 2, 0, 1, 0, 0.0),
                  ("CONST", 1, 0, 0, 0, 0.5), ("ADD", 3, 2, 1, 0, 0.0), ("EXP", 4, 3, 0, 0, 0.0),
                  ("LOG1P", 5, 4, 0, 0, 0.0), ("MAX", 6, 5, 0, 0, 0.0), ("CONST", 1, 0, 0, 0, 0.0),
                  ("CMP_GT", 7, 0, 1, 0, 0.0), ("SELECT", 8, 7, 6, 3, 0.0)]


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_chain6_full_size(dt):
    ops = _ops()
    print(f"[fullsize] chain6 {dt} 8192x8192", flush=True)
    raw, xf, xd = _x(dt, 15)
    y = ops.elementwise(CHAIN6_PROGRAM, [xd], out_slot=8)
    torch.cuda.synchronize()
    out = y.cpu().numpy() if dt == "f32" else host_bf16(y)
    ref = eltwise.evaluate(eltwise.CHAIN6, [xf], dt)
    assert_rel_close(out, ref, F32_RTOL if dt == "f32" else BF16_RTOL, f"chain6 {dt}")


def test_plumbing_full_size():
    """tanh(A @ B).sum(axis=1), A, B f32 [1024, 1024] ~ N(0, 1) from seed 0,
    through the runtime (StableHLO text -> compile -> execute)."""
    need_gpu()
    from mi355x import programs as P
    from mi355x import runtime as rt
    n = 1024
    rng = np.random.default_rng(0)
    a = rng.standard_normal((n, n)).astype(np.float32)
    b = rng.standard_normal((n, n)).astype(np.float32)
    print("[fullsize] plumbing n=1024", flush=True)
    client = rt.Client()
    try:
        exe = client.compile(P.plumbing(n))
        bufs = [client.buffer(a), client.buffer(b)]
        (o,), done = exe.execute(bufs)
        done.wait()
        y = o.to_numpy()
        for t in bufs + [o]:
            t.close()
        exe.close()
    finally:
        client.close()
    ref = np.tanh(a.astype(np.float64) @ b.astype(np.float64)).sum(axis=1)
    # The stated f32 measure, normwise (max|y - ref| / max|ref| <= 1e-5).
    assert_rel_close(y, ref, F32_RTOL, "plumbing n=1024", elem=False)


# ---------------------------------------------------------------- decoder

def _host_weight(w):
    return (w.packed.cpu().numpy(), host_bf16_bits(w.scale), w.zero.cpu().numpy())


def test_decoder_layer_full_config_vs_oracle():
    """Layer 0 of the workload's decoder at its full size on the GPU, checked
    on batch elements 0 and 3 at 24 positions (the first and last, tile
    boundaries, random ones):

    * end to end against the oracle's layer from the same input, at the
      workload's bf16 measure per token (max |err| / max |ref| over the row);
    * stage by stage, each stage against the oracle applied to the GPU's own
      input to that stage (attention block, output projection + residual,
      SwiGLU MLP activation, down projection + residual), elementwise.  One
      bf16 ulp at an early stage moves later bf16 roundings, so the end-to-end
      comparison cannot be elementwise; the stages can."""
    need_gpu()
    from mi355x import decoder
    from oracle import decoder as odec

    cfg = decoder.DecoderConfig()
    print(f"[fullsize] decoder layer {cfg}", flush=True)
    weights = decoder.init_weights(cfg, seed=0)
    cos, sin = decoder.rope_tables(cfg)
    buf = decoder.Buffers(cfg)
    gen = torch.Generator("cuda").manual_seed(0)
    buf.x.copy_(torch.randn((cfg.tokens, cfg.hidden), device="cuda", generator=gen).to(torch.bfloat16))
    x0 = host_bf16(buf.x).reshape(cfg.batch, cfg.seq, cfg.hidden)
    taps = {}
    decoder.layer_forward(cfg, weights[0], buf, cos, sin, taps=taps)
    torch.cuda.synchronize()
    shape = (cfg.batch, cfg.seq, -1)
    out = host_bf16(buf.x).reshape(shape)
    g = {k: host_bf16(v).reshape(shape) for k, v in taps.items()}
    lw = weights[0]
    w = {"g_attn": host_bf16_bits(lw.g_attn), "g_mlp": host_bf16_bits(lw.g_mlp),
         "w_qkv": _host_weight(lw.w_qkv), "w_o": _host_weight(lw.w_o), "w_gate": _host_weight(lw.w_gate),
         "w_up": _host_weight(lw.w_up), "w_down": _host_weight(lw.w_down)}
    rng = np.random.default_rng(5)
    fixed = [0, 1, 2, 63, 64, 127, 128, 129, 1023, 1024, 2046, 2047]
    pos = np.unique(np.concatenate([fixed, rng.integers(3, cfg.seq - 2, size=12)]))
    for b in (0, cfg.batch - 1):
        ref = odec.layer_rows(x0[b], pos, w, cfg.heads, cfg.head_dim, cfg.eps, cfg.rope_base, parts=True)
        o, r = out[b, pos].astype(np.float64), ref["out"].astype(np.float64)
        row_rel = np.abs(o - r).max(axis=1) / np.abs(r).max(axis=1)
        print(f"[fullsize] decoder batch {b}: worst row rel err {row_rel.max():.3e}", flush=True)
        assert row_rel.max() <= BF16_RTOL, f"batch {b}: worst row rel err {row_rel.max():.3e}"
        # stage by stage, elementwise
        assert_rel_close(g["attn"][b, pos], ref["attn"], BF16_RTOL, f"attention block, batch {b}")
        x1 = odec.output_residual(x0[b, pos], g["attn"][b, pos], w["w_o"])["x1"]
        assert_rel_close(g["x1"][b, pos], x1, BF16_RTOL, f"output projection + residual, batch {b}")
        act = odec.mlp_act(g["x1"][b, pos], w, cfg.eps)
        assert_rel_close(g["act"][b, pos], act, BF16_RTOL, f"SwiGLU activation, batch {b}")
        fin = odec.down_residual(g["x1"][b, pos], g["act"][b, pos], w["w_down"])["out"]
        assert_rel_close(out[b, pos], fin, BF16_RTOL, f"down projection + residual, batch {b}")


def test_decoder_forward_full_config_is_finite():
    """The 4-layer forward bench.py times: finite, and the residual stream's
    scale stays in the range a random-init layer stack gives (it grows by the
    projections' outputs, not by orders of magnitude)."""
    need_gpu()
    from mi355x import decoder

    cfg = decoder.DecoderConfig()
    print("[fullsize] decoder 4-layer forward", flush=True)
    weights = decoder.init_weights(cfg, seed=0)
    cos, sin = decoder.rope_tables(cfg)
    buf = decoder.Buffers(cfg)
    gen = torch.Generator("cuda").manual_seed(0)
    buf.x.copy_(torch.randn((cfg.tokens, cfg.hidden), device="cuda", generator=gen).to(torch.bfloat16))
    decoder.forward(cfg, weights, buf, cos, sin)
    torch.cuda.synchronize()
    y = buf.x.float()
    assert bool(torch.isfinite(y).all())
    std = float(y.std())
    assert 0.5 < std < 1e3, std
    # every token changed
    assert int((y.abs().sum(dim=1) == 0).sum()) == 0
