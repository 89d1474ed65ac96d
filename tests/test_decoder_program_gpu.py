"""GPU parity of the Llama-style decoder layer compiled from its StableHLO
(mi355x/programs.decoder_layer: the layer as jax.jit lowers it, the
reference's transformer-layer benchmark, benchmarks/vs_cpu.py:603-626)
through the runtime's compile -> execute path, against the float64 oracle
layer (oracle/decoder.py) at the workload's bf16 tolerance per token.

The program rounds where jax's bf16 ops round (RMSNorm's x * x, the
scores, softmax's exp and quotient) and the oracle rounds once per block,
so the comparison is the bf16 measure max |err| / max |ref| per row, not an
elementwise one.

The oracle's weight convention follows the route the plan takes for the
layer's row count: below 128 rows the streaming dequant-matmul kernels apply
(q - z) * s exactly (exact_weights=True); from 128 rows the many-row kernels
(the fused qgemm kernel, or the dequantise-then-GEMM pass) round each
dequantised weight to bf16 once, as XLA:CPU rounds a bf16 (q - z) * s.  The
two conventions alone move a 4-layer stack by up to ~4e-2 per row, so the
oracle must use the one the kernels use."""

QMM_MANY_ROWS = 128  # qmatmul.hip kQgMinRows: from here the dequantised weight is rounded to bf16


def _exact_route(rows):
    return rows < QMM_MANY_ROWS

import numpy as np
import pytest

from mi355x import programs as P
from mi355x import runtime as rt
from mi355x import synthetic
from oracle import decoder as odec
from oracle.bf16 import bf16_bits_to_f32, round_bf16

from _gpu import BF16_RTOL

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def client():
    try:
        c = rt.Client()
    except rt.PluginError as e:
        pytest.fail(f"GPU test selected but the runtime has no device: {e}")
    yield c
    c.close()


def _run_layer(client, B, S, hidden, H, D, F, seed):
    """Compile the layer's StableHLO, run it once on a synthetic case;
    returns (output [B, S, hidden] as float32, x bits, weights, plan text)."""
    x, w, cos, sin = synthetic.decoder_layer_case(np.random.default_rng(seed), B, S, hidden, H, D, F)
    text = P.decoder_layer(B, S, hidden, H, D, F)
    print(f"[decoder-program] B={B} S={S} hidden={hidden} H={H} D={D} F={F}", flush=True)
    exe = client.compile(text)
    args = [client.buffer(a, rt.BF16) if is_bf16 else client.buffer(a)
            for a, is_bf16 in synthetic.decoder_layer_arguments(x, w, cos, sin)]
    outs, done = exe.execute(args)
    done.wait()
    (y,) = [o.to_numpy() for o in outs]
    plan = exe.plan
    for b in args + outs:
        b.close()
    exe.close()
    return bf16_bits_to_f32(y).reshape(B, S, hidden), x, w, plan


def _check_rows(y, x, w, B, S, hidden, H, D, pos, batches):
    x3 = bf16_bits_to_f32(x).reshape(B, S, hidden)
    for b in batches:
        ref = odec.layer_rows(x3[b], pos, w, H, D, exact_weights=_exact_route(B * S))
        o = y[b, pos].astype(np.float64)
        assert np.isfinite(o).all()
        row_rel = np.abs(o - ref).max(axis=1) / np.abs(ref).max(axis=1)
        print(f"[decoder-program] batch {b}: worst row rel err {row_rel.max():.3e}", flush=True)
        assert row_rel.max() <= BF16_RTOL, (b, pos[int(row_rel.argmax())], row_rel.max())


@pytest.mark.parametrize("fused", [True, False], ids=["decoder-kernels", "op-by-op"])
@pytest.mark.parametrize("B,S,hidden,H,D,F", [(1, 64, 128, 2, 64, 256), (2, 128, 256, 2, 128, 512)])
def test_decoder_program_small_vs_oracle(client, monkeypatch, B, S, hidden, H, D, F, fused):
    if not fused:
        monkeypatch.setenv("MK_PLAN_DECODER_FUSION", "0")
    y, x, w, plan = _run_layer(client, B, S, hidden, H, D, F, seed=B * 1000 + S)
    # the projections and norms run on their kernels; RoPE and attention on
    # the decoder kernels where their shapes allow (head_dim 128, S % 128)
    assert plan.count("int4_g64_matmul") == 5 and plan.count("rmsnorm") == 2
    if fused and D == 128:
        assert "rope_qkv_split" in plan and "attention_causal" in plan and "softmax" not in plan
    else:
        assert "softmax" in plan and plan.count("gemm_bf16") == 2 and "attention_causal" not in plan
    _check_rows(y, x, w, B, S, hidden, H, D, np.arange(S), range(B))


@pytest.mark.parametrize("fused", [True, False], ids=["decoder-kernels", "op-by-op"])
def test_decoder_program_full_config_vs_oracle(client, monkeypatch, fused):
    """The workload's decoder layer (hidden 2048, 16 x 128 heads, SwiGLU 8192,
    batch 4 x 2048 tokens) compiled from StableHLO, checked on batch elements
    0 and 3 at 16 positions (first and last rows, tile boundaries, random)."""
    if not fused:
        monkeypatch.setenv("MK_PLAN_DECODER_FUSION", "0")
    B, S, hidden, H, D, F = 4, 2048, 2048, 16, 128, 8192
    y, x, w, plan = _run_layer(client, B, S, hidden, H, D, F, seed=7)
    assert ("attention_causal" in plan) == fused
    assert np.isfinite(y).all()
    rng = np.random.default_rng(3)
    pos = np.unique(np.concatenate([[0, 1, 63, 64, 1023, 2047], rng.integers(2, S - 1, size=10)]))
    _check_rows(y, x, w, B, S, hidden, H, D, pos, (0, B - 1))


@pytest.mark.parametrize("fused", [True, False], ids=["decoder-kernels", "op-by-op"])
@pytest.mark.parametrize("transpose_k", [True, False], ids=["k-transposed", "k-last-axis"])
def test_causal_attention_program_vs_oracle(client, monkeypatch, transpose_k, fused):
    """softmax(where(causal, q k^T / sqrt(D), -inf)) @ v from its StableHLO,
    against the oracle's causal attention per (b, h) row block, at the bf16
    measure per row; row 0 sees only key 0, so it must equal v[0] to bf16
    rounding."""
    if not fused:
        monkeypatch.setenv("MK_PLAN_DECODER_FUSION", "0")
    B, H, S, D = 2, 3, 256, 128
    rng = np.random.default_rng(11)
    q, k, v = (synthetic.bf16_bits(rng.standard_normal((B, H, S, D)).astype(np.float32)) for _ in range(3))
    print(f"[decoder-program] attention B={B} H={H} S={S} fused={fused} transpose_k={transpose_k}", flush=True)
    exe = client.compile(P.causal_attention(B, H, S, D, transpose_k=transpose_k))
    assert ("attention_causal" in exe.plan) == fused
    args = [client.buffer(a, rt.BF16) for a in (q, k, v)]
    outs, done = exe.execute(args)
    done.wait()
    y = bf16_bits_to_f32(outs[0].to_numpy()).astype(np.float64)  # [B, S, H, D]
    for b_ in args + outs:
        b_.close()
    exe.close()
    qf, kf, vf = (bf16_bits_to_f32(a).astype(np.float64) for a in (q, k, v))
    scale = float(bf16_bits_to_f32(synthetic.bf16_bits(np.array([D ** -0.5], np.float32)))[0])
    pos = np.arange(S)
    for b_ in range(B):
        for h in range(H):
            ref = odec.attention_causal_rows(qf[b_, h], pos, kf[b_, h], vf[b_, h], scale)
            got = y[b_, :, h]
            row_rel = np.abs(got - ref).max(axis=1) / np.abs(ref).max(axis=1)
            assert row_rel.max() <= BF16_RTOL, (b_, h, row_rel.max())
            assert np.allclose(got[0], vf[b_, h, 0], rtol=2 ** -7, atol=0)


def test_store_epilogues_are_bit_identical(client, monkeypatch):
    """The planner folds the residual adds and silu(g) * u into the
    dequant-matmul's store; the layer's output must equal, bit for bit, the
    plan that runs them as elementwise programs."""
    B, S, hidden, H, D, F = 2, 128, 256, 2, 128, 512
    monkeypatch.setenv("MK_PLAN_EPILOGUES", "all")
    y1, _, _, plan1 = _run_layer(client, B, S, hidden, H, D, F, seed=21)
    monkeypatch.setenv("MK_PLAN_EPILOGUES", "0")
    y0, _, _, plan0 = _run_layer(client, B, S, hidden, H, D, F, seed=21)
    assert "epilogue" in plan1 and "epilogue" not in plan0
    assert np.array_equal(y1.view(np.uint32), y0.view(np.uint32))


@pytest.mark.parametrize("op", ["add", "swiglu"])
@pytest.mark.parametrize("fmt,M", [("int4", 16), ("int4", 256), ("int4", 1024), ("int8", 16), ("int8", 1024)])
def test_qmm_epilogue_programs_bit_identical(client, monkeypatch, fmt, M, op):
    """aux + qmm(x, W) and silu(aux) * qmm(x, W) at every quantized route
    (streaming, fused many-row, dequantise-then-GEMM): the epilogue plan
    against the two-step plan, bit for bit."""
    K, N = 256, 512
    rng = np.random.default_rng(M + len(op))
    if fmt == "int4":
        x, p, s_, z = synthetic.int4_case(rng, M, K, N)
        w = [(x, rt.BF16), (p, None), (s_, rt.BF16), (z, None)]
    else:
        x, w8, s8 = synthetic.int8_case(rng, M, K, N)
        w = [(x, rt.BF16), (w8, None), (s8, None)]
    aux = synthetic.bf16_bits(rng.standard_normal((M, N)).astype(np.float32))
    text = P.qmm_epilogue(M, K, N, fmt, op)
    outs = []
    for env in ("all", "0"):
        monkeypatch.setenv("MK_PLAN_EPILOGUES", env)
        print(f"[decoder-program] {fmt} M={M} {op} epilogues={env}", flush=True)
        exe = client.compile(text)
        assert ("epilogue" in exe.plan) == (env == "all")
        args = [client.buffer(aux, rt.BF16)] + [client.buffer(a, t) if t else client.buffer(a) for a, t in w]
        res, done = exe.execute(args)
        done.wait()
        outs.append(res[0].to_numpy())
        for b_ in args + res:
            b_.close()
        exe.close()
    assert np.array_equal(outs[0], outs[1])


def test_decoder_stack_vs_oracle(client):
    """Two layers as one jitted function (programs.decoder_stack), against
    the oracle's layer applied twice on every row, each oracle layer fed the
    oracle's previous output."""
    B, S, hidden, H, D, F, L = 2, 128, 256, 2, 128, 512, 2
    x, ws, cos, sin = synthetic.decoder_stack_case(np.random.default_rng(31), L, B, S, hidden, H, D, F)
    print(f"[decoder-program] stack L={L} B={B} S={S}", flush=True)
    exe = client.compile(P.decoder_stack(L, B, S, hidden, H, D, F))
    assert exe.plan.count("attention_causal") == L
    args = [client.buffer(a, rt.BF16) if is_bf16 else client.buffer(a)
            for a, is_bf16 in synthetic.decoder_stack_arguments(x, ws, cos, sin)]
    outs, done = exe.execute(args)
    done.wait()
    y = bf16_bits_to_f32(outs[0].to_numpy()).reshape(B, S, hidden).astype(np.float64)
    for b_ in args + outs:
        b_.close()
    exe.close()
    x3 = bf16_bits_to_f32(x).reshape(B, S, hidden)
    pos = np.arange(S)
    for b in range(B):
        ref = x3[b].astype(np.float64)
        for w in ws:
            ref = odec.layer_rows(ref, pos, w, H, D, exact_weights=_exact_route(B * S))
        row_rel = np.abs(y[b] - ref).max(axis=1) / np.abs(ref).max(axis=1)
        print(f"[decoder-program] stack batch {b}: worst row rel err {row_rel.max():.3e}", flush=True)
        assert row_rel.max() <= BF16_RTOL, (b, row_rel.max())


@pytest.mark.parametrize("fmt", ["int4", "int8"])
def test_swiglu_pair_program_bit_identical_and_vs_oracle(client, monkeypatch, fmt):
    """silu(x @ Wg) * (x @ Wu) from its StableHLO at a many-row shape: the
    paired plan (one step) against the two-product plan, bit for bit, and
    against the float64 oracle at the bf16 tolerance."""
    from oracle import quant
    M, K, N = 1024, 512, 256
    rng = np.random.default_rng(41 + len(fmt))
    if fmt == "int4":
        x, pg, sg, zg = synthetic.int4_case(rng, M, K, N)
        _, pu, su, zu = synthetic.int4_case(rng, M, K, N)
        args = [(x, rt.BF16), (pg, None), (sg, rt.BF16), (zg, None), (pu, None), (su, rt.BF16), (zu, None)]
        g, _ = quant.int4_g64_matmul(x, pg, sg, zg)
        u, _ = quant.int4_g64_matmul(x, pu, su, zu)
    else:
        x, wg, sg = synthetic.int8_case(rng, M, K, N)
        _, wu, su = synthetic.int8_case(rng, M, K, N)
        args = [(x, rt.BF16), (wg, None), (sg, None), (wu, None), (su, None)]
        g, _ = quant.int8_pc_matmul(x, wg, sg)
        u, _ = quant.int8_pc_matmul(x, wu, su)
    text = P.swiglu_mlp(M, K, N, fmt)
    outs = []
    for env in ("1", "0"):
        monkeypatch.setenv("MK_PLAN_PAIRS", env)
        print(f"[decoder-program] swiglu pair {fmt} M={M} K={K} N={N} pairs={env}", flush=True)
        exe = client.compile(text)
        assert ("swiglu pair" in exe.plan) == (env == "1")
        bufs = [client.buffer(a, t) if t else client.buffer(a) for a, t in args]
        res, done = exe.execute(bufs)
        done.wait()
        outs.append(res[0].to_numpy())
        for b_ in bufs + res:
            b_.close()
        exe.close()
    assert np.array_equal(outs[0], outs[1])
    ref = g / (1.0 + np.exp(-g)) * u
    y = bf16_bits_to_f32(outs[0]).astype(np.float64)
    row_rel = np.abs(y - ref).max(axis=1) / np.abs(ref).max(axis=1)
    assert row_rel.max() <= BF16_RTOL, row_rel.max()


def _hand_fused_weights(ws):
    """The synthetic layer weights (numpy bits) as the hand-fused forward's
    LayerWeights on cuda:0."""
    import torch
    from mi355x import decoder

    def bf16(bits):
        return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).cuda()

    def int4(w):
        packed, s, z = w
        return decoder.Int4Weight(torch.from_numpy(packed).cuda(), bf16(s), torch.from_numpy(z).cuda())

    layers = []
    for w in ws:
        lw = decoder.LayerWeights(g_attn=bf16(w["g_attn"]), w_qkv=int4(w["w_qkv"]), w_o=int4(w["w_o"]),
                                  g_mlp=bf16(w["g_mlp"]), w_gate=int4(w["w_gate"]), w_up=int4(w["w_up"]),
                                  w_down=int4(w["w_down"]))
        lw.w_gateup = decoder.interleave_int4(lw.w_gate, lw.w_up)
        layers.append(lw)
    return layers


def _oracle_stack(x_rows, ws, H, D, exact):
    """The oracle's layer stack on one sequence prefix."""
    ref = x_rows
    for w in ws:
        ref = odec.layer_rows(ref, np.arange(len(x_rows)), w, H, D, exact_weights=exact)
    return ref


def _row_measures(got, ref):
    """(per-row max measure max|err|/max|ref|, per-row relative L2, normwise
    over the whole block)."""
    d = got - ref
    return (np.abs(d).max(axis=1) / np.abs(ref).max(axis=1),
            np.linalg.norm(d, axis=1) / np.linalg.norm(ref, axis=1),
            np.abs(d).max() / np.abs(ref).max())


def test_decoder_stack_full_config(client):
    """The 4-layer forward bench.py times: programs.decoder_stack(4, 4, 2048,
    2048, 16, 128, 8192) compiled from its StableHLO and run once.

    * every output finite and every token changed by the stack;
    * batches 0 and 3 against the oracle's 4 layers on the position prefix
      [0, P) (causal attention makes a prefix self-contained, so the oracle
      needs only P rows per layer), and the hand-fused forward
      (mi355x/decoder.forward) on the same weights held to the same checks:
      - normwise over the block, max|err| / max|ref| <= 2e-2 (the workload's
        bf16 measure);
      - per row (max measure and relative L2) within the oracle's own
        sensitivity.  This random-init stack amplifies perturbations about
        11x per layer: moving 1 % of the input elements by one bf16 ulp moves
        the oracle's 4-layer output by ~2e-2 per row (median) and ~4e-2
        (worst), so any evaluation that rounds to bf16 at other points than
        the oracle carries that much.  The test measures this spread live
        (the oracle run twice, on x and on x with 1 % of its elements one ulp
        up) and asserts each GPU row within max(2e-2, the spread's worst
        row);
    * every row of the program within twice that bound of the hand-fused
      forward (each is within the bound of the exact stack; triangle
      inequality)."""
    import torch
    from mi355x import decoder

    L, B, S, hidden, H, D, F = 4, 4, 2048, 2048, 16, 128, 8192
    P_ = 192
    x, ws, cos, sin = synthetic.decoder_stack_case(np.random.default_rng(43), L, B, S, hidden, H, D, F)
    print(f"[decoder-program] full stack L={L} B={B} S={S} hidden={hidden}", flush=True)
    exe = client.compile(P.decoder_stack(L, B, S, hidden, H, D, F))
    assert exe.plan.count("attention_causal") == L
    args = [client.buffer(a, rt.BF16) if is_bf16 else client.buffer(a)
            for a, is_bf16 in synthetic.decoder_stack_arguments(x, ws, cos, sin)]
    outs, done = exe.execute(args)
    done.wait()
    y = bf16_bits_to_f32(outs[0].to_numpy()).reshape(B, S, hidden).astype(np.float64)
    for b_ in args + outs:
        b_.close()
    exe.close()
    x3 = bf16_bits_to_f32(x).reshape(B, S, hidden).astype(np.float64)
    assert np.isfinite(y).all()
    changed = np.any(y != x3, axis=2)
    assert changed.all(), f"{int((~changed).sum())} tokens unchanged by the stack"

    print("[decoder-program] full stack: hand-fused forward on the same weights", flush=True)
    cfg = decoder.DecoderConfig(layers=L, hidden=hidden, heads=H, head_dim=D, ffn=F, batch=B, seq=S)
    buf = decoder.Buffers(cfg)
    buf.x.copy_(torch.from_numpy(x.view(np.int16)).view(torch.bfloat16).reshape(B * S, hidden).cuda())
    decoder.forward(cfg, _hand_fused_weights(ws), buf, torch.from_numpy(cos).cuda(), torch.from_numpy(sin).cuda())
    torch.cuda.synchronize()
    hf = buf.x.float().cpu().numpy().reshape(B, S, hidden).astype(np.float64)

    exact = _exact_route(B * S)
    bounds = []
    for b in (0, B - 1):
        print(f"[decoder-program] full stack: oracle, batch {b}, positions [0, {P_})", flush=True)
        x0 = x3[b, :P_]
        ref = _oracle_stack(x0, ws, H, D, exact)
        up = np.random.default_rng(100 + b).random(x0.shape) < 0.01
        xp = x0.copy()
        xp[up] = round_bf16(x0[up] * (1 + 2.0 ** -7))
        sp_max, sp_l2, _ = _row_measures(_oracle_stack(xp, ws, H, D, exact), ref)
        bound_max, bound_l2 = max(BF16_RTOL, sp_max.max()), max(BF16_RTOL, sp_l2.max())
        bounds.append(bound_max)
        print(f"[decoder-program] oracle spread (1% of inputs +1 ulp), batch {b}: per-row max measure worst "
              f"{sp_max.max():.3e} median {np.median(sp_max):.3e}; L2 worst {sp_l2.max():.3e}", flush=True)
        for name, got in (("program", y), ("hand-fused", hf)):
            rr, l2, nw = _row_measures(got[b, :P_], ref)
            print(f"[decoder-program] full stack {name} vs oracle, batch {b}: normwise {nw:.3e}; per-row max "
                  f"measure worst {rr.max():.3e} median {np.median(rr):.3e} (bound {bound_max:.3e}); per-row L2 "
                  f"worst {l2.max():.3e} (bound {bound_l2:.3e})", flush=True)
            assert nw <= BF16_RTOL, (name, b, nw)
            assert rr.max() <= bound_max, (name, b, int(rr.argmax()), rr.max())
            assert l2.max() <= bound_l2, (name, b, int(l2.argmax()), l2.max())

    row_rel = np.abs(y - hf).max(axis=2) / np.abs(hf).max(axis=2)
    print(f"[decoder-program] full stack vs hand-fused, all {row_rel.size} rows: per-row max measure worst "
          f"{row_rel.max():.3e}, median {np.median(row_rel):.3e} (bound {2 * max(bounds):.3e})", flush=True)
    assert row_rel.max() <= 2 * max(bounds), (np.unravel_index(int(row_rel.argmax()), row_rel.shape), row_rel.max())


def _run_program(client, text, arrays):
    args = [client.buffer(a, rt.BF16) if is_bf16 else client.buffer(a) for a, is_bf16 in arrays]
    exe = client.compile(text)
    outs, done = exe.execute(args)
    done.wait()
    y = outs[0].to_numpy()
    plan = exe.plan
    for b_ in args + outs:
        b_.close()
    exe.close()
    return y, plan


@pytest.mark.parametrize("cfg", [(3, 2, 128, 256, 2, 128, 512), (4, 4, 2048, 2048, 16, 128, 8192)],
                         ids=["small", "full"])
def test_scan_decoder_bit_identical_to_inline_stack(client, cfg):
    """The decoder written with lax.scan over stacked weights (a counted
    stablehlo.while, unrolled at compile; each layer's weights a view of the
    stacked arrays) against the stack written layer by layer: the same
    kernels on the same bytes, so the same bits."""
    L, B, S, hidden, H, D, F = cfg
    x, ws, cos, sin = synthetic.decoder_stack_case(np.random.default_rng(51), L, B, S, hidden, H, D, F)
    print(f"[decoder-program] scan vs inline L={L} B={B} S={S} hidden={hidden}", flush=True)
    y_scan, plan_scan = _run_program(client, P.decoder_stack_scan(L, B, S, hidden, H, D, F),
                                     synthetic.decoder_stack_scan_arguments(x, ws, cos, sin))
    y_inline, plan_inline = _run_program(client, P.decoder_stack(L, B, S, hidden, H, D, F),
                                         synthetic.decoder_stack_arguments(x, ws, cos, sin))
    assert plan_scan == plan_inline
    assert np.array_equal(y_scan, y_inline)
    assert np.isfinite(bf16_bits_to_f32(y_scan)).all()


@pytest.mark.parametrize("trips", [0, 3, 16])
def test_counted_loop_numerics(client, trips):
    """fori_loop(0, trips, x * 2 + i) unrolled: every step is exact or one
    f32 rounding, evaluated in the same order as numpy's float32 loop, so the
    bits agree."""
    x = np.random.default_rng(trips).standard_normal(8).astype(np.float32)
    y, _ = _run_program(client, P.counted_loop(trips), [(x, False)])
    ref = x.copy()
    for i in range(trips):
        ref = (ref * np.float32(2.0) + np.float32(i)).astype(np.float32)
    assert np.array_equal(y, ref), (y, ref)
