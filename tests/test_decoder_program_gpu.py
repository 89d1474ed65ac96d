"""GPU parity of the Llama-style decoder layer compiled from its StableHLO
(mi355x/programs.decoder_layer: the layer as jax.jit lowers it, the
reference's transformer-layer benchmark, benchmarks/vs_cpu.py:603-626)
through the runtime's compile -> execute path, against the float64 oracle
layer (oracle/decoder.py) at the workload's bf16 tolerance per token.

The program rounds where jax's bf16 ops round (RMSNorm's x * x, the
scores, softmax's exp and quotient) and the oracle rounds once per block,
so the comparison is the bf16 measure max |err| / max |ref| per row, not an
elementwise one."""

import numpy as np
import pytest

from mi355x import programs as P
from mi355x import runtime as rt
from oracle import decoder as odec
from oracle import quant
from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits

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


def _weight(rng, K, N):
    """int4 g64 weight (packed, scale bits, zero) with q, z ~ U{0..15} and
    s ~ U(0.004, 0.006): scales that keep a random layer's activations O(1)."""
    q = rng.integers(0, 16, size=(K, N), dtype=np.uint8)
    s = f32_to_bf16_bits(rng.uniform(0.004, 0.006, size=(K // 64, N)).astype(np.float32))
    z = rng.integers(0, 16, size=(K // 64, N), dtype=np.uint8)
    return quant.pack_int4_k(q), s, z


def _layer_case(seed, B, S, hidden, H, D, F):
    rng = np.random.default_rng(seed)
    A = H * D
    x = f32_to_bf16_bits(rng.standard_normal((B * S, hidden)).astype(np.float32))
    g1 = f32_to_bf16_bits(rng.uniform(0.5, 1.5, size=hidden).astype(np.float32))
    g2 = f32_to_bf16_bits(rng.uniform(0.5, 1.5, size=hidden).astype(np.float32))
    w = {"g_attn": g1, "g_mlp": g2, "w_qkv": _weight(rng, hidden, 3 * A), "w_o": _weight(rng, A, hidden),
         "w_gate": _weight(rng, hidden, F), "w_up": _weight(rng, hidden, F), "w_down": _weight(rng, F, hidden)}
    cos, sin = odec.rope_tables(S, D)
    return x, w, cos.astype(np.float32), sin.astype(np.float32)


def _run_layer(client, B, S, hidden, H, D, F, x, w, cos, sin):
    text = P.decoder_layer(B, S, hidden, H, D, F)
    print(f"[decoder-program] B={B} S={S} hidden={hidden} H={H} D={D} F={F}", flush=True)
    exe = client.compile(text)
    bf = lambda a: client.buffer(np.ascontiguousarray(a, dtype=np.uint16), rt.BF16)
    args = [bf(x), bf(w["g_attn"])]
    for name in ("w_qkv", "w_o"):
        p, s, z = w[name]
        args += [client.buffer(p), bf(s), client.buffer(z)]
    args.append(bf(w["g_mlp"]))
    for name in ("w_gate", "w_up", "w_down"):
        p, s, z = w[name]
        args += [client.buffer(p), bf(s), client.buffer(z)]
    args += [client.buffer(cos), client.buffer(sin)]
    outs, done = exe.execute(args)
    done.wait()
    (y,) = [o.to_numpy() for o in outs]
    plan = exe.plan
    for b in args + outs:
        b.close()
    exe.close()
    return bf16_bits_to_f32(y).reshape(B, S, hidden), plan


def _check_rows(y, x, w, B, S, hidden, H, D, pos, batches):
    x3 = bf16_bits_to_f32(x).reshape(B, S, hidden)
    for b in batches:
        ref = odec.layer_rows(x3[b], pos, w, H, D)
        o = y[b, pos].astype(np.float64)
        assert np.isfinite(o).all()
        row_rel = np.abs(o - ref).max(axis=1) / np.abs(ref).max(axis=1)
        print(f"[decoder-program] batch {b}: worst row rel err {row_rel.max():.3e}", flush=True)
        assert row_rel.max() <= BF16_RTOL, (b, pos[int(row_rel.argmax())], row_rel.max())


@pytest.mark.parametrize("B,S,hidden,H,D,F", [(1, 64, 128, 2, 64, 256), (2, 128, 256, 2, 128, 512)])
def test_decoder_program_small_vs_oracle(client, B, S, hidden, H, D, F):
    x, w, cos, sin = _layer_case(B * 1000 + S, B, S, hidden, H, D, F)
    y, plan = _run_layer(client, B, S, hidden, H, D, F, x, w, cos, sin)
    # the projections, norms and attention products run on their kernels
    assert plan.count("int4_g64_matmul") == 5 and plan.count("rmsnorm") == 2
    assert "softmax" in plan and plan.count("gemm_bf16") == 2
    _check_rows(y, x, w, B, S, hidden, H, D, np.arange(S), range(B))


def test_decoder_program_full_config_vs_oracle(client):
    """The workload's decoder layer (hidden 2048, 16 x 128 heads, SwiGLU 8192,
    batch 4 x 2048 tokens) compiled from StableHLO, checked on batch elements
    0 and 3 at 16 positions (first and last rows, tile boundaries, random)."""
    B, S, hidden, H, D, F = 4, 2048, 2048, 16, 128, 8192
    x, w, cos, sin = _layer_case(7, B, S, hidden, H, D, F)
    y, _ = _run_layer(client, B, S, hidden, H, D, F, x, w, cos, sin)
    assert np.isfinite(y).all()
    rng = np.random.default_rng(3)
    pos = np.unique(np.concatenate([[0, 1, 63, 64, 1023, 2047], rng.integers(2, S - 1, size=10)]))
    _check_rows(y, x, w, B, S, hidden, H, D, pos, (0, B - 1))
