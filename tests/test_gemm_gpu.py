"""GPU parity of the dot_general GEMM kernels (mk_gemm_bf16 / mk_gemm_f32)
against the oracle (float64 matmul, oracle/gemm.py) and closed forms.

Tolerances are the workload's: bf16 output rel 2e-2, f32 rel 1e-5 (the
reference's measure max|out - ref| / max|ref|,
tests/test_f32_gemm_precision.py:25-27 under /root/reference)."""

import numpy as np
import pytest

from _gpu import (BF16_RTOL, F32_RTOL, assert_rel_close, dev, dev_bf16, f32_sum_bound, host_bf16, need_gpu,
                  torch)
from oracle import bf16 as obf
from oracle import gemm

pytestmark = pytest.mark.gpu


def _ops():
    need_gpu()
    from mi355x import ops
    return ops


def _accum_bound(a_bits, b_bits, K):
    """Per-element f32 accumulation bound gamma_{K-1} * (|A| |B|)_ij for
    bf16 operands (their products are exact in f32)."""
    af = np.abs(obf.bf16_bits_to_f32(a_bits).astype(np.float64))
    bf = np.abs(obf.bf16_bits_to_f32(b_bits).astype(np.float64))
    return f32_sum_bound(np.matmul(af, bf), K)


def _case(rng, shape, scale):
    return obf.f32_to_bf16_bits((rng.standard_normal(shape) * scale).astype(np.float32))


BF16_SHAPES = [
    (1, 16, 16, 64), (1, 128, 128, 128), (1, 200, 264, 72), (1, 1024, 1024, 1024),
    (3, 64, 96, 40), (2, 300, 520, 136), (1, 4096, 4096, 4096), (16, 2048, 2048, 128),
]


@pytest.mark.parametrize("batch,M,N,K", BF16_SHAPES)
@pytest.mark.parametrize("out_f32", [False, True])
def test_gemm_bf16_matches_oracle(batch, M, N, K, out_f32):
    ops = _ops()
    rng = np.random.default_rng(batch * 131 + M + N + K)
    a = _case(rng, (batch, M, K), 1.0 / np.sqrt(np.sqrt(K)))
    b = _case(rng, (batch, K, N), 1.0 / np.sqrt(np.sqrt(K)))
    print(f"gemm bf16 case b={batch} M={M} N={N} K={K} out_f32={out_f32}", flush=True)
    c = ops.gemm_bf16(dev_bf16(a), dev_bf16(b), out_f32=out_f32)
    torch.cuda.synchronize()
    if M * N * K * batch > 2 ** 31:
        # float64 reference on a row sample keeps the CPU cost bounded.
        rows = np.random.default_rng(1).choice(M, size=min(M, 64), replace=False)
        af = obf.bf16_bits_to_f32(a[:, rows]).astype(np.float64)
        bf = obf.bf16_bits_to_f32(b).astype(np.float64)
        ref = np.matmul(af, bf)
        out = (c if out_f32 else c.float()).cpu().numpy()[:, rows]
    else:
        af = obf.bf16_bits_to_f32(a).astype(np.float64)
        bf = obf.bf16_bits_to_f32(b).astype(np.float64)
        ref, _ = gemm.matmul_bf16(a, b)
        out = (c.float() if not out_f32 else c).cpu().numpy()
        out = out.reshape(ref.shape)
    if out_f32:
        # f32 output: exact bf16 products accumulated in f32, held to the
        # stated f32 rel 1e-5 normwise and, per element, to the f32
        # summation bound gamma_{K-1} * (|A| |B|)_ij.
        assert_rel_close(out, ref, F32_RTOL, f"bf16 gemm {batch}x{M}x{N}x{K} f32 out",
                         elem=f32_sum_bound(np.matmul(np.abs(af), np.abs(bf)), K))
    else:
        assert_rel_close(out, ref, BF16_RTOL, f"bf16 gemm {batch}x{M}x{N}x{K}")


def test_gemm_bf16_closed_forms():
    ops = _ops()
    K = 512
    eye = np.eye(K, dtype=np.float32)
    rng = np.random.default_rng(3)
    a = obf.f32_to_bf16_bits(rng.standard_normal((64, K)).astype(np.float32))
    c = ops.gemm_bf16(dev_bf16(a), dev_bf16(obf.f32_to_bf16_bits(eye)), out_f32=True)
    assert np.array_equal(c.cpu().numpy(), obf.bf16_bits_to_f32(a))  # A @ I == A exactly
    ones = obf.f32_to_bf16_bits(np.ones((32, K), np.float32))
    ones_b = obf.f32_to_bf16_bits(np.ones((K, 24), np.float32))
    c = ops.gemm_bf16(dev_bf16(ones), dev_bf16(ones_b), out_f32=True)
    assert np.all(c.cpu().numpy() == K)


F32_SHAPES = [(1, 16, 16, 32), (1, 2048, 2048, 2048), (1, 100, 136, 48), (4, 256, 128, 512),
              (1, 1024, 1024, 1024)]


@pytest.mark.parametrize("batch,M,N,K", F32_SHAPES)
def test_gemm_f32_matches_oracle(batch, M, N, K):
    ops = _ops()
    rng = np.random.default_rng(batch + M + 7 * N + K)
    a = (rng.standard_normal((batch, M, K)) / np.sqrt(np.sqrt(K))).astype(np.float32)
    b = (rng.standard_normal((batch, K, N)) / np.sqrt(np.sqrt(K))).astype(np.float32)
    print(f"gemm f32 case b={batch} M={M} N={N} K={K}", flush=True)
    c = ops.gemm_f32(dev(a), dev(b))
    torch.cuda.synchronize()
    ref, _ = gemm.matmul_f32(a, b)
    assert_rel_close(c.cpu().numpy().reshape(ref.shape), ref, F32_RTOL, f"f32 gemm {batch}x{M}x{N}x{K}")


@pytest.mark.parametrize("batch,M,N,K", [(1, 1024, 1024, 1024), (1, 100, 136, 48), (3, 200, 72, 96)])
def test_gemm_f32_tiles_agree(batch, M, N, K, monkeypatch):
    """The 64 x 64 tiles (small grids) and the 128 x 128 tiles run k in the
    same order: the same bits, ragged edges included."""
    ops = _ops()
    rng = np.random.default_rng(M + N + K)
    a = dev(rng.standard_normal((batch, M, K)).astype(np.float32))
    b = dev(rng.standard_normal((batch, K, N)).astype(np.float32))
    outs = []
    for t in ("64", "128"):
        monkeypatch.setenv("MK_GEMM_F32_TILE", t)
        outs.append(ops.gemm_f32(a, b).cpu())
    assert torch.equal(outs[0], outs[1])


@pytest.mark.parametrize("scale", [1.0, 1e3, 1e5])
def test_gemm_f32_precision_scales(scale):
    """The reference's f32 GEMM precision test: rel <= 2e-5 at scales 1, 1e3,
    1e5 (tests/test_f32_gemm_precision.py:40-52); here at the workload's 1e-5."""
    ops = _ops()
    rng = np.random.default_rng(0)
    a = (rng.standard_normal((256, 256)) * scale).astype(np.float32)
    b = rng.standard_normal((256, 256)).astype(np.float32)
    c = ops.gemm_f32(dev(a), dev(b))
    ref, _ = gemm.matmul_f32(a, b)
    assert_rel_close(c.cpu().numpy(), ref, F32_RTOL, f"scale {scale}")


def test_gemm_f32_overflow_case():
    """7e4-magnitude case of tests/test_f32_gemm_precision.py:55-60: the f32
    path must not narrow to f16 (65504 max)."""
    ops = _ops()
    a = np.full((32, 32), 7e4, np.float32)
    b = np.eye(32, dtype=np.float32)
    c = ops.gemm_f32(dev(a), dev(b)).cpu().numpy()
    assert np.all(c == 7e4)


@pytest.mark.parametrize("batch,M,N,K", [(1, 256, 256, 64), (3, 512, 768, 320), (2, 1024, 256, 1024)])
def test_gemm_bf16_large_tile_path(batch, M, N, K, monkeypatch):
    """The 256x256 kernel (transposing LDS reads for B) on shapes small enough
    for a full float64 check, forced with MK_GEMM_TILE=256 (and the short-K
    kernel off)."""
    ops = _ops()
    monkeypatch.setenv("MK_GEMM_TILE", "256")
    monkeypatch.setenv("MK_GEMM_SHORTK", "0")
    monkeypatch.setenv("MK_GEMM_PERSIST", "0")
    rng = np.random.default_rng(batch + M + N + K)
    a = _case(rng, (batch, M, K), 1.0 / np.sqrt(np.sqrt(K)))
    b = _case(rng, (batch, K, N), 1.0 / np.sqrt(np.sqrt(K)))
    c = ops.gemm_bf16(dev_bf16(a), dev_bf16(b), out_f32=True)
    ref, _ = gemm.matmul_bf16(a, b)
    assert_rel_close(c.cpu().numpy().reshape(ref.shape), ref, F32_RTOL, f"256 tile {batch}x{M}x{N}x{K}",
                     elem=_accum_bound(a, b, K))
    cb = ops.gemm_bf16(dev_bf16(a), dev_bf16(b), out_f32=False)
    assert_rel_close(cb.float().cpu().numpy().reshape(ref.shape), ref, BF16_RTOL, "256 tile bf16 out")


@pytest.mark.parametrize("batch,M,N,K", [(1, 256, 512, 4096), (2, 512, 256, 4128), (1, 256, 256, 4160),
                                         (1, 512, 512, 2048), (1, 256, 256, 2080)])
def test_gemm_bf16_pipelined_path(batch, M, N, K, monkeypatch):
    """The pipelined 256x256 kernel (K >= 2048, no epilogue operand): the K
    loop ends with 6 (K = 4096, 2048) or 5 (K = 4128, 2080) iterations that
    issue no further DMA, covering both tails.  Checked against float64 on every
    element, and bit for bit against the other 256x256 kernel with f32
    output: both accumulate each k in the same order in the same MFMA."""
    ops = _ops()
    rng = np.random.default_rng(batch + M + N + K)
    a = _case(rng, (batch, M, K), 1.0 / np.sqrt(np.sqrt(K)))
    b = _case(rng, (batch, K, N), 1.0 / np.sqrt(np.sqrt(K)))
    print(f"gemm pipelined case b={batch} M={M} N={N} K={K}", flush=True)
    ref, _ = gemm.matmul_bf16(a, b)
    c = ops.gemm_bf16(dev_bf16(a), dev_bf16(b), out_f32=True)
    assert_rel_close(c.cpu().numpy().reshape(ref.shape), ref, F32_RTOL, f"pipelined {batch}x{M}x{N}x{K}",
                     elem=_accum_bound(a, b, K))
    # bf16 output: the LDS-staged store rounds the same f32 accumulator.
    cb = ops.gemm_bf16(dev_bf16(a), dev_bf16(b), out_f32=False)
    cb_bits = cb.view(torch.int16).cpu().numpy().view(np.uint16)
    assert np.array_equal(cb_bits, obf.f32_to_bf16_bits(c.cpu().numpy())), "bf16 store != r(f32 accumulator)"
    assert_rel_close(cb.float().cpu().numpy().reshape(ref.shape), ref, BF16_RTOL, f"pipelined bf16 out")
    monkeypatch.setenv("MK_GEMM_PIPE", "0")
    c0 = ops.gemm_bf16(dev_bf16(a), dev_bf16(b), out_f32=True)
    torch.cuda.synchronize()
    assert np.array_equal(c.cpu().numpy(), c0.cpu().numpy()), "pipelined and ring kernels differ"


@pytest.mark.parametrize("batch,M,N,K", [(1, 256, 256, 32), (2, 256, 512, 320), (1, 512, 768, 2048),
                                         (1, 256, 256, 4160), (1, 1024, 512, 1056)])
@pytest.mark.parametrize("epilogue", [None, "add", "swiglu", "swiglu_pairs"])
def test_gemm_bf16_nt_bit_identical(batch, M, N, K, epilogue, monkeypatch):
    """B given transposed (bt [N, K]): the same bits as the [K, N] product of
    its transposed copy, on the ring kernel (K < 2048) and the pipelined one
    (both loop tails), with every epilogue; and against float64."""
    ops = _ops()
    rng = np.random.default_rng(batch * 7 + M + N + K)
    a = dev_bf16(_case(rng, (batch, M, K), 1.0 / np.sqrt(np.sqrt(K))))
    bt_h = _case(rng, (batch, N, K), 1.0 / np.sqrt(np.sqrt(K)))
    bt = dev_bf16(bt_h)
    b = bt.transpose(-1, -2).contiguous()
    aux = None
    if epilogue in ("add", "swiglu"):
        aux = dev_bf16(_case(rng, (batch, M, N), 1.0))
    print(f"gemm nt case b={batch} M={M} N={N} K={K} epilogue={epilogue}", flush=True)
    c_nt = ops.gemm_bf16_nt(a, bt, epilogue=epilogue, aux=aux)
    c_nn = ops.gemm_bf16(a, b, epilogue=epilogue, aux=aux)
    torch.cuda.synchronize()
    assert torch.equal(c_nt.view(torch.int16), c_nn.view(torch.int16)), "NT and NN products differ"
    if epilogue is None:
        monkeypatch.setenv("MK_GEMM_PIPE", "0")
        c_ring = ops.gemm_bf16_nt(a, bt)
        torch.cuda.synchronize()
        assert torch.equal(c_nt.view(torch.int16), c_ring.view(torch.int16)), "NT pipelined and ring differ"
        ah = obf.bf16_bits_to_f32(a.view(torch.int16).cpu().numpy().view(np.uint16)).astype(np.float64)
        ref = np.matmul(ah, obf.bf16_bits_to_f32(bt_h).astype(np.float64).transpose(0, 2, 1))
        assert_rel_close(c_nt.float().cpu().numpy(), ref, BF16_RTOL, f"nt {batch}x{M}x{N}x{K}")


def test_gemm_bf16_nt_rejects_unaligned_shapes():
    ops = _ops()
    a = torch.zeros((200, 64), dtype=torch.bfloat16, device="cuda")
    bt = torch.zeros((256, 64), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(Exception, match="M % 256 == 0"):
        ops.gemm_bf16_nt(a, bt)


@pytest.mark.parametrize("batch,M,N,K", [(1, 256, 256, 32), (16, 256, 512, 128), (2, 512, 768, 96),
                                         (1, 256, 256, 256), (3, 384, 640, 64), (1, 128, 128, 160),
                                         (16, 2048, 2048, 128), (5, 512, 256, 64), (1, 4096, 4096, 128)])
@pytest.mark.parametrize("epilogue", [None, "add", "swiglu"])
def test_gemm_bf16_short_k_kernels(batch, M, N, K, epilogue):
    """The two short-K kernels: the 128 x 128 one with all of K in LDS
    (route "short", K <= 256) and the persistent 256 x 256 one (route
    "persist", K <= 128, M and N multiples of 256).  Against float64 on
    every element, bit for bit against each other and the 256 x 256 ring
    kernel (each k in the same order in the same MFMA), and with the ADD /
    SWIGLU epilogue bit for bit against the plain product followed by the
    elementwise program.  The persistent grid holds one workgroup per CU, so
    the larger shapes walk several tiles per workgroup."""
    ops = _ops()
    rng = np.random.default_rng(batch * 5 + M + N + K)
    a_h = _case(rng, (batch, M, K), 1.0 / np.sqrt(np.sqrt(K)))
    b_h = _case(rng, (batch, K, N), 1.0 / np.sqrt(np.sqrt(K)))
    a, b = dev_bf16(a_h), dev_bf16(b_h)
    aux = dev_bf16(_case(rng, (batch, M, N), 1.0)) if epilogue else None
    print(f"gemm short-k case b={batch} M={M} N={N} K={K} epilogue={epilogue}", flush=True)

    def run(route):
        out = ops.gemm_bf16_route(a, b, route, epilogue=epilogue, aux=aux)
        torch.cuda.synchronize()
        return out

    c = run("short")
    if epilogue is None:
        if batch * M * N * K <= 2 ** 30:
            ref, _ = gemm.matmul_bf16(a_h, b_h)
            assert_rel_close(c.float().cpu().numpy().reshape(ref.shape), ref, BF16_RTOL, f"short-k {batch}x{M}x{N}x{K}")
    else:
        plain = ops.gemm_bf16(a, b)
        prog = ([("LOAD", 0, 0, 0, 0, 0.0), ("LOAD", 1, 1, 0, 0, 0.0), ("ADD", 2, 0, 1, 0, 0.0)]
                if epilogue == "add" else
                [("LOAD", 0, 0, 0, 0, 0.0), ("LOAD", 1, 1, 0, 0, 0.0), ("LOGISTIC", 2, 1, 0, 0, 0.0),
                 ("MUL", 3, 1, 2, 0, 0.0), ("MUL", 4, 3, 0, 0, 0.0)])
        want = ops.elementwise(prog, [plain, aux], out_slot=2 if epilogue == "add" else 4)
        torch.cuda.synchronize()
        assert torch.equal(c.view(torch.int16), want.view(torch.int16)), f"short-k {epilogue} epilogue"
    if M % 256 == 0 and N % 256 == 0:
        ring = run("ring")
        assert torch.equal(c.view(torch.int16), ring.view(torch.int16)), "short-k and ring kernels differ"
        if K <= 128:
            pers = run("persist")
            assert torch.equal(pers.view(torch.int16), ring.view(torch.int16)), "persistent and ring kernels differ"


ROUTE_SHAPES = [(1, 256, 256, 64), (2, 512, 768, 320), (16, 256, 512, 128), (3, 384, 640, 96),
                (1, 200, 264, 72), (1, 512, 512, 2048), (2, 256, 256, 4160), (1, 128, 384, 256)]


@pytest.mark.parametrize("batch,M,N,K", ROUTE_SHAPES)
@pytest.mark.parametrize("epilogue,out_f32", [(None, False), (None, True), ("add", False), ("swiglu", False)])
def test_gemm_routes_bit_identical(batch, M, N, K, epilogue, out_f32):
    """Every route that takes a product (the measured route choice picks
    among them) gives the built-in choice's bits: the same k order in the
    same MFMA on every kernel, ragged shapes and f32 outputs included."""
    from mi355x import _lib as L
    ops = _ops()
    rng = np.random.default_rng(batch * 3 + M + N + K)
    a = dev_bf16(_case(rng, (batch, M, K), 1.0 / np.sqrt(np.sqrt(K))))
    b = dev_bf16(_case(rng, (batch, K, N), 1.0 / np.sqrt(np.sqrt(K))))
    aux = dev_bf16(_case(rng, (batch, M, N), 1.0)) if epilogue else None
    ref = ops.gemm_bf16(a, b, out_f32=out_f32, epilogue=epilogue, aux=aux)
    bits = torch.int32 if out_f32 else torch.int16
    ran = []
    for route in L.GEMM_ROUTES:
        if route == "default" or not ops.gemm_route_fits(route, M, N, K, epilogue, out_f32):
            continue
        print(f"gemm route {route} b={batch} M={M} N={N} K={K} epilogue={epilogue} f32={out_f32}", flush=True)
        c = ops.gemm_bf16_route(a, b, route, out_f32=out_f32, epilogue=epilogue, aux=aux)
        torch.cuda.synchronize()
        assert torch.equal(c.view(bits), ref.view(bits)), f"route {route} differs"
        ran.append(route)
    assert len(ran) >= 2, ran


@pytest.mark.parametrize("batch,M,N,K", [(1, 1024, 1024, 1024), (16, 256, 512, 128), (1, 384, 640, 64)])
def test_gemm_autotune_records_a_fitting_route(batch, M, N, K, tmp_path):
    """The measured choice: a route that takes the product, recorded in the
    table for this device, the product left in c, and the table written and
    read back."""
    ops = _ops()
    ops.gemm_autotune_clear()
    rng = np.random.default_rng(M + N + K)
    a = dev_bf16(_case(rng, (batch, M, K), 1.0 / np.sqrt(np.sqrt(K))))
    b = dev_bf16(_case(rng, (batch, K, N), 1.0 / np.sqrt(np.sqrt(K))))
    name, us, c = ops.gemm_bf16_autotune(a, b)
    torch.cuda.synchronize()
    print(f"autotune b={batch} M={M} N={N} K={K}: {name} {us:.1f} us", flush=True)
    assert name != "default" and ops.gemm_route_fits(name, M, N, K) and us > 0
    assert torch.equal(c.view(torch.int16), ops.gemm_bf16(a, b).view(torch.int16))
    assert ops.gemm_tuned_route(batch, M, N, K) == name
    assert ops.gemm_tuned_route(batch, M, N, K, out_f32=True) == "default"
    path = tmp_path / "routes.txt"
    assert ops.gemm_autotune_save(path) == 1
    ops.gemm_autotune_clear()
    assert ops.gemm_tuned_route(batch, M, N, K) == "default"
    assert ops.gemm_autotune_load(path) == 1
    assert ops.gemm_tuned_route(batch, M, N, K) == name
    ops.gemm_autotune_clear()


def test_runtime_tunes_gemm_steps(tmp_path, monkeypatch):
    """The plugin runtime measures each bf16 GEMM step's route at the first
    plan build and keeps the table in the cache directory (MK_CACHE_DIR);
    the outputs equal the untuned plan's bit for bit (MK_GEMM_AUTOTUNE=0)."""
    from mi355x import programs
    from mi355x import runtime as rt
    ops = _ops()
    monkeypatch.setenv("MK_CACHE_DIR", str(tmp_path))
    monkeypatch.delenv("MK_DISABLE_CACHE_PERSIST", raising=False)
    rng = np.random.default_rng(11)
    M, K, N = 512, 320, 768
    a = _case(rng, (M, K), 1.0 / np.sqrt(np.sqrt(K)))
    b = _case(rng, (K, N), 1.0 / np.sqrt(np.sqrt(K)))
    outs = {}
    for tune in ("1", "0"):
        monkeypatch.setenv("MK_GEMM_AUTOTUNE", tune)
        ops.gemm_autotune_clear()
        client = rt.Client()
        try:
            exe = client.compile(programs.matmul(M, K, N))
            ba, bb = client.buffer(a, rt.BF16), client.buffer(b, rt.BF16)
            (o,), done = exe.execute([ba, bb])
            done.wait()
            outs[tune] = o.to_numpy()
            if tune == "1":
                assert ops.gemm_tuned_route(1, M, N, K) != "default"
            else:
                assert ops.gemm_tuned_route(1, M, N, K) == "default"
            for h in (ba, bb, o):
                h.close()
            exe.close()
        finally:
            client.close()
    assert np.array_equal(outs["1"], outs["0"])
    lines = (tmp_path / "gemm_routes.txt").read_text().splitlines()
    from mi355x import _lib as L
    assert lines[0] == L.lib().mk_gemm_autotune_header().decode()
    assert any(l.split()[2:6] == ["1", str(M), str(N), str(K)] for l in lines[1:]), lines
    ops.gemm_autotune_clear()
