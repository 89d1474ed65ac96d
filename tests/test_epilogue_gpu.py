"""GPU checks of the fused store epilogues (mk_gemm_bf16_epilogue and
mk_int4g64 / mk_int8pc _matmul_epilogue_bf16): each must equal, bit for bit,
the plain product followed by the bf16 elementwise program it replaces
(residual add; silu(g) * u), on every kernel path (DMA / 256 / 128-tile
GEMMs; streaming, wide, many-row and dequantise-then-GEMM quantized paths),
in place (aux == out) and out of place."""

import numpy as np
import pytest

from _gpu import dev, dev_bf16, need_gpu, torch
from oracle import quant

pytestmark = pytest.mark.gpu

ADD = [("LOAD", 0, 0, 0, 0, 0.0), ("LOAD", 1, 1, 0, 0, 0.0), ("ADD", 2, 0, 1, 0, 0.0)]
SWIGLU = [("LOAD", 0, 0, 0, 0, 0.0), ("LOAD", 1, 1, 0, 0, 0.0),
          ("LOGISTIC", 2, 0, 0, 0, 0.0), ("MUL", 3, 0, 2, 0, 0.0), ("MUL", 4, 3, 1, 0, 0.0)]


def _ops():
    need_gpu()
    from mi355x import ops
    return ops


def _unfused(ops, y, aux, epilogue):
    if epilogue == "add":
        return ops.elementwise(ADD, [aux, y], out_slot=2)
    return ops.elementwise(SWIGLU, [aux, y], out_slot=4)


@pytest.mark.parametrize("epilogue", ["add", "swiglu"])
# (1, 256, 256, 2048) and (2, 256, 512, 4096): the pipelined kernel (K >= 2048).
@pytest.mark.parametrize("batch,M,N,K", [(1, 512, 512, 256), (1, 256, 768, 64), (2, 256, 256, 96),
                                         (1, 200, 136, 64), (3, 64, 128, 32), (1, 256, 256, 2048),
                                         (2, 256, 512, 4096)])
def test_gemm_epilogue_matches_unfused(epilogue, batch, M, N, K):
    ops = _ops()
    g = torch.Generator().manual_seed(M + N + K + batch)
    shape_a = (M, K) if batch == 1 else (batch, M, K)
    shape_b = (K, N) if batch == 1 else (batch, K, N)
    shape_c = (M, N) if batch == 1 else (batch, M, N)
    a = (torch.randn(shape_a, generator=g) / 8).to(torch.bfloat16).cuda()
    b = (torch.randn(shape_b, generator=g) / 8).to(torch.bfloat16).cuda()
    aux = (torch.randn(shape_c, generator=g) * 2).to(torch.bfloat16).cuda()
    ref = _unfused(ops, ops.gemm_bf16(a, b), aux, epilogue)
    y = ops.gemm_bf16(a, b, epilogue=epilogue, aux=aux)
    z = aux.clone()
    ops.gemm_bf16(a, b, out=z, epilogue=epilogue, aux=z)  # in place
    torch.cuda.synchronize()
    assert torch.equal(y, ref)
    assert torch.equal(z, ref)


# M = 1 / 16: streaming and wide kernels; 130 / 256: many-row kernel; 800:
# dequantise-then-GEMM; (16, 1024, 1024): split-K with the reduce pass;
# (16, 4096, 14336): the headline shape, on both wide kernels (int4, int8)
# with their in-kernel split-K exchange.
@pytest.mark.parametrize("epilogue", ["add", "swiglu"])
@pytest.mark.parametrize("M,K,N", [(1, 512, 256), (16, 4096, 1024), (16, 1024, 14336), (130, 256, 192),
                                   (256, 512, 512), (800, 256, 256), (5, 512, 136), (16, 4096, 14336)])
def test_quantized_epilogue_matches_unfused(epilogue, M, K, N):
    ops = _ops()
    rng = np.random.default_rng(M * 3 + K + N)
    x, packed, s, z = quant.make_int4_case(rng, M, K, N)
    args4 = (dev_bf16(x), dev(packed), dev_bf16(s), dev(z))
    aux = (torch.randn((M, N), generator=torch.Generator().manual_seed(M + N)) * 2).to(torch.bfloat16).cuda()
    ref = _unfused(ops, ops.int4_g64_matmul(*args4), aux, epilogue)
    y = ops.int4_g64_matmul(*args4, epilogue=epilogue, aux=aux)
    zz = aux.clone()
    ops.int4_g64_matmul(*args4, out=zz, epilogue=epilogue, aux=zz)
    torch.cuda.synchronize()
    assert torch.equal(y, ref), f"int4 {M}x{K}x{N} {epilogue}"
    assert torch.equal(zz, ref), f"int4 {M}x{K}x{N} {epilogue} in place"
    x8, w8, s8 = quant.make_int8_case(rng, M, K, N)
    args8 = (dev_bf16(x8), dev(w8), dev(s8))
    from mi355x import _lib
    L = _lib.lib()
    y8 = ops.int8_pc_matmul(*args8)
    ref8 = _unfused(ops, y8, aux, epilogue)
    out8 = torch.empty_like(y8)
    nb = L.mk_qmatmul_workspace_bytes(_lib.MK_QFMT_INT8_PC, M, K, N)
    ws = ops.workspace(nb, "cuda:0") if nb > 0 else None
    code = {"add": _lib.MK_EPI_ADD, "swiglu": _lib.MK_EPI_SWIGLU}[epilogue]
    rc = L.mk_int8pc_matmul_epilogue_bf16(args8[0].data_ptr(), args8[1].data_ptr(), args8[2].data_ptr(),
                                         out8.data_ptr(), aux.data_ptr(), code, M, K, N,
                                         ws.data_ptr() if ws is not None else None, max(nb, 0),
                                         torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rc == 0, L.mk_last_error().decode()
    assert torch.equal(out8, ref8), f"int8 {M}x{K}x{N} {epilogue}"


def test_epilogue_rejects_bad_arguments():
    ops = _ops()
    from mi355x import _lib
    L = _lib.lib()
    a = torch.zeros((256, 64), dtype=torch.bfloat16, device="cuda")
    b = torch.zeros((64, 256), dtype=torch.bfloat16, device="cuda")
    c = torch.empty((256, 256), dtype=torch.bfloat16, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    assert L.mk_gemm_bf16_epilogue(a.data_ptr(), b.data_ptr(), c.data_ptr(), None, _lib.MK_EPI_ADD, 1, 256,
                                   256, 64, st) == _lib.MK_EINVAL
    assert L.mk_gemm_bf16_epilogue(a.data_ptr(), b.data_ptr(), c.data_ptr(), c.data_ptr(), 7, 1, 256, 256, 64,
                                   st) == _lib.MK_EINVAL
    with pytest.raises(ValueError):
        ops.gemm_bf16(a, b, epilogue="add", aux=torch.zeros((8, 8), dtype=torch.bfloat16, device="cuda"))


# (512, 256, 256): the ring kernel; (256, 4096, 256): the pipelined kernel
# (K >= 4096); (256, 64, 512): two 32-k stages per tile.
@pytest.mark.parametrize("M,K,F", [(512, 256, 256), (256, 4096, 256), (256, 64, 512)])
def test_gemm_swiglu_pairs_matches_two_products(M, K, F):
    """One product against [Wg | Wu] (16-column blocks interleaved) equals,
    bit for bit, g = x @ Wg and silu(g) * (x @ Wu) as the "swiglu" epilogue
    (itself bit-identical to the elementwise program) computes it."""
    ops = _ops()
    g = torch.Generator().manual_seed(M + K + F)
    x = (torch.randn((M, K), generator=g) / 4).to(torch.bfloat16).cuda()
    wg = (torch.randn((K, F), generator=g) / 8).to(torch.bfloat16).cuda()
    wu = (torch.randn((K, F), generator=g) / 8).to(torch.bfloat16).cuda()
    print(f"[epilogue] gemm swiglu_pairs M={M} K={K} F={F}", flush=True)
    gate = ops.gemm_bf16(x, wg)
    ref = ops.gemm_bf16(x, wu, epilogue="swiglu", aux=gate)
    ref2 = _unfused(ops, ops.gemm_bf16(x, wu), gate, "swiglu")
    y = ops.gemm_bf16(x, ops.interleave_gate_up(wg, wu), epilogue="swiglu_pairs")
    torch.cuda.synchronize()
    assert y.shape == (M, F)
    assert torch.equal(ref, ref2)
    assert torch.equal(y, ref)


def test_int4_swiglu_pairs_matches_two_products():
    """The decoder's form: int4 g64 gate and up weights interleaved by
    column (scales and zero points alike), dequantise-then-GEMM route."""
    ops = _ops()
    M, K, F = 1024, 512, 256
    rng = np.random.default_rng(11)
    x, pg, sg, zg = quant.make_int4_case(rng, M, K, F)
    _, pu, su, zu = quant.make_int4_case(rng, M, K, F)
    xd = dev_bf16(x)
    wg = (dev(pg), dev_bf16(sg), dev(zg))
    wu = (dev(pu), dev_bf16(su), dev(zu))
    print(f"[epilogue] int4 swiglu_pairs M={M} K={K} F={F}", flush=True)
    gate = ops.int4_g64_matmul(xd, *wg)
    ref = ops.int4_g64_matmul(xd, *wu, epilogue="swiglu", aux=gate)
    wgu = [ops.interleave_gate_up(a, b) for a, b in zip(wg, wu)]
    y = ops.int4_g64_matmul(xd, *wgu, epilogue="swiglu_pairs")
    torch.cuda.synchronize()
    assert y.shape == (M, F)
    assert torch.equal(y, ref)


def test_swiglu_pairs_rejects_unsupported_shapes():
    ops = _ops()
    from mi355x import _lib
    L = _lib.lib()
    st = torch.cuda.current_stream().cuda_stream
    a = torch.zeros((200, 64), dtype=torch.bfloat16, device="cuda")
    b = torch.zeros((64, 256), dtype=torch.bfloat16, device="cuda")
    c = torch.empty((200, 128), dtype=torch.bfloat16, device="cuda")
    assert L.mk_gemm_bf16_epilogue(a.data_ptr(), b.data_ptr(), c.data_ptr(), None, _lib.MK_EPI_SWIGLU_PAIRS, 1,
                                   200, 256, 64, st) == _lib.MK_EUNSUPPORTED
    # Decode-sized rows take the streaming kernels, which have no paired form.
    rng = np.random.default_rng(2)
    x, p, s, z = quant.make_int4_case(rng, 16, 256, 256)
    with pytest.raises(RuntimeError):
        ops.int4_g64_matmul(dev_bf16(x), dev(p), dev_bf16(s), dev(z), epilogue="swiglu_pairs")


# (1024, 512, 256) / (768, 2048, 1024): the dequantise-then-GEMM route with the
# ring and the pipelined GEMM; (1024, 256, 384): N not a multiple of 256.
@pytest.mark.parametrize("fmt", ["int4", "int8"])
@pytest.mark.parametrize("M,K,N", [(1024, 512, 256), (768, 2048, 1024), (1024, 256, 384)])
def test_swiglu_pair_from_separate_weights_matches_two_products(fmt, M, K, N):
    """mk_*_matmul_swiglu_pair_bf16 (both weights dequantised into one
    interleaved buffer, one GEMM) equals, bit for bit, the two products
    followed by the SwiGLU elementwise program."""
    ops = _ops()
    rng = np.random.default_rng(M + K + N + len(fmt))
    if fmt == "int4":
        x, pg, sg, zg = quant.make_int4_case(rng, M, K, N)
        _, pu, su, zu = quant.make_int4_case(rng, M, K, N)
        wg, wu = (dev(pg), dev_bf16(sg), dev(zg)), (dev(pu), dev_bf16(su), dev(zu))
        mm = ops.int4_g64_matmul
    else:
        x, wg8, sg = quant.make_int8_case(rng, M, K, N)
        _, wu8, su = quant.make_int8_case(rng, M, K, N)
        wg, wu = (dev(wg8), dev(sg)), (dev(wu8), dev(su))
        mm = ops.int8_pc_matmul
    xd = dev_bf16(x)
    print(f"[epilogue] {fmt} swiglu pair from separate weights M={M} K={K} N={N}", flush=True)
    ref = _unfused(ops, mm(xd, *wu), mm(xd, *wg), "swiglu")
    y = ops.swiglu_pair_matmul(xd, wg, wu)
    torch.cuda.synchronize()
    assert torch.equal(y, ref)


def test_swiglu_pair_rejects_decode_shapes():
    ops = _ops()
    from mi355x import _lib
    L = _lib.lib()
    assert L.mk_qmatmul_swiglu_pair_workspace_bytes(_lib.MK_QFMT_INT4_G64, 16, 256, 256) == -1
    assert L.mk_qmatmul_swiglu_pair_workspace_bytes(_lib.MK_QFMT_INT4_G64, 1024, 256, 200) == -1
    assert L.mk_qmatmul_swiglu_pair_workspace_bytes(_lib.MK_QFMT_INT8_PC, 1024, 256, 256) == 64 * 1024 + 256 * 512 * 2
    rng = np.random.default_rng(3)
    x, p, s, z = quant.make_int4_case(rng, 16, 256, 256)
    w = (dev(p), dev_bf16(s), dev(z))
    with pytest.raises(RuntimeError):
        ops.swiglu_pair_matmul(dev_bf16(x), w, w)
