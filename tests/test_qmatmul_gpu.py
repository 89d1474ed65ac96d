"""GPU parity of the int4 group-64 and int8 per-channel dequant-matmul
kernels (mk_int4g64_matmul_bf16 / mk_int8pc_matmul_bf16) against the oracle.

The oracle restates Y = X @ ((W - z) * s) in float64 (oracle/quant.py) and
in C (oracle/c/oracle.c); the workload's bf16 tolerance is rel 2e-2.
"""

import numpy as np
import pytest

from _gpu import (BF16_RTOL, assert_rel_close, dev, dev_bf16, host_bf16, host_bf16_bits, need_gpu,
                  torch)
from oracle import cport, quant
from oracle.bf16 import bf16_bits_to_f32

pytestmark = pytest.mark.gpu


def _ops():
    need_gpu()
    from mi355x import ops
    return ops


INT4_SHAPES = [
    (1, 64, 8), (16, 128, 128), (5, 256, 264), (16, 1024, 1024), (3, 512, 136),
    (17, 256, 384), (33, 192, 512), (16, 4096, 1024), (64, 2048, 896),
]


@pytest.mark.parametrize("M,K,N", INT4_SHAPES)
def test_int4_g64_matches_oracle(M, K, N):
    ops = _ops()
    rng = np.random.default_rng(1000 + M * 7 + K + N)
    x, packed, s, z = quant.make_int4_case(rng, M, K, N)
    print(f"int4 case M={M} K={K} N={N}", flush=True)
    y = ops.int4_g64_matmul(dev_bf16(x), dev(packed), dev_bf16(s), dev(z))
    torch.cuda.synchronize()
    ref, _ = quant.int4_g64_matmul(x, packed, s, z)
    assert_rel_close(host_bf16(y), ref, BF16_RTOL, f"int4 {M}x{K}x{N}")


def test_int4_g64_headline_shape():
    """M=16, K=4096, N=14336 (the workload's headline case) vs the C oracle."""
    ops = _ops()
    rng = np.random.default_rng(0)
    M, K, N = 16, 4096, 14336
    x, packed, s, z = quant.make_int4_case(rng, M, K, N)
    y = ops.int4_g64_matmul(dev_bf16(x), dev(packed), dev_bf16(s), dev(z))
    torch.cuda.synchronize()
    ref = cport.int4_g64_matmul(x, packed, s, z)
    assert_rel_close(host_bf16(y), ref, BF16_RTOL, "int4 headline")


def test_int4_g64_deterministic_and_reusable_workspace():
    ops = _ops()
    rng = np.random.default_rng(5)
    x, packed, s, z = quant.make_int4_case(rng, 16, 4096, 2048)
    args = (dev_bf16(x), dev(packed), dev_bf16(s), dev(z))
    y1 = host_bf16_bits(ops.int4_g64_matmul(*args))
    y2 = host_bf16_bits(ops.int4_g64_matmul(*args))
    torch.cuda.synchronize()
    assert np.array_equal(y1, y2)


def test_int4_g64_shapes_in_sequence_share_workspace():
    """Calls of different shapes back to back through one cached workspace
    (a split-K shape between whole-K shapes) all match the oracle."""
    ops = _ops()
    rng = np.random.default_rng(11)
    for (M, K, N) in [(16, 1024, 1024), (3, 512, 136), (16, 4096, 14336), (5, 4096, 512)]:
        x, packed, s, z = quant.make_int4_case(rng, M, K, N)
        y = ops.int4_g64_matmul(dev_bf16(x), dev(packed), dev_bf16(s), dev(z))
        torch.cuda.synchronize()
        ref = cport.int4_g64_matmul(x, packed, s, z)
        assert_rel_close(host_bf16(y), ref, BF16_RTOL, f"int4 seq {M}x{K}x{N}")


def test_int4_g64_known_answer_all_ones():
    """x = 1, q = 15, z = 14, s = 0.5: every output is K * 0.5."""
    ops = _ops()
    M, K, N = 4, 256, 128
    x = np.full((M, K), 0x3F80, np.uint16)
    packed = np.full((K // 2, N), 0xFF, np.uint8)
    s = np.full((K // 64, N), 0x3F00, np.uint16)
    z = np.full((K // 64, N), 14, np.uint8)
    y = host_bf16(ops.int4_g64_matmul(dev_bf16(x), dev(packed), dev_bf16(s), dev(z)))
    assert np.all(y == K * 0.5)


INT8_SHAPES = [(1, 64, 8), (16, 256, 128), (7, 512, 264), (16, 4096, 1024), (20, 320, 256)]


@pytest.mark.parametrize("M,K,N", INT8_SHAPES)
def test_int8_pc_matches_oracle(M, K, N):
    ops = _ops()
    rng = np.random.default_rng(2000 + M + K + N)
    x, w, s = quant.make_int8_case(rng, M, K, N)
    print(f"int8 case M={M} K={K} N={N}", flush=True)
    y = ops.int8_pc_matmul(dev_bf16(x), dev(w), dev(s))
    torch.cuda.synchronize()
    ref, _ = quant.int8_pc_matmul(x, w, s)
    assert_rel_close(host_bf16(y), ref, BF16_RTOL, f"int8 {M}x{K}x{N}")


def test_int8_pc_headline_shape():
    ops = _ops()
    rng = np.random.default_rng(0)
    M, K, N = 16, 4096, 14336
    x, w, s = quant.make_int8_case(rng, M, K, N)
    y = ops.int8_pc_matmul(dev_bf16(x), dev(w), dev(s))
    torch.cuda.synchronize()
    ref = cport.int8_pc_matmul(x, w, s)
    assert_rel_close(host_bf16(y), ref, BF16_RTOL, "int8 headline")


# Many rows (M >= 128): the qgemm kernel (N % 128 == 0; K split in two when
# the grid has fewer than 192 tiles) or, for other N, W dequantised to bf16 in
# the workspace and the bf16 GEMM.  The workload's M = 256 and 4096 rows at
# reduced K, N; ragged M; K of 1, 2, 3 and 5 steps of 64 (the kernel's loop
# tail); N = 776 and N = 64 take the dequantise-then-GEMM path.
LARGE_M_SHAPES = [(256, 4096, 2048), (4096, 512, 512), (300, 1024, 776), (512, 256, 14336),
                  (130, 192, 128), (256, 64, 64), (1000, 320, 192), (128, 128, 640), (300, 1024, 256),
                  (200, 384, 384)]


@pytest.mark.parametrize("M,K,N", LARGE_M_SHAPES)
def test_int4_g64_large_m_matches_oracle(M, K, N):
    ops = _ops()
    rng = np.random.default_rng(3000 + M + K + N)
    x, packed, s, z = quant.make_int4_case(rng, M, K, N)
    print(f"int4 large-M case M={M} K={K} N={N}", flush=True)
    y = ops.int4_g64_matmul(dev_bf16(x), dev(packed), dev_bf16(s), dev(z))
    torch.cuda.synchronize()
    ref = cport.int4_g64_matmul(x, packed, s, z)
    assert_rel_close(host_bf16(y), ref, BF16_RTOL, f"int4 {M}x{K}x{N}")


@pytest.mark.parametrize("M,K,N", LARGE_M_SHAPES)
def test_int8_pc_large_m_matches_oracle(M, K, N):
    ops = _ops()
    rng = np.random.default_rng(4000 + M + K + N)
    x, w, s = quant.make_int8_case(rng, M, K, N)
    print(f"int8 large-M case M={M} K={K} N={N}", flush=True)
    y = ops.int8_pc_matmul(dev_bf16(x), dev(w), dev(s))
    torch.cuda.synchronize()
    ref = cport.int8_pc_matmul(x, w, s)
    assert_rel_close(host_bf16(y), ref, BF16_RTOL, f"int8 {M}x{K}x{N}")


@pytest.mark.parametrize("fmt", ["int4", "int8"])
def test_many_row_paths_agree(monkeypatch, fmt):
    """M = 256 through the three paths: qgemm (default), dequantise-then-GEMM
    (MK_QMM_QG_M=0) and the streaming kernels (MK_QMM_DEQ_M=0 as well).  They
    differ in the bf16 rounding of the dequantised int4 weights and in
    summation order; all meet the oracle and each other at the workload's
    bf16 tolerance."""
    ops = _ops()
    rng = np.random.default_rng(77)
    M, K, N = 256, 2048, 1024
    if fmt == "int4":
        x, packed, s, z = quant.make_int4_case(rng, M, K, N)
        args = (dev_bf16(x), dev(packed), dev_bf16(s), dev(z))
        run, ref = ops.int4_g64_matmul, cport.int4_g64_matmul(x, packed, s, z)
    else:
        x, w, s = quant.make_int8_case(rng, M, K, N)
        args = (dev_bf16(x), dev(w), dev(s))
        run, ref = ops.int8_pc_matmul, cport.int8_pc_matmul(x, w, s)
    y_qg = host_bf16(run(*args))
    monkeypatch.setenv("MK_QMM_QG_M", "0")
    y_deq = host_bf16(run(*args))
    monkeypatch.setenv("MK_QMM_DEQ_M", "0")
    y_str = host_bf16(run(*args))
    torch.cuda.synchronize()
    for name, y in [("qgemm", y_qg), ("dequantise+GEMM", y_deq), ("streaming", y_str)]:
        assert_rel_close(y, ref, BF16_RTOL, f"{fmt} {name} path")
    assert_rel_close(y_qg, y_str, BF16_RTOL, f"{fmt} qgemm vs streaming")
    assert_rel_close(y_deq, y_str, BF16_RTOL, f"{fmt} dequantise+GEMM vs streaming")


@pytest.mark.parametrize("fmt", ["int4", "int8"])
def test_qgemm_kernel_many_row_tiles(monkeypatch, fmt):
    """The qgemm kernel itself over several 256-row tiles with a ragged last
    one (MK_QMM_DEQ_M=0 keeps larger M off the dequantise-then-GEMM path)."""
    ops = _ops()
    monkeypatch.setenv("MK_QMM_DEQ_M", "0")
    rng = np.random.default_rng(91)
    M, K, N = 1000, 320, 256
    if fmt == "int4":
        x, packed, s, z = quant.make_int4_case(rng, M, K, N)
        y = ops.int4_g64_matmul(dev_bf16(x), dev(packed), dev_bf16(s), dev(z))
        ref = cport.int4_g64_matmul(x, packed, s, z)
    else:
        x, w, s = quant.make_int8_case(rng, M, K, N)
        y = ops.int8_pc_matmul(dev_bf16(x), dev(w), dev(s))
        ref = cport.int8_pc_matmul(x, w, s)
    torch.cuda.synchronize()
    assert_rel_close(host_bf16(y), ref, BF16_RTOL, f"{fmt} qgemm {M}x{K}x{N}")


@pytest.mark.parametrize("fmt", ["int4", "int8"])
@pytest.mark.parametrize("M,K,N", [(256, 4096, 2048), (300, 1024, 256), (128, 256, 128)])
def test_qgemm_split_k(monkeypatch, fmt, M, K, N):
    """The qgemm kernel with its K split in two (the second arriver adds the
    other partial) against the unsplit kernel (MK_QG_KS=1) and the oracle; a
    repeated split call is bit-identical (two addends: the arrival order
    cannot change the sum), including after the unsplit call reused the
    workspace's counters."""
    ops = _ops()
    rng = np.random.default_rng(5000 + M + K + N)
    if fmt == "int4":
        x, packed, s, z = quant.make_int4_case(rng, M, K, N)
        args = (dev_bf16(x), dev(packed), dev_bf16(s), dev(z))
        run, ref = ops.int4_g64_matmul, cport.int4_g64_matmul(x, packed, s, z)
    else:
        x, w, s = quant.make_int8_case(rng, M, K, N)
        args = (dev_bf16(x), dev(w), dev(s))
        run, ref = ops.int8_pc_matmul, cport.int8_pc_matmul(x, w, s)
    print(f"qgemm split-K {fmt} M={M} K={K} N={N}", flush=True)
    y2 = host_bf16_bits(run(*args))
    monkeypatch.setenv("MK_QG_KS", "1")
    y1 = host_bf16_bits(run(*args))
    monkeypatch.delenv("MK_QG_KS")
    y2b = host_bf16_bits(run(*args))
    torch.cuda.synchronize()
    assert np.array_equal(y2, y2b)
    from oracle.bf16 import bf16_bits_to_f32
    assert_rel_close(bf16_bits_to_f32(y2), ref, BF16_RTOL, f"{fmt} qgemm split")
    assert_rel_close(bf16_bits_to_f32(y1), ref, BF16_RTOL, f"{fmt} qgemm unsplit")
    assert_rel_close(bf16_bits_to_f32(y2), bf16_bits_to_f32(y1), BF16_RTOL, f"{fmt} split vs unsplit")


@pytest.mark.parametrize("fmt", ["int4", "int8"])
@pytest.mark.parametrize("M,K,N", [(256, 4096, 14336), (256, 4096, 2048), (200, 1024, 1024)])
def test_qgemm_exchange_in_l2_matches_device_scope(monkeypatch, fmt, M, K, N):
    """The qgemm kernel's split-K exchange inside one XCD's L2 (taken when the
    placement probe has seen round-robin dealing and the grid keeps each
    tile's two K parts on one XCD) against the device-scope exchange
    (MK_QMM_XCH=device): both add the other partial to their own, so the
    outputs are bit-identical, on repeated calls too; the counters return to
    zero."""
    ops = _ops()
    rng = np.random.default_rng(6000 + M + K + N)
    if fmt == "int4":
        x, packed, s, z = quant.make_int4_case(rng, M, K, N)
        args = (dev_bf16(x), dev(packed), dev_bf16(s), dev(z))
        run, ref = ops.int4_g64_matmul, cport.int4_g64_matmul(x[:64], packed, s, z)
    else:
        x, w, s = quant.make_int8_case(rng, M, K, N)
        args = (dev_bf16(x), dev(w), dev(s))
        run, ref = ops.int8_pc_matmul, cport.int8_pc_matmul(x[:64], w, s)
    print(f"qgemm exchange {fmt} M={M} K={K} N={N}", flush=True)
    local = [host_bf16_bits(run(*args)) for _ in range(3)]
    monkeypatch.setenv("MK_QMM_XCH", "device")
    dev_ = host_bf16_bits(run(*args))
    torch.cuda.synchronize()
    for y in local:
        assert np.array_equal(y, dev_)
    from oracle.bf16 import bf16_bits_to_f32
    assert_rel_close(bf16_bits_to_f32(local[0])[:64], ref, BF16_RTOL, f"{fmt} qgemm {M}x{K}x{N} rows 0..63")
    ws = ops.workspace(1, "cuda:0")
    assert int(ws[: 64 * 1024].count_nonzero()) == 0


@pytest.mark.parametrize("fmt", ["int4", "int8"])
@pytest.mark.parametrize("M,K,N", [(256, 4096, 14336), (1000, 320, 256), (256, 64, 128), (200, 1024, 1024),
                                   (512, 2048, 640)])
def test_qgemm_warp_specialised_bit_identical(monkeypatch, fmt, M, K, N):
    """The warp-specialised qgemm kernel (producer waves stream and
    dequantise, consumer waves multiply) runs the same tile, k order,
    dequantisation and split as the one-wave-per-SIMD kernel
    (MK_QG_WS=0): the outputs are bit-identical, for split and unsplit K,
    one step (K = 64), ragged row tiles; and within the bf16 tolerance of
    the oracle on sampled rows."""
    ops = _ops()
    monkeypatch.setenv("MK_QMM_DEQ_M", "0")
    rng = np.random.default_rng(7000 + M + K + N)
    rows = np.array([0, 1, M // 2, M - 1])
    if fmt == "int4":
        x, packed, s, z = quant.make_int4_case(rng, M, K, N)
        args = (dev_bf16(x), dev(packed), dev_bf16(s), dev(z))
        run, ref = ops.int4_g64_matmul, cport.int4_g64_matmul(x[rows], packed, s, z)
    else:
        x, w, s = quant.make_int8_case(rng, M, K, N)
        args = (dev_bf16(x), dev(w), dev(s))
        run, ref = ops.int8_pc_matmul, cport.int8_pc_matmul(x[rows], w, s)
    print(f"qgemm warp-specialised {fmt} M={M} K={K} N={N}", flush=True)
    y_ws = [host_bf16_bits(run(*args)) for _ in range(2)]
    monkeypatch.setenv("MK_QG_WS", "0")
    y_old = host_bf16_bits(run(*args))
    torch.cuda.synchronize()
    assert np.array_equal(y_ws[0], y_old)
    assert np.array_equal(y_ws[1], y_old)
    from oracle.bf16 import bf16_bits_to_f32
    assert_rel_close(bf16_bits_to_f32(y_ws[0])[rows], ref, BF16_RTOL, f"{fmt} qgemm ws {M}x{K}x{N}")


def test_int4_g64_large_m_known_answer():
    """x = 1, q = 15, z = 14, s = 0.5 at M = 512: every output is K * 0.5."""
    ops = _ops()
    M, K, N = 512, 1024, 512
    x = torch.ones((M, K), dtype=torch.bfloat16, device="cuda:0")
    w = torch.full((K // 2, N), 0xFF, dtype=torch.uint8, device="cuda:0")
    s = torch.full((K // 64, N), 0.5, dtype=torch.bfloat16, device="cuda:0")
    z = torch.full((K // 64, N), 14, dtype=torch.uint8, device="cuda:0")
    y = ops.int4_g64_matmul(x, w, s, z)
    torch.cuda.synchronize()
    assert torch.all(y.float() == K * 0.5)


def test_workspace_too_small_is_rejected_before_launch():
    ops = _ops()
    from mi355x import _lib
    L = _lib.lib()
    M, K, N = 16, 4096, 1024  # 16 column tiles: K is split, a workspace is needed
    need = L.mk_qmatmul_workspace_bytes(_lib.MK_QFMT_INT4_G64, M, K, N)
    assert need > 0
    x = torch.zeros((M, K), dtype=torch.bfloat16, device="cuda:0")
    w = torch.zeros((K // 2, N), dtype=torch.uint8, device="cuda:0")
    s = torch.zeros((K // 64, N), dtype=torch.bfloat16, device="cuda:0")
    z = torch.zeros((K // 64, N), dtype=torch.uint8, device="cuda:0")
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda:0")
    ws = torch.zeros(16, dtype=torch.uint8, device="cuda:0")
    rc = L.mk_int4g64_matmul_bf16(x.data_ptr(), w.data_ptr(), s.data_ptr(), z.data_ptr(),
                                  y.data_ptr(), M, K, N, ws.data_ptr(), 16, None)
    assert rc == _lib.MK_EWORKSPACE
    assert b"workspace" in L.mk_last_error()


# Shapes that take the wide kernel: every group
# count per wave (G = 1, 2, 4), split-K factors 1..8 with the in-kernel
# last-arriver reduction, and two row blocks with a partial second block.
WIDE_SHAPES = [
    (16, 4096, 14336),   # the headline
    (16, 2048, 14336),
    (1, 8192, 8192),
    (20, 4096, 8192),    # two row blocks
    (1, 2048, 65536),    # no split at the 256-column tiles
]

# Wave layouts: (tile columns, column split).  256 / 1: every wave over all
# 256 columns; 256 / 2: waves split over two 128-column halves; 128 / 1:
# narrow tiles, every wave over all 128 columns.
WIDE_LAYOUTS = {"all-columns": ("256", "1"), "column-split": ("256", "2"), "narrow": ("128", "1")}


@pytest.mark.parametrize("M,K,N,layout", [(M, K, N, lay) for (M, K, N) in WIDE_SHAPES + [(16, 4096, 4992)]
                                             for lay in WIDE_LAYOUTS if N % int(WIDE_LAYOUTS[lay][0]) == 0])
def test_int4_wide_kernel_matches_oracle(monkeypatch, M, K, N, layout):
    """Every wave layout of the wide kernel against the C oracle, on the
    shapes whose N the layout's tile divides (N = 4992 = 39 x 128: narrow
    tiles only, with 39 tiles the exchange goes through device scope)."""
    ops = _ops()
    tn, cs = WIDE_LAYOUTS[layout]
    monkeypatch.setenv("MK_QMM_WIDE_TN", tn)
    monkeypatch.setenv("MK_QMM_WIDE_CS", cs)
    rng = np.random.default_rng(7 * M + K + N)
    x, packed, s, z = quant.make_int4_case(rng, M, K, N)
    print(f"int4 wide case M={M} K={K} N={N} layout={layout}", flush=True)
    y = ops.int4_g64_matmul(dev_bf16(x), dev(packed), dev_bf16(s), dev(z))
    torch.cuda.synchronize()
    ref = cport.int4_g64_matmul(x, packed, s, z)
    assert_rel_close(host_bf16(y), ref, BF16_RTOL, f"int4 wide {M}x{K}x{N} {layout}")


@pytest.mark.parametrize("nw,tn", [("8", "256"), ("8", "128"), ("4", "256")], ids=["8w", "8w-narrow", "4w"])
@pytest.mark.parametrize("M,K,N", [(16, 4096, 14336), (20, 4096, 8192), (1, 8192, 8192), (40, 2048, 14336),
                                   (16, 4096, 2048)])
def test_int4_wide_exchange_in_l2_matches_device_scope(monkeypatch, nw, tn, M, K, N):
    """The split-K exchange inside one XCD's L2 (taken when the placement
    probe has seen round-robin dealing) against the device-scope exchange
    (MK_QMM_XCH=device): both sum the partials in k order from memory, so the
    outputs are bit-identical; with 8 and 4 waves per workgroup, 256- and
    128-column tiles, one and several row blocks (2D grids), K split 2, 4
    and 8 ways (N = 2048 at 128 columns: 8)."""
    ops = _ops()
    monkeypatch.setenv("MK_QMM_WIDE_NW", nw)
    monkeypatch.setenv("MK_QMM_WIDE_TN", tn)
    rng = np.random.default_rng(5 * M + K + N)
    x, packed, s, z = quant.make_int4_case(rng, M, K, N)
    args = (dev_bf16(x), dev(packed), dev_bf16(s), dev(z))
    print(f"int4 wide exchange case M={M} K={K} N={N} waves={nw} tile={tn}", flush=True)
    local = [host_bf16_bits(ops.int4_g64_matmul(*args)) for _ in range(3)]
    monkeypatch.setenv("MK_QMM_XCH", "device")
    dev_ = host_bf16_bits(ops.int4_g64_matmul(*args))
    torch.cuda.synchronize()
    for y in local:
        assert np.array_equal(y, dev_)
    ref = cport.int4_g64_matmul(x, packed, s, z)
    assert_rel_close(bf16_bits_to_f32(local[0]), ref, BF16_RTOL, f"int4 wide {M}x{K}x{N} waves={nw} tile={tn}")
    ws = ops.workspace(1, "cuda:0")
    assert int(ws[: 64 * 1024].count_nonzero()) == 0


def test_int4_wide_kernel_deterministic_across_calls():
    """The split-K sum runs in k order whichever workgroup arrives last, and
    every call returns the arrival counters to zero: repeated calls give the
    same bits."""
    ops = _ops()
    rng = np.random.default_rng(21)
    x, packed, s, z = quant.make_int4_case(rng, 16, 4096, 14336)
    args = (dev_bf16(x), dev(packed), dev_bf16(s), dev(z))
    first = host_bf16_bits(ops.int4_g64_matmul(*args))
    for _ in range(5):
        assert np.array_equal(host_bf16_bits(ops.int4_g64_matmul(*args)), first)


def test_int4_wide_and_split_k_paths_share_a_workspace():
    """Wide-kernel calls (counters in the workspace's first 64 KB) interleaved
    with 64-column split-K calls and the dequantise-then-GEMM path (both
    write after the counters) through one workspace."""
    ops = _ops()
    rng = np.random.default_rng(23)
    for (M, K, N) in [(16, 4096, 14336), (16, 4096, 1024), (1, 8192, 8192), (5, 4096, 512),
                      (800, 1024, 2048), (16, 4096, 14336)]:
        x, packed, s, z = quant.make_int4_case(rng, M, K, N)
        y = ops.int4_g64_matmul(dev_bf16(x), dev(packed), dev_bf16(s), dev(z))
        torch.cuda.synchronize()
        ref = cport.int4_g64_matmul(x, packed, s, z)
        assert_rel_close(host_bf16(y), ref, BF16_RTOL, f"int4 mixed {M}x{K}x{N}")
    # Every completed call leaves the arrival counters at zero.
    ws = ops.workspace(1, "cuda:0")
    assert int(ws[: 64 * 1024].count_nonzero()) == 0


# Shapes that take the 256-column int8 kernel (plan "wide8"): steps per wave
# S = 4, 8, 16, split-K factors 1, 2, 4 with the in-kernel last-arriver
# reduction, a partial second row block, and N not a multiple of the 64-column
# kernels' 192-workgroup split.
WIDE8_SHAPES = [
    (16, 4096, 14336),   # ks = 4, S = 4 (the headline plan)
    (20, 4096, 14336),   # two row blocks (the second has 4 rows), ks = 2, S = 8
    (64, 4096, 14336),   # four row blocks, ks = 1, S = 16
    (1, 4096, 8192),     # ks = 4, S = 4, 128 workgroups
    (16, 8192, 14336),   # ks = 4, S = 8
]


@pytest.mark.parametrize("cs", ["1", "2"], ids=["all-columns", "column-split"])
@pytest.mark.parametrize("M,K,N", WIDE8_SHAPES)
def test_int8_wide_kernel_matches_oracle(M, K, N, cs, monkeypatch):
    """Both wave layouts of the wide int8 kernel (MK_QMM_WIDE8_CS: every
    wave over all 256 columns, or waves split over two 128-column halves
    with twice the k steps) against the C oracle."""
    ops = _ops()
    monkeypatch.setenv("MK_QMM_WIDE8_CS", cs)
    rng = np.random.default_rng(11 * M + K + N)
    x, w, s = quant.make_int8_case(rng, M, K, N)
    print(f"int8 wide case M={M} K={K} N={N} cs={cs}", flush=True)
    y = ops.int8_pc_matmul(dev_bf16(x), dev(w), dev(s))
    torch.cuda.synchronize()
    ref = cport.int8_pc_matmul(x, w, s)
    assert_rel_close(host_bf16(y), ref, BF16_RTOL, f"int8 wide {M}x{K}x{N} cs={cs}")


def test_int8_wide_kernel_is_planned_and_deterministic(monkeypatch):
    """The headline shape plans the wide int8 kernel (its workspace holds the
    split-K partials), repeated calls give the same bits, the arrival
    counters return to zero, and the 64-column kernel (MK_QMM_WIDE=0) agrees
    within the bf16 tolerance."""
    ops = _ops()
    from mi355x import _lib
    M, K, N = 16, 4096, 14336
    assert _lib.lib().mk_qmatmul_workspace_bytes(_lib.MK_QFMT_INT8_PC, M, K, N) == 64 * 1024 + 4 * 56 * 16 * 256 * 4
    rng = np.random.default_rng(29)
    x, w, s = quant.make_int8_case(rng, M, K, N)
    args = (dev_bf16(x), dev(w), dev(s))
    first = host_bf16_bits(ops.int8_pc_matmul(*args))
    for _ in range(4):
        assert np.array_equal(host_bf16_bits(ops.int8_pc_matmul(*args)), first)
    ws = ops.workspace(1, "cuda:0")
    assert int(ws[: 64 * 1024].count_nonzero()) == 0
    monkeypatch.setenv("MK_QMM_WIDE", "0")
    assert _lib.lib().mk_qmatmul_workspace_bytes(_lib.MK_QFMT_INT8_PC, M, K, N) == 0
    y64 = ops.int8_pc_matmul(*args)
    torch.cuda.synchronize()
    ref = cport.int8_pc_matmul(x, w, s)
    assert_rel_close(host_bf16(y64), ref, BF16_RTOL, "int8 64-column kernel")


# The 64-column kernels' split-K: partials combined in the kernel by the last
# arriving workgroup (default) or by the separate reduce pass
# (MK_QMM_REDUCE_PASS=1); both sum in k order from zero, so the results are
# the same bits.  Shapes: per-shard (N = 1792), streaming ks = 2 / 4 with a
# ragged row block, and the generic kernels (N % 16 != 0).
SPLIT_SHAPES = [(16, 4096, 1792), (5, 2048, 1024), (20, 4096, 512), (3, 4096, 1032), (1, 8192, 256)]


@pytest.mark.parametrize("fmt", ["int4", "int8"])
@pytest.mark.parametrize("M,K,N", SPLIT_SHAPES)
def test_split_k_exchange_matches_reduce_pass(monkeypatch, fmt, M, K, N):
    ops = _ops()
    from mi355x import _lib
    rng = np.random.default_rng(M + K + N + len(fmt))
    if fmt == "int4":
        x, p, s, z = quant.make_int4_case(rng, M, K, N)
        args = (dev_bf16(x), dev(p), dev_bf16(s), dev(z))
        run, ref = ops.int4_g64_matmul, cport.int4_g64_matmul(x, p, s, z)
    else:
        x, w, s = quant.make_int8_case(rng, M, K, N)
        args = (dev_bf16(x), dev(w), dev(s))
        run, ref = ops.int8_pc_matmul, cport.int8_pc_matmul(x, w, s)
    print(f"split-k exchange {fmt} M={M} K={K} N={N}", flush=True)
    fmt_code = _lib.MK_QFMT_INT4_G64 if fmt == "int4" else _lib.MK_QFMT_INT8_PC
    assert _lib.lib().mk_qmatmul_workspace_bytes(fmt_code, M, K, N) > 0  # the shape splits K
    first = host_bf16_bits(run(*args))
    for _ in range(3):  # the counters return to zero: repeated calls, same bits
        assert np.array_equal(host_bf16_bits(run(*args)), first)
    assert int(ops.workspace(1, "cuda:0")[: 64 * 1024].count_nonzero()) == 0
    monkeypatch.setenv("MK_QMM_REDUCE_PASS", "1")
    two_pass = host_bf16_bits(run(*args))
    assert np.array_equal(two_pass, first)
    assert_rel_close(bf16_bits_to_f32(first), ref, BF16_RTOL, f"{fmt} split-K {M}x{K}x{N}")
