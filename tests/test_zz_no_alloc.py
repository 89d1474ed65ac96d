"""The no-allocation int4 entry point (mk_int4g64_matmul_bf16_noalloc) against
the workspace entry point (mk_int4g64_matmul_bf16) through the C-ABI: two
calls in a row, the second with a smaller input, each bit-identical to the
workspace call (the same plan and kernels run) and within the workload's
bf16 tolerance of the oracle; a shape whose workspace exceeds the array is
rejected before any launch."""

import numpy as np
import pytest

from _gpu import BF16_RTOL, assert_rel_close, dev, dev_bf16, host_bf16, host_bf16_bits, need_gpu, torch
from oracle import cport, quant

pytestmark = pytest.mark.gpu


def _noalloc(L, x, w, s, z, M, K, N):
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda:0")
    stream = torch.cuda.current_stream().cuda_stream
    rc = L.mk_int4g64_matmul_bf16_noalloc(x.data_ptr(), w.data_ptr(), s.data_ptr(), z.data_ptr(), y.data_ptr(),
                                          M, K, N, stream)
    assert rc == 0, L.mk_last_error()
    return y


def test_noalloc_matches_workspace_entry_point():
    need_gpu()
    from mi355x import _lib, ops
    L = _lib.lib()
    rng = np.random.default_rng(70)
    # Headline shape (wide kernel, split-K with the in-kernel exchange through
    # the array's counters), then a smaller one (64-column kernel, split-K
    # partials and the reduce pass) and the headline again.
    for (M, K, N) in [(16, 4096, 14336), (5, 4096, 512), (16, 4096, 14336)]:
        print(f"[noalloc] M={M} K={K} N={N}", flush=True)
        x, packed, s, z = quant.make_int4_case(rng, M, K, N)
        args = (dev_bf16(x), dev(packed), dev_bf16(s), dev(z))
        y_na = host_bf16_bits(_noalloc(L, *args, M, K, N))
        y_ws = host_bf16_bits(ops.int4_g64_matmul(*args))
        torch.cuda.synchronize()
        assert np.array_equal(y_na, y_ws), f"noalloc differs from the workspace call at {M}x{K}x{N}"
        ref = cport.int4_g64_matmul(x, packed, s, z)
        from oracle.bf16 import bf16_bits_to_f32
        assert_rel_close(bf16_bits_to_f32(y_na), ref, BF16_RTOL, f"noalloc {M}x{K}x{N}")


def test_noalloc_rejects_shapes_beyond_the_array():
    need_gpu()
    from mi355x import _lib
    L = _lib.lib()
    M, K, N = 4096, 4096, 14336  # dequantise-then-GEMM: 117 MB of workspace
    assert L.mk_qmatmul_workspace_bytes(_lib.MK_QFMT_INT4_G64, M, K, N) > 8 << 20
    # Real device buffers of the full shapes (contents unused: the size check
    # fails before any launch).  Should that check ever regress, the call
    # reads and writes valid memory and fails the asserts below; it cannot
    # touch an address that was never allocated.
    dev0 = dict(device="cuda:0")
    x = torch.empty((M, K), dtype=torch.bfloat16, **dev0)
    w = torch.empty((K // 2, N), dtype=torch.uint8, **dev0)
    s = torch.empty((K // 64, N), dtype=torch.bfloat16, **dev0)
    z = torch.empty((K // 64, N), dtype=torch.uint8, **dev0)
    y = torch.empty((M, N), dtype=torch.bfloat16, **dev0)
    stream = torch.cuda.current_stream().cuda_stream
    rc = L.mk_int4g64_matmul_bf16_noalloc(x.data_ptr(), w.data_ptr(), s.data_ptr(), z.data_ptr(), y.data_ptr(),
                                          M, K, N, stream)
    torch.cuda.synchronize()
    assert rc == _lib.MK_EWORKSPACE
    assert b"no-allocation" in L.mk_last_error()


def test_noalloc_many_rows_runs_unsplit():
    """M = 256 at the workload's K, N: the many-row kernel's split-K partials
    (28 MB) do not fit the array, so this entry point runs it unsplit; the
    result agrees with the workspace entry point (split) at the bf16
    tolerance, and both with the oracle on sampled rows.  A smaller shape
    whose partials fit runs split and is bit-identical."""
    need_gpu()
    from mi355x import _lib, ops
    from oracle.bf16 import bf16_bits_to_f32
    L = _lib.lib()
    rng = np.random.default_rng(71)
    M, K, N = 256, 4096, 14336
    print(f"[noalloc] M={M} K={K} N={N}", flush=True)
    x, packed, s, z = quant.make_int4_case(rng, M, K, N)
    args = (dev_bf16(x), dev(packed), dev_bf16(s), dev(z))
    y_na = host_bf16_bits(_noalloc(L, *args, M, K, N))
    y_ws = host_bf16_bits(ops.int4_g64_matmul(*args))
    torch.cuda.synchronize()
    assert_rel_close(bf16_bits_to_f32(y_na), bf16_bits_to_f32(y_ws), BF16_RTOL, "noalloc vs workspace at M=256")
    rows = np.array([0, 1, 127, 255])
    ref = cport.int4_g64_matmul(x[rows], packed, s, z)
    assert_rel_close(bf16_bits_to_f32(y_na)[rows], ref, BF16_RTOL, "noalloc M=256 rows vs oracle")
    M2, K2, N2 = 256, 1024, 2048  # 4 MB of partials: split here too
    print(f"[noalloc] M={M2} K={K2} N={N2}", flush=True)
    x2, p2, s2, z2 = quant.make_int4_case(rng, M2, K2, N2)
    a2 = (dev_bf16(x2), dev(p2), dev_bf16(s2), dev(z2))
    y2_na = host_bf16_bits(_noalloc(L, *a2, M2, K2, N2))
    y2_ws = host_bf16_bits(ops.int4_g64_matmul(*a2))
    torch.cuda.synchronize()
    assert np.array_equal(y2_na, y2_ws)
