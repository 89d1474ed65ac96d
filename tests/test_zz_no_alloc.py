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
    fake = 0x1000  # never dereferenced: the size check fails first
    rc = L.mk_int4g64_matmul_bf16_noalloc(fake, fake, fake, fake, fake, M, K, N, None)
    assert rc == _lib.MK_EWORKSPACE
    assert b"no-allocation" in L.mk_last_error()
