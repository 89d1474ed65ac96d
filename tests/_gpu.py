"""Helpers shared by the GPU parity tests: device transfer of bf16 bit
patterns and the workload's tolerances (bf16 rel 2e-2, f32 rel 1e-5)."""

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle.bf16 import bf16_bits_to_f32  # noqa: E402

BF16_RTOL = 2e-2
F32_RTOL = 1e-5


def need_gpu():
    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no GPU is visible")


def dev_bf16(bits):
    """uint16 bf16 bit patterns (numpy) -> torch.bfloat16 on cuda:0."""
    t = torch.from_numpy(np.ascontiguousarray(bits).view(np.int16))
    return t.view(torch.bfloat16).to("cuda:0")


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")


def host_bf16_bits(t):
    return t.detach().view(torch.int16).cpu().numpy().view(np.uint16)


def host_bf16(t):
    return bf16_bits_to_f32(host_bf16_bits(t))


U_F32 = 2.0 ** -24  # f32 unit roundoff


def gamma(n, u=U_F32):
    """gamma_n = n u / (1 - n u): the classical bound on the relative error
    of n rounded operations (Higham, Accuracy and Stability of Numerical
    Algorithms, 2nd ed., Lemma 3.1)."""
    return n * u / (1.0 - n * u)


def f32_sum_bound(abs_terms_sum, n):
    """Per-element bound on |fl(sum) - sum| for n terms summed in f32 in any
    order: gamma_{n-1} * sum |t_i| (Higham Eq. 4.4).  The unit roundoff is
    doubled to 2^-23 so the bound also holds for an adder that truncates
    instead of rounding to nearest (the matrix cores' internal order and
    rounding are not published)."""
    return gamma(max(n - 1, 1), 2 * U_F32) * np.asarray(abs_terms_sum, dtype=np.float64)


def assert_rel_close(out, ref, rtol, what="", elem=None):
    """Normwise: max|out - ref| / max|ref| <= rtol (the reference's error
    measure, tests/test_f32_gemm_precision.py:25-27).

    Elementwise, one of:
      elem None   -- every element within rtol*|ref| + 0.1*rtol*max|ref|;
      elem array  -- every element within its own derived bound (for
                     example f32_sum_bound for an f32 reduction or an f32
                     accumulation of exact products);
      elem False  -- no elementwise check (the normwise one only)."""
    out = np.asarray(out, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert out.shape == ref.shape, (out.shape, ref.shape)
    assert np.array_equal(np.isnan(out), np.isnan(ref)), f"{what}: NaN mask differs"
    fin = ~np.isnan(ref)
    o, r = out[fin], ref[fin]
    if r.size == 0:
        return
    scale = np.max(np.abs(r))
    scale = scale if scale > 0 else 1.0
    err = np.abs(o - r)
    rel = float(np.max(err) / scale)
    print(f"{what}: normwise rel err {rel:.3e} (bound {rtol})", flush=True)
    assert rel <= rtol, f"{what}: normwise rel err {rel:.3e} > {rtol}"
    if elem is False:
        return
    if elem is None:
        bound = rtol * np.abs(r) + 0.1 * rtol * scale
    else:
        bound = np.broadcast_to(np.asarray(elem, dtype=np.float64), out.shape)[fin]
    bad = err > bound
    assert not bad.any(), (f"{what}: {int(bad.sum())} elements outside the elementwise bound, "
                           f"worst excess {float((err - bound).max()):.3e}")
