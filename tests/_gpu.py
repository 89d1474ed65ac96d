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


def assert_rel_close(out, ref, rtol, what=""):
    """max|out - ref| / max|ref| <= rtol (the reference's GEMM error measure,
    tests/test_f32_gemm_precision.py:25-27) and every element within
    rtol*|ref| + rtol*0.1*max|ref|."""
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
    assert rel <= rtol, f"{what}: normwise rel err {rel:.3e} > {rtol}"
    bad = err > rtol * np.abs(r) + 0.1 * rtol * scale
    assert not bad.any(), f"{what}: {int(bad.sum())} elements outside tolerance, worst {float(err.max()):.3e}"
