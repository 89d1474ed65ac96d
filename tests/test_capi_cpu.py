"""Host-only checks of the C-ABI (no GPU needed): the built library loads,
exports every entry point include/mk_kernels.h and include/mk_runtime.h
declare, and rejects bad arguments on the host before any launch."""

import ctypes
import os
import re

import pytest

from mi355x import _lib

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared(header, prefix="mk_"):
    text = open(os.path.join(REPO, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(" + prefix + r"[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported_and_bound():
    L = _lib.lib()
    names = _declared("mk_kernels.h")
    assert names, "no declarations parsed"
    for n in names:
        assert hasattr(L, n), f"{n} declared but not exported"
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature in mi355x/_lib.py"


def test_every_runtime_symbol_is_exported_and_bound():
    L = _lib.lib()
    names = _declared("mk_runtime.h", "mkrt_")
    assert len(names) >= 30, names
    for n in names:
        assert hasattr(L, n), f"{n} declared but not exported"
        assert n in _lib.RUNTIME_SIGNATURES, f"{n} has no ctypes signature in mi355x/_lib.py"


def test_workspace_query_is_host_only():
    L = _lib.lib()
    assert L.mk_qmatmul_workspace_bytes(_lib.MK_QFMT_INT4_G64, 16, 4096, 14336) >= 0
    assert L.mk_qmatmul_workspace_bytes(_lib.MK_QFMT_INT4_G64, 16, 4096, 1024) > 0
    assert L.mk_qmatmul_workspace_bytes(_lib.MK_QFMT_INT4_G64, 16, 4000, 14336) == -1
    assert L.mk_qmatmul_workspace_bytes(7, 16, 4096, 14336) == -1


@pytest.mark.parametrize("M,K,N,code", [
    (0, 64, 8, _lib.MK_EINVAL),
    (16, 100, 8, _lib.MK_EINVAL),   # K not a multiple of 64
    (16, 64, 12, _lib.MK_EINVAL),   # N not a multiple of 8
])
def test_bad_shapes_rejected_before_launch(M, K, N, code):
    L = _lib.lib()
    fake = ctypes.c_void_p(0x1000)  # never dereferenced: validation fails first
    rc = L.mk_int4g64_matmul_bf16(fake, fake, fake, fake, fake, M, K, N, fake, 1 << 30, None)
    assert rc == code
    assert L.mk_last_error()
    rc = L.mk_int8pc_matmul_bf16(fake, fake, fake, fake, M, K, N, fake, 1 << 30, None)
    assert rc == code


def test_null_pointer_rejected():
    L = _lib.lib()
    rc = L.mk_int4g64_matmul_bf16(None, None, None, None, None, 16, 64, 8, None, 0, None)
    assert rc == _lib.MK_EINVAL
    assert b"null" in L.mk_last_error()


def test_missing_workspace_rejected():
    L = _lib.lib()
    fake = ctypes.c_void_p(0x1000)
    # N = 1024 gives 16 column tiles, so K is split across workgroups and a
    # workspace is required; validation fails before any launch.
    assert L.mk_qmatmul_workspace_bytes(_lib.MK_QFMT_INT4_G64, 16, 4096, 1024) > 0
    rc = L.mk_int4g64_matmul_bf16(fake, fake, fake, fake, fake, 16, 4096, 1024, None, 0, None)
    assert rc == _lib.MK_EWORKSPACE


def test_elementwise_program_validated_on_host():
    L = _lib.lib()
    fake = ctypes.c_void_p(0x1000)
    ins = (_lib.EwInstr * 1)(_lib.EwInstr(_lib.EW["ADD"], 0, 1, 2, 0, 0.0))
    ptrs = (ctypes.c_void_p * 1)(fake.value)
    numel = (ctypes.c_int64 * 1)(16)
    rc = L.mk_elementwise(_lib.MK_DT_F32, ins, 1, ptrs, numel, 1, 0, fake, 16, None)
    assert rc == _lib.MK_EINVAL and b"undefined slot" in L.mk_last_error()
    ins = (_lib.EwInstr * 1)(_lib.EwInstr(_lib.EW["LOAD"], 0, 0, 0, 0, 0.0))
    numel = (ctypes.c_int64 * 1)(7)  # neither 1 nor n
    rc = L.mk_elementwise(_lib.MK_DT_F32, ins, 1, ptrs, numel, 1, 0, fake, 16, None)
    assert rc == _lib.MK_EINVAL


def test_rowops_reject_bad_args_on_host():
    L = _lib.lib()
    fake = ctypes.c_void_p(0x1000)
    assert L.mk_softmax_lastdim(_lib.MK_DT_F32, fake, fake, 0, 8, None) == _lib.MK_EINVAL
    assert L.mk_softmax_lastdim(7, fake, fake, 1, 8, None) == _lib.MK_EUNSUPPORTED
    assert L.mk_rmsnorm_lastdim(_lib.MK_DT_F32, fake, None, fake, 1, 8, 1e-6, None) == _lib.MK_EINVAL
    assert L.mk_reduce_lastdim(_lib.MK_DT_F32, 9, fake, fake, 1, 8, None) == _lib.MK_EUNSUPPORTED
    assert L.mk_gemm_bf16(fake, fake, fake, 1, 16, 12, 16, 0, None) == _lib.MK_EUNSUPPORTED


def test_gemm_routes_fit_and_reject_on_host():
    """Which route takes which product, and the host-side refusals of a
    route call (nothing launched)."""
    L = _lib.lib()
    R, E = _lib.GEMM_ROUTES, _lib
    fits = lambda r, M, N, K, epi=E.MK_EPI_NONE, f32=0: L.mk_gemm_bf16_route_fits(R[r], M, N, K, epi, f32)
    assert fits("ring", 256, 512, 32) and not fits("ring", 384, 512, 32) and not fits("ring", 256, 512, 48)
    assert fits("pipe", 256, 256, 320) and not fits("pipe", 256, 256, 288)
    assert fits("persist", 512, 256, 128) and not fits("persist", 512, 256, 160)
    assert not fits("persist", 512, 256, 64, f32=1) and not fits("persist", 512, 256, 64, E.MK_EPI_SWIGLU_PAIRS)
    assert fits("short", 384, 640, 256) and not fits("short", 384, 640, 288) and not fits("short", 200, 640, 64)
    assert fits("reg256", 256, 256, 64) and not fits("reg256", 256, 256, 32)
    assert fits("generic128", 200, 264, 72) and fits("generic256", 7, 8, 8)
    assert not fits("generic128", 256, 256, 64, E.MK_EPI_SWIGLU_PAIRS)
    assert not fits("default", 256, 256, 64)
    fake = ctypes.c_void_p(0x1000)
    assert L.mk_gemm_bf16_route(fake, fake, fake, None, 0, 1, 256, 256, 64, 0, 99, None) == E.MK_EINVAL
    assert L.mk_gemm_bf16_route(fake, fake, fake, None, 0, 1, 256, 256, 160, 0, R["persist"], None) == \
        E.MK_EUNSUPPORTED
    assert b"route 3" in L.mk_last_error()


def test_gemm_route_table_file_round_trip(tmp_path):
    """The route table's text file: load merges entries (any device's), save
    writes them back byte for byte (sorted by key), and a file with another
    header (another format, or a table measured against another build of the
    library) or a malformed line is refused with the table unchanged."""
    L = _lib.lib()
    L.mk_gemm_autotune_clear()
    hdr = L.mk_gemm_autotune_header().decode()
    assert hdr.startswith("mk-gemm-autotune 1 build ") and " " not in hdr[len("mk-gemm-autotune 1 build "):]
    text = (hdr + "\n"
            "gfx950 256 1 4096 4096 4096 0 0 2 112.500\n"
            "gfx950 256 16 2048 2048 128 0 0 3 50.125\n"
            "gfx942 304 1 384 640 64 1 0 4 9.000\n")
    src = tmp_path / "routes.txt"
    src.write_text(text)
    assert L.mk_gemm_autotune_load(str(src).encode()) == 3
    out = tmp_path / "saved.txt"
    assert L.mk_gemm_autotune_save(str(out).encode()) == 3
    lines = out.read_text().splitlines()
    assert lines[0] == hdr and sorted(lines[1:]) == lines[1:]
    assert set(lines[1:]) == set(text.splitlines()[1:])
    good = "gfx950 256 1 64 64 64 0 0 2 1.0\n"
    for bad in ("mk-gemm-autotune 1\n" + good,  # no build stamp
                "mk-gemm-autotune 1 build Jan_1_2000_00:00:00\n" + good,  # another build's table
                hdr + "X\n" + good, "mk-gemm-autotune 2\n",
                hdr + "\ngfx950 256 1 64 64 64 0 0 9 1.0\n",
                hdr + "\ngfx950 256 1 64 64 0 0 2 1.0\n",
                hdr + "\ngfx950 256 1 64 64 64 0 0 2 1.0 extra\n"):
        f = tmp_path / "bad.txt"
        f.write_text(bad)
        assert L.mk_gemm_autotune_load(str(f).encode()) == -_lib.MK_EINVAL, bad
        assert L.mk_last_error()
    assert L.mk_gemm_autotune_load(str(tmp_path / "missing.txt").encode()) == -_lib.MK_EINVAL
    assert L.mk_gemm_autotune_save(str(out).encode()) == 3  # unchanged by the refused loads
    L.mk_gemm_autotune_clear()
    assert L.mk_gemm_autotune_save(str(out).encode()) == 0
