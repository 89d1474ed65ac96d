"""torch-tensor wrappers over the kernel C-ABI.

torch supplies device memory and the current HIP stream; every computation
runs in the gfx950 kernels of libmk_kernels.so.  bf16 tensors may be passed as
torch.bfloat16 or as int16/uint16 bit patterns.
"""

import torch

from . import _lib
from ._lib import check, lib

_WORKSPACES = {}


def _ptr(t):
    return t.data_ptr() if t is not None else None


def _stream(device):
    return torch.cuda.current_stream(device).cuda_stream


def _require(t, dtypes, name):
    if not t.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if t.dtype not in dtypes:
        raise ValueError(f"{name} has dtype {t.dtype}, expected one of {dtypes}")


_BF16 = (torch.bfloat16, torch.int16, torch.uint16)


def workspace(nbytes, device):
    """A device workspace of at least nbytes, cached per device (the kernels
    need no particular initial contents)."""
    key = torch.device(device).index or 0
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.zeros(max(int(nbytes), 256), dtype=torch.uint8, device=device)
        _WORKSPACES[key] = ws
    return ws


def int4_g64_matmul(x, w_packed, scale, zero, out=None):
    """y = x @ ((w - zero) * scale): x bf16 [M,K], w uint8 [K/2,N], scale bf16
    [K/64,N], zero uint8 [K/64,N] -> bf16 [M,N]."""
    _require(x, _BF16, "x")
    _require(w_packed, (torch.uint8,), "w_packed")
    _require(scale, _BF16, "scale")
    _require(zero, (torch.uint8,), "zero")
    M, K = x.shape
    N = w_packed.shape[1]
    if w_packed.shape[0] * 2 != K or scale.shape != (K // 64, N) or zero.shape != (K // 64, N):
        raise ValueError("int4_g64_matmul: inconsistent shapes")
    y = out if out is not None else torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    nb = lib().mk_qmatmul_workspace_bytes(_lib.MK_QFMT_INT4_G64, M, K, N)
    ws = workspace(nb, x.device) if nb > 0 else None
    check(lib().mk_int4g64_matmul_bf16(_ptr(x), _ptr(w_packed), _ptr(scale), _ptr(zero), _ptr(y),
                                       M, K, N, _ptr(ws), max(nb, 0), _stream(x.device)))
    return y


def int8_pc_matmul(x, w, scale, out=None):
    """y = x @ (w * scale): x bf16 [M,K], w int8 [K,N], scale f32 [N] -> bf16 [M,N]."""
    _require(x, _BF16, "x")
    _require(w, (torch.int8,), "w")
    _require(scale, (torch.float32,), "scale")
    M, K = x.shape
    N = w.shape[1]
    if w.shape[0] != K or scale.shape != (N,):
        raise ValueError("int8_pc_matmul: inconsistent shapes")
    y = out if out is not None else torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    nb = lib().mk_qmatmul_workspace_bytes(_lib.MK_QFMT_INT8_PC, M, K, N)
    ws = workspace(nb, x.device) if nb > 0 else None
    check(lib().mk_int8pc_matmul_bf16(_ptr(x), _ptr(w), _ptr(scale), _ptr(y), M, K, N, _ptr(ws),
                                      max(nb, 0), _stream(x.device)))
    return y


def _bmk(a, b):
    if a.dim() == 2:
        a2, b2 = a.unsqueeze(0), b.unsqueeze(0)
    else:
        a2, b2 = a, b
    if a2.dim() != 3 or b2.dim() != 3 or a2.shape[0] != b2.shape[0] or a2.shape[2] != b2.shape[1]:
        raise ValueError(f"gemm: incompatible shapes {tuple(a.shape)} x {tuple(b.shape)}")
    return a2.shape[0], a2.shape[1], b2.shape[2], a2.shape[2]


def gemm_bf16(a, b, out_f32=False, out=None):
    """[batch,] M x K @ K x N in bf16 with f32 accumulation -> bf16 (or f32)."""
    _require(a, _BF16, "a")
    _require(b, _BF16, "b")
    batch, M, N, K = _bmk(a, b)
    shape = (M, N) if a.dim() == 2 else (batch, M, N)
    c = out if out is not None else torch.empty(
        shape, dtype=torch.float32 if out_f32 else torch.bfloat16, device=a.device)
    check(lib().mk_gemm_bf16(_ptr(a), _ptr(b), _ptr(c), batch, M, N, K, 1 if out_f32 else 0,
                             _stream(a.device)))
    return c


def gemm_f32(a, b, out=None):
    """[batch,] M x K @ K x N in f32."""
    _require(a, (torch.float32,), "a")
    _require(b, (torch.float32,), "b")
    batch, M, N, K = _bmk(a, b)
    shape = (M, N) if a.dim() == 2 else (batch, M, N)
    c = out if out is not None else torch.empty(shape, dtype=torch.float32, device=a.device)
    check(lib().mk_gemm_f32(_ptr(a), _ptr(b), _ptr(c), batch, M, N, K, _stream(a.device)))
    return c
