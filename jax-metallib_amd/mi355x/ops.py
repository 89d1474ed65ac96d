"""torch-tensor wrappers over the kernel C-ABI.

torch supplies device memory and the current HIP stream; every computation
runs in the gfx950 kernels of libmk_kernels.so.  bf16 tensors may be passed as
torch.bfloat16 or as int16/uint16 bit patterns.
"""

import ctypes

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


def workspace(nbytes, device, stream=None):
    """A device workspace of at least nbytes, cached per (device, stream):
    calls that share a workspace must be ordered, and calls on one stream
    are.  It starts zero-filled (its first 64 KB are arrival counters that
    every completed call leaves at zero).  A workspace that grows is replaced;
    torch's caching allocator keeps the old block until the stream's work on
    it is done."""
    dev = torch.device(device)
    index = dev.index if dev.index is not None else torch.cuda.current_device()
    sid = stream if stream is not None else _stream(torch.device("cuda", index))
    key = (index, int(sid or 0))
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.zeros(max(int(nbytes), 256), dtype=torch.uint8, device=dev)
        _WORKSPACES[key] = ws
    return ws


_EPI = {None: _lib.MK_EPI_NONE, "add": _lib.MK_EPI_ADD, "swiglu": _lib.MK_EPI_SWIGLU,
        "swiglu_pairs": _lib.MK_EPI_SWIGLU_PAIRS}


def _epilogue(epilogue, aux, shape, name):
    code = _EPI[epilogue]
    if code == _lib.MK_EPI_SWIGLU_PAIRS:
        if aux is not None:
            raise ValueError(f"{name}: the paired SwiGLU takes no aux")
    elif code != _lib.MK_EPI_NONE:
        _require(aux, _BF16, "aux")
        if tuple(aux.shape) != tuple(shape):
            raise ValueError(f"{name}: aux must have the output's shape {tuple(shape)}")
    return code


def _out_cols(N, epilogue, name):
    """Output columns: N, or N/2 for the paired SwiGLU (gate and up 16-column
    blocks interleaved in the N weight columns)."""
    if epilogue != "swiglu_pairs":
        return N
    if N % 32:
        raise ValueError(f"{name}: the paired SwiGLU needs N % 32 == 0")
    return N // 2


def int4_swiglu_pairs_supported(M, K, N):
    """Whether int4_g64_matmul(..., epilogue="swiglu_pairs") runs at this
    shape (N = the interleaved width): only the many-row route has it."""
    return bool(lib().mk_qmatmul_epilogue_supported(_lib.MK_QFMT_INT4_G64, M, K, N, _lib.MK_EPI_SWIGLU_PAIRS))


def interleave_gate_up(gate, up, block=16):
    """[..., F] gate and up weights (any per-column layout: packed int4,
    scales, zero points, bf16) -> [..., 2F] with 16-column blocks alternating
    gate, up: the B operand of the "swiglu_pairs" epilogue."""
    if gate.shape != up.shape or gate.shape[-1] % block:
        raise ValueError("interleave_gate_up: gate and up need the same shape, last dim % 16 == 0")
    lead, F = gate.shape[:-1], gate.shape[-1]
    g = gate.reshape(*lead, F // block, 1, block)
    u = up.reshape(*lead, F // block, 1, block)
    return torch.cat([g, u], dim=-2).reshape(*lead, 2 * F).contiguous()


def int4_g64_matmul(x, w_packed, scale, zero, out=None, epilogue=None, aux=None):
    """y = x @ ((w - zero) * scale): x bf16 [M,K], w uint8 [K/2,N], scale bf16
    [K/64,N], zero uint8 [K/64,N] -> bf16 [M,N].  epilogue "add" gives
    y = r(r(xW) + aux), "swiglu" y = r(r(aux * r(logistic(aux))) * r(xW)),
    "swiglu_pairs" (W from interleave_gate_up, no aux) y [M, N/2] =
    silu(gate) * up as "swiglu" computes it."""
    _require(x, _BF16, "x")
    _require(w_packed, (torch.uint8,), "w_packed")
    _require(scale, _BF16, "scale")
    _require(zero, (torch.uint8,), "zero")
    M, K = x.shape
    N = w_packed.shape[1]
    if w_packed.shape[0] * 2 != K or scale.shape != (K // 64, N) or zero.shape != (K // 64, N):
        raise ValueError("int4_g64_matmul: inconsistent shapes")
    NO = _out_cols(N, epilogue, "int4_g64_matmul")
    y = out if out is not None else torch.empty((M, NO), dtype=torch.bfloat16, device=x.device)
    epi = _epilogue(epilogue, aux, (M, N), "int4_g64_matmul")
    nb = lib().mk_qmatmul_workspace_bytes(_lib.MK_QFMT_INT4_G64, M, K, N)
    ws = workspace(nb, x.device) if nb > 0 else None
    if epi == _lib.MK_EPI_NONE:
        check(lib().mk_int4g64_matmul_bf16(_ptr(x), _ptr(w_packed), _ptr(scale), _ptr(zero), _ptr(y),
                                           M, K, N, _ptr(ws), max(nb, 0), _stream(x.device)))
    else:
        check(lib().mk_int4g64_matmul_epilogue_bf16(_ptr(x), _ptr(w_packed), _ptr(scale), _ptr(zero), _ptr(y),
                                                    _ptr(aux), epi, M, K, N, _ptr(ws), max(nb, 0),
                                                    _stream(x.device)))
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


def swiglu_pair_matmul(x, wg, wu, out=None):
    """y = silu(x @ Wg) * (x @ Wu) -> bf16 [M, N] from two separate quantized
    weights: wg, wu = (w_packed, scale, zero) as for int4_g64_matmul, or
    (w, scale) as for int8_pc_matmul.  Bit-identical to the two products
    followed by the SwiGLU elementwise program; many-row shapes only (the C-ABI
    returns MK_EUNSUPPORTED otherwise)."""
    int4 = len(wg) == 3
    if len(wu) != len(wg) or len(wg) not in (2, 3):
        raise ValueError("swiglu_pair_matmul: wg and wu must both be int4 (3 arrays) or int8 (2 arrays)")
    _require(x, _BF16, "x")
    M, K = x.shape
    N = wg[0].shape[1]
    for w in (wg, wu):
        if int4:
            _require(w[0], (torch.uint8,), "w_packed")
            _require(w[1], _BF16, "scale")
            _require(w[2], (torch.uint8,), "zero")
            if w[0].shape != (K // 2, N) or w[1].shape != (K // 64, N) or w[2].shape != (K // 64, N):
                raise ValueError("swiglu_pair_matmul: inconsistent int4 shapes")
        else:
            _require(w[0], (torch.int8,), "w")
            _require(w[1], (torch.float32,), "scale")
            if w[0].shape != (K, N) or w[1].shape != (N,):
                raise ValueError("swiglu_pair_matmul: inconsistent int8 shapes")
    fmt = _lib.MK_QFMT_INT4_G64 if int4 else _lib.MK_QFMT_INT8_PC
    y = out if out is not None else torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    nb = lib().mk_qmatmul_swiglu_pair_workspace_bytes(fmt, M, K, N)
    ws = workspace(nb, x.device) if nb > 0 else None
    if int4:
        check(lib().mk_int4g64_matmul_swiglu_pair_bf16(_ptr(x), *(_ptr(a) for a in wg), *(_ptr(a) for a in wu),
                                                       _ptr(y), M, K, N, _ptr(ws), max(nb, 0), _stream(x.device)))
    else:
        check(lib().mk_int8pc_matmul_swiglu_pair_bf16(_ptr(x), *(_ptr(a) for a in wg), *(_ptr(a) for a in wu),
                                                      _ptr(y), M, K, N, _ptr(ws), max(nb, 0), _stream(x.device)))
    return y


def _bmk(a, b):
    if a.dim() == 2:
        a2, b2 = a.unsqueeze(0), b.unsqueeze(0)
    else:
        a2, b2 = a, b
    if a2.dim() != 3 or b2.dim() != 3 or a2.shape[0] != b2.shape[0] or a2.shape[2] != b2.shape[1]:
        raise ValueError(f"gemm: incompatible shapes {tuple(a.shape)} x {tuple(b.shape)}")
    return a2.shape[0], a2.shape[1], b2.shape[2], a2.shape[2]


def gemm_bf16(a, b, out_f32=False, out=None, epilogue=None, aux=None):
    """[batch,] M x K @ K x N in bf16 with f32 accumulation -> bf16 (or f32).
    epilogue "add" / "swiglu" with aux (bf16, the output's shape) or
    "swiglu_pairs" (output N/2 columns) as in int4_g64_matmul (bf16 output
    only)."""
    _require(a, _BF16, "a")
    _require(b, _BF16, "b")
    batch, M, N, K = _bmk(a, b)
    shape = (M, N) if a.dim() == 2 else (batch, M, N)
    NO = _out_cols(N, epilogue, "gemm_bf16")
    oshape = shape[:-1] + (NO,)
    c = out if out is not None else torch.empty(
        oshape, dtype=torch.float32 if out_f32 else torch.bfloat16, device=a.device)
    epi = _epilogue(epilogue, aux, shape, "gemm_bf16")
    if epi == _lib.MK_EPI_NONE:
        check(lib().mk_gemm_bf16(_ptr(a), _ptr(b), _ptr(c), batch, M, N, K, 1 if out_f32 else 0,
                                 _stream(a.device)))
    else:
        if out_f32:
            raise ValueError("gemm_bf16: epilogues write bf16")
        check(lib().mk_gemm_bf16_epilogue(_ptr(a), _ptr(b), _ptr(c), _ptr(aux), epi, batch, M, N, K,
                                          _stream(a.device)))
    return c


def _gemm_route_args(a, b, out_f32, out, epilogue, aux, name):
    _require(a, _BF16, "a")
    _require(b, _BF16, "b")
    batch, M, N, K = _bmk(a, b)
    shape = (M, N) if a.dim() == 2 else (batch, M, N)
    NO = _out_cols(N, epilogue, name)
    c = out if out is not None else torch.empty(
        shape[:-1] + (NO,), dtype=torch.float32 if out_f32 else torch.bfloat16, device=a.device)
    epi = _epilogue(epilogue, aux, shape, name)
    if epi != _lib.MK_EPI_NONE and out_f32:
        raise ValueError(f"{name}: epilogues write bf16")
    return batch, M, N, K, c, epi


def gemm_bf16_route(a, b, route, out_f32=False, out=None, epilogue=None, aux=None):
    """gemm_bf16 on a given route ("ring", "pipe", "persist", "short",
    "reg256", "generic256", "generic128" or "default"): every route gives
    the same bits; a route that does not take the shape raises."""
    batch, M, N, K, c, epi = _gemm_route_args(a, b, out_f32, out, epilogue, aux, "gemm_bf16_route")
    check(lib().mk_gemm_bf16_route(_ptr(a), _ptr(b), _ptr(c), _ptr(aux) if aux is not None else None, epi, batch,
                                   M, N, K, 1 if out_f32 else 0, _lib.GEMM_ROUTES[route], _stream(a.device)))
    return c


def gemm_route_fits(route, M, N, K, epilogue=None, out_f32=False):
    epi = {None: _lib.MK_EPI_NONE, "add": _lib.MK_EPI_ADD, "swiglu": _lib.MK_EPI_SWIGLU,
           "swiglu_pairs": _lib.MK_EPI_SWIGLU_PAIRS}[epilogue]
    return bool(lib().mk_gemm_bf16_route_fits(_lib.GEMM_ROUTES[route], M, N, K, epi, 1 if out_f32 else 0))


def gemm_bf16_autotune(a, b, out_f32=False, out=None, epilogue=None, aux=None):
    """Times every route that takes the product and records the fastest in
    the library's route table for this device and shape.  Returns (route
    name, median us, the product)."""
    batch, M, N, K, c, epi = _gemm_route_args(a, b, out_f32, out, epilogue, aux, "gemm_bf16_autotune")
    route, us = ctypes.c_int(0), ctypes.c_float(0.0)
    check(lib().mk_gemm_bf16_autotune(_ptr(a), _ptr(b), _ptr(c), _ptr(aux) if aux is not None else None, epi,
                                      batch, M, N, K, 1 if out_f32 else 0, _stream(a.device), ctypes.byref(route),
                                      ctypes.byref(us)))
    names = {v: k for k, v in _lib.GEMM_ROUTES.items()}
    return names[route.value], us.value, c


def gemm_tuned_route(batch, M, N, K, epilogue=None, out_f32=False):
    """The route table's entry for the product on the current device
    ("default" when none)."""
    epi = {None: _lib.MK_EPI_NONE, "add": _lib.MK_EPI_ADD, "swiglu": _lib.MK_EPI_SWIGLU,
           "swiglu_pairs": _lib.MK_EPI_SWIGLU_PAIRS}[epilogue]
    names = {v: k for k, v in _lib.GEMM_ROUTES.items()}
    return names[lib().mk_gemm_tuned_route(batch, M, N, K, epi, 1 if out_f32 else 0)]


def gemm_autotune_save(path):
    """Writes the route table to `path`; returns the number of entries."""
    n = lib().mk_gemm_autotune_save(str(path).encode())
    if n < 0:
        raise RuntimeError(lib().mk_last_error().decode())
    return n


def gemm_autotune_load(path):
    """Merges a saved route table; returns the number of entries read."""
    n = lib().mk_gemm_autotune_load(str(path).encode())
    if n < 0:
        raise RuntimeError(lib().mk_last_error().decode())
    return n


def gemm_autotune_clear():
    lib().mk_gemm_autotune_clear()


def gemm_bf16_nt(a, bt, out=None, epilogue=None, aux=None):
    """[batch,] M x K @ (N x K)^T in bf16 with f32 accumulation -> bf16: the
    rhs given with K contiguous (x @ W.T, q @ k^T).  The same bits as
    gemm_bf16(a, bt.transpose(-1, -2).contiguous(), ...).  Needs M and N
    multiples of 256 and K of 32."""
    _require(a, _BF16, "a")
    _require(bt, _BF16, "bt")
    if a.dim() != bt.dim() or a.dim() not in (2, 3) or a.shape[-1] != bt.shape[-1] or \
            (a.dim() == 3 and a.shape[0] != bt.shape[0]):
        raise ValueError(f"gemm_bf16_nt: incompatible shapes {tuple(a.shape)} x {tuple(bt.shape)}^T")
    batch = a.shape[0] if a.dim() == 3 else 1
    M, K, N = a.shape[-2], a.shape[-1], bt.shape[-2]
    shape = (M, N) if a.dim() == 2 else (batch, M, N)
    NO = _out_cols(N, epilogue, "gemm_bf16_nt")
    c = out if out is not None else torch.empty(shape[:-1] + (NO,), dtype=torch.bfloat16, device=a.device)
    epi = _epilogue(epilogue, aux, shape, "gemm_bf16_nt")
    check(lib().mk_gemm_bf16_nt(_ptr(a), _ptr(bt), _ptr(c), _ptr(aux) if aux is not None else None, epi, batch,
                                M, N, K, _stream(a.device)))
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


def _dt(t):
    if t.dtype == torch.float32:
        return _lib.MK_DT_F32
    if t.dtype in _BF16:
        return _lib.MK_DT_BF16
    raise ValueError(f"unsupported dtype {t.dtype}")


def _rows_cols(x):
    cols = x.shape[-1]
    return x.numel() // cols, cols


def softmax(x, out=None):
    """Softmax over the last axis (f32 or bf16)."""
    _require(x, (torch.float32,) + _BF16, "x")
    rows, cols = _rows_cols(x)
    y = out if out is not None else torch.empty_like(x)
    check(lib().mk_softmax_lastdim(_dt(x), _ptr(x), _ptr(y), rows, cols, _stream(x.device)))
    return y


def rmsnorm(x, g, eps=1e-6, out=None):
    """x * rsqrt(mean(x^2, -1) + eps) * g."""
    _require(x, (torch.float32,) + _BF16, "x")
    _require(g, (x.dtype,), "g")
    rows, cols = _rows_cols(x)
    if g.numel() != cols:
        raise ValueError("rmsnorm: g must have cols elements")
    y = out if out is not None else torch.empty_like(x)
    check(lib().mk_rmsnorm_lastdim(_dt(x), _ptr(x), _ptr(g), _ptr(y), rows, cols, eps, _stream(x.device)))
    return y


def argmax(x, out=None):
    """Index (int32) of the first NaN, else of the first maximum, per row."""
    _require(x, (torch.float32,) + _BF16, "x")
    rows, cols = _rows_cols(x)
    y = out if out is not None else torch.empty(x.shape[:-1], dtype=torch.int32, device=x.device)
    check(lib().mk_argmax_lastdim(_dt(x), _ptr(x), _ptr(y), rows, cols, _stream(x.device)))
    return y


def reduce_lastdim(x, op="sum", out=None):
    """Row sum (f32 accumulation) or NaN-propagating row max, in x's dtype."""
    _require(x, (torch.float32,) + _BF16, "x")
    rows, cols = _rows_cols(x)
    y = out if out is not None else torch.empty(x.shape[:-1], dtype=x.dtype, device=x.device)
    code = {"sum": _lib.MK_REDUCE_SUM, "max": _lib.MK_REDUCE_MAX, "min": _lib.MK_REDUCE_MIN}[op]
    check(lib().mk_reduce_lastdim(_dt(x), code, _ptr(x), _ptr(y), rows, cols, _stream(x.device)))
    return y


def elementwise(program, inputs, out_slot, out=None, dtype=None):
    """Evaluate an elementwise register program (list of (op, dst, a, b, c,
    imm) tuples, op a name from mi355x._lib.EW_OPS or an op code, possibly
    or'ed with MK_EW_KEEP_F32) over inputs of the output's shape, 1-element
    scalars or periodic inputs (a divisor of its size).  dtype
    (torch.float32 / torch.bfloat16) is the program's and the output's type,
    by default the first non-scalar input's; inputs of the other type are
    loaded with MK_EW_IN_F32 / MK_EW_IN_BF16 in their LOAD's b."""
    import ctypes as _ct

    big = [t for t in inputs if t.numel() != 1]
    ref = big[0] if big else inputs[0]
    for t in inputs:
        _require(t, (torch.float32,) + _BF16, "input")
    n = ref.numel() if out is None else out.numel()
    out_dtype = dtype if dtype is not None else ref.dtype
    dt = _lib.MK_DT_F32 if out_dtype == torch.float32 else _lib.MK_DT_BF16
    arr = (_lib.EwInstr * len(program))()
    for i, (op, dst, a, b, c, imm) in enumerate(program):
        arr[i] = _lib.EwInstr(_lib.EW[op] if isinstance(op, str) else op, dst, a, b, c, imm)
    ptrs = (_ct.c_void_p * max(1, len(inputs)))(*[t.data_ptr() for t in inputs])
    numel = (_ct.c_int64 * max(1, len(inputs)))(*[t.numel() for t in inputs])
    y = out if out is not None else torch.empty(ref.shape, dtype=out_dtype, device=ref.device)
    check(lib().mk_elementwise_prepare(dt, arr, len(program), len(inputs), out_slot))
    check(lib().mk_elementwise(dt, arr, len(program), ptrs, numel, len(inputs), out_slot, _ptr(y), n,
                               _stream(ref.device)))
    return y


def rope_qkv_split(qkv, cos_table, sin_table, B, S, H, D=128, q=None, k=None, v=None, k_transposed=True):
    """qkv bf16 [B*S, 3*H*D] (blocks q | k | v) -> q [B*H, S, D], k, v
    [B*H, S, D], with rotary embedding (rotate-half) applied to q and k from
    the f32 tables cos_table / sin_table [S, D/2].  With k_transposed, k is
    written as kT [B*H, D, S] (the B operand of q @ k^T)."""
    _require(qkv, _BF16, "qkv")
    _require(cos_table, (torch.float32,), "cos_table")
    _require(sin_table, (torch.float32,), "sin_table")
    if qkv.shape != (B * S, 3 * H * D) or cos_table.shape != (S, D // 2) or sin_table.shape != (S, D // 2):
        raise ValueError("rope_qkv_split: inconsistent shapes")
    dev = qkv.device
    q = q if q is not None else torch.empty((B * H, S, D), dtype=torch.bfloat16, device=dev)
    kshape = (B * H, D, S) if k_transposed else (B * H, S, D)
    k = k if k is not None else torch.empty(kshape, dtype=torch.bfloat16, device=dev)
    v = v if v is not None else torch.empty((B * H, S, D), dtype=torch.bfloat16, device=dev)
    check(lib().mk_rope_qkv_split_bf16(_ptr(qkv), _ptr(cos_table), _ptr(sin_table), _ptr(q), _ptr(k), _ptr(v),
                                       B, S, H, D, 0 if k_transposed else 1, _stream(dev)))
    return q, k, v


def attention_causal(q, k, v, B, H, scale, out=None):
    """Causal attention of q, k, v bf16 [B*H, S, D] in one pass -> out bf16
    [B*S, H*D] (heads merged)."""
    for t, n in ((q, "q"), (k, "k"), (v, "v")):
        _require(t, _BF16, n)
    if q.dim() != 3 or q.shape[0] != B * H or k.shape != q.shape or v.shape != q.shape:
        raise ValueError("attention_causal: q, k, v must all be [B*H, S, D]")
    S, D = q.shape[1], q.shape[2]
    y = out if out is not None else torch.empty((B * S, H * D), dtype=torch.bfloat16, device=q.device)
    check(lib().mk_attention_causal_bf16(_ptr(q), _ptr(k), _ptr(v), _ptr(y), B, H, S, D, float(scale),
                                         _stream(q.device)))
    return y


def softmax_causal(scores, scale, out=None):
    """Causal softmax of bf16 scores [batches, S, S]: row i keeps columns
    j <= i, p = exp(scale*s - m) / sum in f32, zeros above the diagonal."""
    _require(scores, _BF16, "scores")
    if scores.dim() != 3 or scores.shape[1] != scores.shape[2]:
        raise ValueError("softmax_causal: scores must be [batches, S, S]")
    p = out if out is not None else torch.empty_like(scores)
    check(lib().mk_softmax_causal_bf16(_ptr(scores), _ptr(p), scores.shape[0], scores.shape[1], float(scale),
                                       _stream(scores.device)))
    return p


def merge_heads(o, B, H, out=None):
    """Attention output o bf16 [B*H, S, D] -> [B*S, H*D]."""
    _require(o, _BF16, "o")
    if o.dim() != 3 or o.shape[0] != B * H:
        raise ValueError("merge_heads: o must be [B*H, S, D]")
    S, D = o.shape[1], o.shape[2]
    y = out if out is not None else torch.empty((B * S, H * D), dtype=torch.bfloat16, device=o.device)
    check(lib().mk_merge_heads_bf16(_ptr(o), _ptr(y), B, H, S, D, _stream(o.device)))
    return y
