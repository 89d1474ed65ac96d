"""GPU tests of the layout kernels (mk_strided_copy, mk_iota) and of the
elementwise engine's periodic and mixed-type inputs, through the C-ABI and
through compiled programs.

Layout ops move values, so they are checked bit for bit against torch's /
numpy's own transpose, slice, broadcast and concatenate (the reference's
MPSGraph handlers, ops/shape_ops.mm:137-153, :304-333, :831-865,
:1208-1265; iota ops/tensor_creation_ops.mm:126-148).  Mixed-type
elementwise programs are checked against numpy float32 arithmetic rounded
to bf16 where the program's type is bf16."""

import ctypes

import numpy as np
import pytest

from _gpu import need_gpu, torch
from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits

pytestmark = pytest.mark.gpu


def _mods():
    need_gpu()
    from mi355x import _lib, ops
    return _lib, ops


def _arr(v):
    return (ctypes.c_int64 * max(1, len(v)))(*v)


def _copy(src, dst, shape, ss, so, ds, do):
    _lib, ops = _mods()
    print(f"[layout] copy {src.dtype} shape={list(shape)} ss={list(ss)} so={so} ds={list(ds)} do={do}", flush=True)
    return _lib.lib().mk_strided_copy(src.data_ptr(), dst.data_ptr(), src.element_size(), len(shape), _arr(shape),
                                      _arr(ss), so, _arr(ds), do, ops._stream(src.device))


def _contig(shape):
    st, acc = [], 1
    for d in reversed(shape):
        st.append(acc)
        acc *= d
    return list(reversed(st))


_DTYPES = [torch.uint8, torch.int16, torch.float32, torch.float64]


def _rand(shape, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    if dtype.is_floating_point:
        return torch.randn(shape, generator=g, dtype=dtype)
    return torch.randint(0, 120, shape, generator=g, dtype=dtype)


@pytest.mark.parametrize("dtype", _DTYPES)
@pytest.mark.parametrize("perm", [(0, 2, 1, 3), (3, 2, 1, 0), (1, 0, 3, 2), (0, 1, 3, 2)])
def test_transpose(dtype, perm):
    _lib, _ = _mods()
    x = _rand((3, 5, 8, 16), dtype, hash(perm) % 1000).cuda()
    want = x.permute(perm).contiguous()
    y = torch.empty_like(want)
    shape = list(want.shape)
    _lib.check(_copy(x, y, shape, [x.stride(p) for p in perm], 0, _contig(shape), 0))
    torch.cuda.synchronize()
    assert torch.equal(y, want)


@pytest.mark.parametrize("dtype", _DTYPES)
def test_strided_slice_and_broadcast(dtype):
    _lib, _ = _mods()
    x = _rand((20, 30), dtype, 1).cuda()
    want = x[2:17:3, 5:29:2].contiguous()
    y = torch.empty_like(want)
    _lib.check(_copy(x, y, list(want.shape), [30 * 3, 2], 2 * 30 + 5, _contig(list(want.shape)), 0))
    b = _rand((5, 1, 7), dtype, 2).cuda()
    wb = b.expand(5, 4, 7).contiguous()
    yb = torch.empty_like(wb)
    _lib.check(_copy(b, yb, [5, 4, 7], [7, 0, 1], 0, _contig([5, 4, 7]), 0))
    torch.cuda.synchronize()
    assert torch.equal(y, want) and torch.equal(yb, wb)


@pytest.mark.parametrize("dtype", _DTYPES)
def test_concatenate_by_offsets(dtype):
    _lib, _ = _mods()
    a, b = _rand((4, 3, 16), dtype, 3).cuda(), _rand((4, 5, 16), dtype, 4).cuda()
    want = torch.cat([a, b], dim=1)
    y = torch.empty_like(want)
    ds = _contig(list(want.shape))
    _lib.check(_copy(a, y, list(a.shape), _contig(list(a.shape)), 0, ds, 0))
    _lib.check(_copy(b, y, list(b.shape), _contig(list(b.shape)), 0, ds, 3 * 16))
    torch.cuda.synchronize()
    assert torch.equal(y, want)


def test_rank_limits_and_empty_copies():
    _lib, _ = _mods()
    x = _rand((2,) * 8, torch.float32, 5).cuda()
    perm = (7, 6, 5, 4, 3, 2, 1, 0)
    want = x.permute(perm).contiguous()
    y = torch.empty_like(want)
    _lib.check(_copy(x, y, [2] * 8, [x.stride(p) for p in perm], 0, _contig([2] * 8), 0))
    s = torch.tensor([3.5], device="cuda")
    t = torch.zeros(1, device="cuda")
    _lib.check(_copy(s, t, [], [], 0, [], 0))  # rank 0: one element
    _lib.check(_copy(s, t, [0, 4], [4, 1], 0, [4, 1], 0))  # nothing to move
    torch.cuda.synchronize()
    assert torch.equal(y, want) and float(t) == 3.5
    bad = [
        ([2] * 9, [1] * 9, [1] * 9),   # rank 9
        ([4], [-1], [1]),              # negative stride
        ([-1], [1], [1]),              # negative dimension
    ]
    for shape, ss, ds in bad:
        assert _copy(x, y, shape, ss, 0, ds, 0) == _lib.MK_EINVAL
    assert _lib.lib().mk_strided_copy(x.data_ptr(), y.data_ptr(), 3, 1, _arr([4]), _arr([1]), 0, _arr([1]), 0,
                                      None) == _lib.MK_EINVAL


def test_large_head_transpose():
    """[B, S, H, D] -> [B, H, S, D] at the decoder's size (bf16 bits), the
    copy the compiled layer runs per projection."""
    _lib, _ = _mods()
    B, S, H, D = 4, 2048, 16, 128
    x = torch.randint(-30000, 30000, (B, S, H, D), dtype=torch.int16, device="cuda")
    y = torch.empty((B, H, S, D), dtype=torch.int16, device="cuda")
    _lib.check(_copy(x, y, [B, H, S, D], [x.stride(0), x.stride(2), x.stride(1), 1], 0, _contig([B, H, S, D]), 0))
    torch.cuda.synchronize()
    assert torch.equal(y, x.permute(0, 2, 1, 3).contiguous())


_IOTA = [("S8", np.int8), ("S16", np.int16), ("S32", np.int32), ("S64", np.int64), ("U8", np.uint8),
         ("U16", np.uint16), ("U32", np.uint32), ("U64", np.uint64), ("F16", np.float16), ("F32", np.float32),
         ("F64", np.float64), ("BF16", None)]


@pytest.mark.parametrize("name,npdt", _IOTA)
@pytest.mark.parametrize("dim", [0, 1, 2])
def test_iota(name, npdt, dim):
    _lib, ops = _mods()
    code = {"S8": 2, "S16": 3, "S32": 4, "S64": 5, "U8": 6, "U16": 7, "U32": 8, "U64": 9, "F16": 10, "F32": 11,
            "F64": 12, "BF16": 13}[name]
    shape = [3, 300, 5] if name not in ("S8", "U8") else [3, 100, 5]
    esz = 2 if npdt is None else np.dtype(npdt).itemsize
    n = int(np.prod(shape))
    buf = torch.empty(n * esz, dtype=torch.uint8, device="cuda")
    print(f"[layout] iota {name} shape={shape} dim={dim}", flush=True)
    _lib.check(_lib.lib().mk_iota(buf.data_ptr(), code, 3, _arr(shape), dim, ops._stream(buf.device)))
    torch.cuda.synchronize()
    raw = buf.cpu().numpy()
    idx = np.indices(shape)[dim]
    if npdt is None:
        got = raw.view(np.uint16).reshape(shape)
        assert np.array_equal(got, f32_to_bf16_bits(idx.astype(np.float32)))
    else:
        assert np.array_equal(raw.view(npdt).reshape(shape), idx.astype(npdt))


# ---------------------------------------------------------------- elementwise
def test_periodic_input():
    """A [T, T] operand read periodically under [B, H, T, T] elements."""
    _lib, ops = _mods()
    rng = np.random.default_rng(0)
    big = rng.standard_normal((2, 3, 16, 16)).astype(np.float32)
    per = rng.standard_normal((16, 16)).astype(np.float32)
    prog = [("LOAD", 0, 0, 0, 0, 0.0), ("LOAD", 1, 1, 0, 0, 0.0), ("MUL", 2, 0, 1, 0, 0.0)]
    y = ops.elementwise(prog, [torch.from_numpy(big).cuda(), torch.from_numpy(per).cuda()], out_slot=2)
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy(), big * per[None, None])
    # a periodic input that is not a multiple of the vector width: scalar path
    odd = rng.standard_normal(7).astype(np.float32)
    z = ops.elementwise(prog, [torch.from_numpy(big[..., :14].copy()).cuda(), torch.from_numpy(odd[:7]).cuda()],
                        out_slot=2)
    ref = (big[..., :14].reshape(-1) * np.tile(odd, big[..., :14].size // 7)).reshape(big[..., :14].shape)
    assert np.array_equal(z.cpu().numpy(), ref)


def test_mixed_input_types():
    """A bf16 input in an f32 program and an f32 input in a bf16 program, the
    latter with f32 arithmetic marked MK_EW_KEEP_F32 and one rounding at the
    end."""
    _lib, ops = _mods()
    rng = np.random.default_rng(1)
    n = 4096 + 8
    a32 = rng.standard_normal(n).astype(np.float32)
    b16 = f32_to_bf16_bits(rng.standard_normal(n).astype(np.float32))
    b32 = bf16_bits_to_f32(b16)
    da = torch.from_numpy(a32).cuda()
    db = torch.from_numpy(b16.view(np.int16)).cuda()
    # f32 program: a * b  (b read as bf16)
    prog = [("LOAD", 0, 0, 0, 0, 0.0), ("LOAD", 1, 1, _lib.MK_EW_IN_BF16, 0, 0.0), ("MUL", 2, 0, 1, 0, 0.0)]
    y = ops.elementwise(prog, [da, db], out_slot=2, dtype=torch.float32)
    # bf16 program: round_bf16(exp(a) * b + a) with the product, exp and sum in f32
    keep = _lib.MK_EW_KEEP_F32
    prog2 = [("LOAD", 0, 0, _lib.MK_EW_IN_F32, 0, 0.0), ("LOAD", 1, 1, 0, 0, 0.0),
             (_lib.EW["EXP"] | keep, 2, 0, 0, 0, 0.0), (_lib.EW["MUL"] | keep, 3, 2, 1, 0, 0.0),
             (_lib.EW["ADD"] | keep, 4, 3, 0, 0, 0.0), ("ROUND_BF16", 5, 4, 0, 0, 0.0)]
    z = ops.elementwise(prog2, [da, db], out_slot=5, dtype=torch.bfloat16)
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy(), a32 * b32)
    got = bf16_bits_to_f32(z.view(torch.int16).cpu().numpy().view(np.uint16)).astype(np.float64)
    ref = np.exp(a32.astype(np.float64)) * b32 + a32
    # one bf16 rounding of an f32 result within a few f32 ulps of ref
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 2.0 ** -8 + 1e-30)
    # the same program without the flag rounds exp and the product too: it
    # must differ somewhere, or the flag is not reaching the kernel
    prog3 = [(op & ~keep if isinstance(op, int) else op, *rest) for op, *rest in prog2]
    w = ops.elementwise(prog3, [da, db], out_slot=5, dtype=torch.bfloat16)
    torch.cuda.synchronize()
    assert not torch.equal(w, z)
    with pytest.raises(_lib.MKError):
        ops.elementwise([("LOAD", 0, 0, 7, 0, 0.0)], [da], out_slot=0)  # bad input type
    with pytest.raises(_lib.MKError):
        ops.elementwise([("LOAD", 0, 0, 0, 0, 0.0), (_lib.EW["CMP_LT"] | keep, 1, 0, 0, 0, 0.0)], [da], out_slot=1)
