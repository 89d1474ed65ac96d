"""The general dot_general path (mk_dot_general through the runtime): the
reference's integer-dot cases (tests/test_int_dot.py:21-57 under
/root/reference: mm, vec, batched, multi_batch, self = a @ a.T,
preferred_element_type=int32, for int8 / uint8 / int16 / int32 / uint32) must
match exactly, and K == 1 must keep XLA's signed zero
(src/pjrt_plugin/ops/binary_ops.mm:904-1004).

Integer expectations are closed forms: numpy int64 products and sums, then
the cast to the result type (two's-complement wraparound, which is exact
whatever width the sum is formed in)."""

import numpy as np
import pytest

from mi355x import programs as P
from mi355x import runtime as rt
from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits

from _gpu import assert_rel_close

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def client():
    try:
        c = rt.Client()
    except rt.PluginError as e:
        pytest.fail(f"GPU test selected but the runtime has no device: {e}")
    yield c
    c.close()


def run(client, text, *arrays):
    exe = client.compile(text)
    assert "dot_general" in exe.plan or exe.num_steps >= 1
    bufs = [client.buffer(*a) if isinstance(a, tuple) else client.buffer(a) for a in arrays]
    outs, done = exe.execute(bufs)
    done.wait()
    res = [o.to_numpy() for o in outs]
    for b in bufs + outs:
        b.close()
    exe.close()
    return res[0]


def _arr(rng, shape, dtype):
    big = dtype in ("int32", "uint32")
    lo, hi = (-(1 << 20), 1 << 20) if big else (-300, 300)
    return rng.integers(lo, hi, size=shape, dtype=np.int64).astype(dtype)


CASES = ["mm", "vec", "batched", "multi_batch", "self", "preferred_i32"]


@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("dtype", ["int8", "uint8", "int16", "int32", "uint32"])
def test_integer_dot_is_exact(client, dtype, case):
    rng = np.random.default_rng(0)
    print(f"[dot] {dtype} {case}", flush=True)
    out_dt = dtype
    if case == "mm":
        a, b = _arr(rng, (5, 7), dtype), _arr(rng, (7, 3), dtype)
        text, args = P.dot_general(a.shape, b.shape, dtype), (a, b)
    elif case == "vec":
        a, b = _arr(rng, (7,), dtype), _arr(rng, (7, 3), dtype)
        text, args = P.dot_general(a.shape, b.shape, dtype), (a, b)
    elif case == "batched":
        a, b = _arr(rng, (2, 5, 7), dtype), _arr(rng, (2, 7, 3), dtype)
        text, args = P.dot_general(a.shape, b.shape, dtype, batch=1), (a, b)
    elif case == "multi_batch":
        a, b = _arr(rng, (2, 3, 4, 5), dtype), _arr(rng, (2, 3, 5, 6), dtype)
        text, args = P.dot_general(a.shape, b.shape, dtype, batch=2), (a, b)
    elif case == "self":
        a = _arr(rng, (5, 7), dtype)
        b = a.T
        text, args = P.dot_general(a.shape, None, dtype, self_transpose=True), (a,)
    else:
        a, b = _arr(rng, (5, 7), dtype), _arr(rng, (7, 3), dtype)
        out_dt = "int32"
        text, args = P.dot_general(a.shape, b.shape, dtype, out_dt="int32"), (a, b)
    ref = np.matmul(a.astype(np.int64), b.astype(np.int64)).astype(out_dt)
    y = run(client, text, *args)
    assert y.dtype == ref.dtype and y.shape == ref.shape
    assert np.array_equal(y, ref)


def test_k1_keeps_signed_zero(client):
    """K == 1 is a plain product: (-1) * 0 = -0 survives (XLA:CPU); with
    K >= 2 the sum starts from +0, so all--0 products give +0."""
    a = np.array([[-1.0], [2.0], [0.0], [-0.0]], np.float32)
    b = np.array([[0.0, -3.0, -0.0]], np.float32)
    y = run(client, P.dot_general(a.shape, b.shape, "float32"), a, b)
    ref = a * b
    assert np.array_equal(y, ref)
    assert np.array_equal(np.signbit(y), np.signbit(ref)), (y, ref)
    assert np.signbit(y[0, 0]) and not np.signbit(y[1, 0])
    ab = f32_to_bf16_bits(a)
    bb = f32_to_bf16_bits(b)
    yb = run(client, P.dot_general(a.shape, b.shape, "bfloat16"), (ab, rt.BF16), (bb, rt.BF16))
    assert np.array_equal(np.signbit(bf16_bits_to_f32(yb)), np.signbit(ref))
    a2 = np.array([[-1.0, -1.0]], np.float32)
    b2 = np.array([[0.0], [0.0]], np.float32)
    y2 = run(client, P.dot_general(a2.shape, b2.shape, "float32"), a2, b2)
    assert y2[0, 0] == 0 and not np.signbit(y2[0, 0])


@pytest.mark.parametrize("shape_a,shape_b,batch,tr", [((33, 7), (7, 5), 0, None), ((6, 10), (3, 10), 0, [1, 0]),
                                                      ((2, 5, 12), (2, 3, 12), 1, [0, 2, 1]), ((9,), (9, 4), 0, None)])
@pytest.mark.parametrize("dt", ["float32", "bfloat16", "float16"])
def test_float_general_dot(client, shape_a, shape_b, batch, tr, dt):
    """Shapes the tiled GEMMs do not take (K or N not a multiple of 8,
    transposed operands, vectors) against float64, at the workload's
    tolerances (f32 rel 1e-5; bf16 / f16 one output rounding)."""
    rng = np.random.default_rng(len(shape_a) + shape_a[-1] + (tr is not None))
    a = rng.standard_normal(shape_a).astype(np.float32)
    b = rng.standard_normal(shape_b).astype(np.float32)
    bt = b if tr is None else np.transpose(b, tr)
    text = P.dot_general(shape_a, shape_b, dt, batch=batch, transpose_b=tr)
    if dt == "bfloat16":
        a64, b64 = bf16_bits_to_f32(f32_to_bf16_bits(a)), bf16_bits_to_f32(f32_to_bf16_bits(bt))
        y = bf16_bits_to_f32(run(client, text, (f32_to_bf16_bits(a), rt.BF16), (f32_to_bf16_bits(b), rt.BF16)))
        tol = 2e-2
    elif dt == "float16":
        a16, b16 = a.astype(np.float16), b.astype(np.float16)
        a64, b64 = a16.astype(np.float64), (b16 if tr is None else np.transpose(b16, tr)).astype(np.float64)
        y = run(client, text, a16, b16).astype(np.float32)
        tol = 2e-3
    else:
        a64, b64 = a, bt
        y = run(client, text, a, b)
        tol = 1e-5
    ref = np.matmul(a64.astype(np.float64), b64.astype(np.float64))
    assert_rel_close(y.reshape(ref.shape), ref, tol, f"dot {dt} {shape_a} {shape_b} tr={tr}")


def test_dot_general_c_abi_rejects_bad_arguments():
    import ctypes
    import torch
    from mi355x import _lib
    L = _lib.lib()
    a = torch.zeros(16, dtype=torch.float32, device="cuda")
    s = (ctypes.c_int64 * 3)(16, 4, 1)
    st = torch.cuda.current_stream().cuda_stream
    assert L.mk_dot_general(11, 13, 11, a.data_ptr(), a.data_ptr(), a.data_ptr(), 1, 2, 2, 2, s, s,
                            st) == _lib.MK_EUNSUPPORTED
    neg = (ctypes.c_int64 * 3)(16, -4, 1)
    assert L.mk_dot_general(11, 11, 11, a.data_ptr(), a.data_ptr(), a.data_ptr(), 1, 2, 2, 2, neg, s,
                            st) == _lib.MK_EINVAL
    assert L.mk_dot_general(4, 4, 11, a.data_ptr(), a.data_ptr(), a.data_ptr(), 1, 2, 2, 2, s, s,
                            st) == _lib.MK_EUNSUPPORTED


# lax.dot_general dimension numbers beyond one contracting dimension with
# leading batch dims (binary_ops.mm:644-1100 handles any): several
# contracting dims (collapsing by strides, or not), none, batch dims in other
# positions, and a shape large enough for the tiled GEMM.
DIMS = [
    ((4, 6, 8), (6, 8, 5), (1, 2), (0, 1), (), ()),
    ((4, 6, 8), (8, 6, 5), (1, 2), (1, 0), (), ()),
    ((6, 4, 8), (8, 5, 6), (0, 2), (2, 0), (), ()),
    ((3, 4), (5, 6), (), (), (), ()),
    ((2, 3, 4), (4, 3, 2), (1,), (1,), (0,), (2,)),
    ((5, 7, 3, 2), (2, 5, 3, 9), (2,), (2,), (3, 0), (0, 1)),
    ((64, 32, 16), (16, 32, 128), (1, 2), (1, 0), (), ()),
]


def _einsum_spec(ra, rb, lc, rc, lb, rb_):
    letters = iter("abcdefghijklmnopqrstuvwxyz")
    sa, sb = [None] * ra, [None] * rb
    for i, j in zip(lb, rb_):
        sa[i] = sb[j] = next(letters)
    for i, j in zip(lc, rc):
        sa[i] = sb[j] = next(letters)
    for i in range(ra):
        sa[i] = sa[i] or next(letters)
    for j in range(rb):
        sb[j] = sb[j] or next(letters)
    out = [sa[i] for i in lb] + [sa[i] for i in range(ra) if i not in lc and i not in lb] + \
          [sb[j] for j in range(rb) if j not in rc and j not in rb_]
    return f"{''.join(sa)},{''.join(sb)}->{''.join(out)}"


@pytest.mark.parametrize("sa,sb,lc,rc,lb,rb", DIMS, ids=[f"case{i}" for i in range(len(DIMS))])
@pytest.mark.parametrize("dt", ["int32", "float32", "bfloat16"])
def test_dimension_numbers_match_einsum(client, sa, sb, lc, rc, lb, rb, dt):
    rng = np.random.default_rng(len(sa) * 7 + len(lc))
    spec = _einsum_spec(len(sa), len(sb), lc, rc, lb, rb)
    print(f"[dot] {dt} {sa} x {sb} {spec}", flush=True)
    text = P.dot_general_dims(sa, sb, dt, lc, rc, lb, rb)
    if dt == "int32":
        a, b = _arr(rng, sa, "int32"), _arr(rng, sb, "int32")
        y = run(client, text, a, b)
        want = np.einsum(spec, a.astype(np.int64), b.astype(np.int64)).astype(np.int32)
        assert y.dtype == np.int32 and np.array_equal(y, want)
        return
    af = rng.standard_normal(sa).astype(np.float32)
    bf = rng.standard_normal(sb).astype(np.float32)
    if dt == "bfloat16":
        ab, bb = f32_to_bf16_bits(af), f32_to_bf16_bits(bf)
        y = bf16_bits_to_f32(run(client, text, (ab, rt.BF16), (bb, rt.BF16)))
        af, bf = bf16_bits_to_f32(ab), bf16_bits_to_f32(bb)
        tol = 2e-2
    else:
        y = run(client, text, af, bf)
        tol = 1e-5
    want = np.einsum(spec, af.astype(np.float64), bf.astype(np.float64))
    assert y.shape == want.shape
    assert_rel_close(y.astype(np.float64), want, tol, f"{dt} {spec}")


@pytest.mark.parametrize("sa,sb,lc,rc,lb,rb", [
    ((512, 256), (768, 256), (1,), (1,), (), ()),              # x @ W.T
    ((2, 256, 64), (2, 512, 64), (2,), (2,), (0,), (0,)),      # q @ k^T per batch
])
def test_rhs_contracting_last_runs_on_the_nt_gemm(client, monkeypatch, sa, sb, lc, rc, lb, rb):
    """An rhs whose contracting dimension is last is read in place by the
    GEMM that takes B^T: no operand copy in the plan, and the same bits as
    the copy-then-GEMM plan (MK_PLAN_GEMM_NT=0)."""
    rng = np.random.default_rng(sum(sa) + sum(sb))
    text = P.dot_general_dims(sa, sb, "bfloat16", lc, rc, lb, rb)
    ab = f32_to_bf16_bits(rng.standard_normal(sa).astype(np.float32))
    bb = f32_to_bf16_bits(rng.standard_normal(sb).astype(np.float32))
    print(f"[dot] nt {sa} x {sb}", flush=True)
    exe = client.compile(text)
    assert "gemm_bf16_nt" in exe.plan and "gemm operand b" not in exe.plan, exe.plan
    exe.close()
    y_nt = run(client, text, (ab, rt.BF16), (bb, rt.BF16))
    monkeypatch.setenv("MK_PLAN_GEMM_NT", "0")
    exe = client.compile(text)
    assert "gemm_bf16_nt" not in exe.plan, exe.plan
    exe.close()
    y_cp = run(client, text, (ab, rt.BF16), (bb, rt.BF16))
    assert np.array_equal(np.asarray(y_nt).view(np.uint16), np.asarray(y_cp).view(np.uint16))
    want = np.einsum(_einsum_spec(len(sa), len(sb), lc, rc, lb, rb), bf16_bits_to_f32(ab).astype(np.float64),
                     bf16_bits_to_f32(bb).astype(np.float64))
    assert_rel_close(bf16_bits_to_f32(y_nt).astype(np.float64), want, 2e-2, f"nt {sa} x {sb}")
