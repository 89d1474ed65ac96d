"""Pins for the CPU oracle (runs without a GPU).

Each oracle function is checked against something that does not retype its
formula: the reference tests' known answers and special-value matrices,
closed forms, invariants and brute-force loops on tiny inputs.  A plausible
mistake (a swapped nibble, a dropped zero-point, a transposed operand, a
wrong NaN rule) fails at least one test here.
"""

import math

import numpy as np
import pytest

from oracle import bf16, eltwise, gemm, quant, rowops


# --------------------------------------------------------------------- bf16

def test_bf16_exact_values_and_rne_ties():
    vals = np.array([1.0, -2.0, 0.0, -0.0, 0.5, 65280.0], np.float32)
    assert list(bf16.f32_to_bf16_bits(vals)) == [0x3F80, 0xC000, 0x0000, 0x8000, 0x3F00, 0x477F]
    # 1 + 2^-8 is halfway between 1.0 (even) and 1 + 2^-7: ties go to even.
    assert bf16.f32_to_bf16_bits(np.float32(1 + 2 ** -8)) == 0x3F80
    # 1 + 3*2^-8 is halfway between 0x3F81 (odd) and 0x3F82 (even).
    assert bf16.f32_to_bf16_bits(np.float32(1 + 3 * 2 ** -8)) == 0x3F82
    # just above halfway rounds up
    assert bf16.f32_to_bf16_bits(np.float32(1 + 2 ** -8 + 2 ** -20)) == 0x3F81


def test_bf16_specials():
    b = bf16.f32_to_bf16_bits(np.array([np.inf, -np.inf, np.nan, 3.4028235e38], np.float32))
    assert b[0] == 0x7F80 and b[1] == 0xFF80
    assert (b[2] & 0x7F80) == 0x7F80 and (b[2] & 0x7F) != 0
    assert b[3] == 0x7F80  # rounds past the largest finite bf16
    x = np.array([1.5, -3.25, 1e-3], np.float32)
    assert np.array_equal(bf16.round_bf16(bf16.round_bf16(x)), bf16.round_bf16(x))


# --------------------------------------------------------------- int4 / int8

def test_int4_pack_literal_bytes():
    q = np.array([[1, 15], [2, 0], [3, 7], [4, 8]], np.uint8)  # K=4, N=2
    p = quant.pack_int4_k(q)
    assert p.tolist() == [[0x21, 0x0F], [0x43, 0x87]]
    assert np.array_equal(quant.unpack_int4_k(p), q)


def test_int4_pack_roundtrip_random():
    rng = np.random.default_rng(0)
    q = rng.integers(0, 16, size=(128, 33), dtype=np.uint8)
    assert np.array_equal(quant.unpack_int4_k(quant.pack_int4_k(q)), q)
    with pytest.raises(ValueError):
        quant.pack_int4_k(np.full((2, 2), 16, np.uint8))


def _brute_int4(x_bits, packed, s_bits, z, round_w):
    # Independent restatement: reads nibbles straight from the bytes.
    M, K = x_bits.shape
    N = packed.shape[1]
    xs = bf16.bf16_bits_to_f32(x_bits)
    ss = bf16.bf16_bits_to_f32(s_bits)
    y = np.zeros((M, N))
    for n in range(N):
        for k in range(K):
            byte = int(packed[k // 2, n])
            qv = (byte >> 4) if (k % 2) else (byte & 0xF)
            w = float(np.float32(qv - int(z[k // 64, n])) * ss[k // 64, n])
            if round_w:
                w = float(bf16.round_bf16(np.float32(w)))
            for m in range(M):
                y[m, n] += float(xs[m, k]) * w
    return y


@pytest.mark.parametrize("round_w", [True, False])
def test_int4_matmul_brute_force(round_w):
    rng = np.random.default_rng(1)
    x, p, s, z = quant.make_int4_case(rng, 3, 128, 5)
    y, yb = quant.int4_g64_matmul(x, p, s, z, round_w=round_w)
    ref = _brute_int4(x, p, s, z, round_w)
    np.testing.assert_allclose(y, ref, rtol=1e-12, atol=1e-12)
    np.testing.assert_array_equal(yb, bf16.f32_to_bf16_bits(ref.astype(np.float32)))


def test_int4_matmul_all_ones_closed_form():
    rng = np.random.default_rng(2)
    K, N = 256, 7
    q = np.ones((K, N), np.uint8)
    z = np.zeros((K // 64, N), np.uint8)
    s = bf16.f32_to_bf16_bits(rng.uniform(1e-3, 1e-2, size=(K // 64, N)).astype(np.float32))
    x = bf16.f32_to_bf16_bits(np.ones((2, K), np.float32))
    y, _ = quant.int4_g64_matmul(x, quant.pack_int4_k(q), s, z)
    expect = 64.0 * bf16.bf16_bits_to_f32(s).astype(np.float64).sum(axis=0)
    np.testing.assert_allclose(y, np.broadcast_to(expect, y.shape), rtol=1e-12)


def test_int4_zero_point_sign():
    # q = z everywhere -> the dequantized weight is exactly zero.
    q = np.full((128, 4), 9, np.uint8)
    z = np.full((2, 4), 9, np.uint8)
    s = bf16.f32_to_bf16_bits(np.full((2, 4), 0.5, np.float32))
    x = bf16.f32_to_bf16_bits(np.arange(256, dtype=np.float32).reshape(2, 128))
    y, _ = quant.int4_g64_matmul(x, quant.pack_int4_k(q), s, z)
    assert np.all(y == 0)
    # q = z + 1 -> weight = s: Y = 0.5 * row sums
    y, _ = quant.int4_g64_matmul(x, quant.pack_int4_k(q + 1), s, z)
    np.testing.assert_allclose(y[:, 0], 0.5 * bf16.bf16_bits_to_f32(x).sum(axis=1))


def test_int8_brute_force_and_identity():
    rng = np.random.default_rng(3)
    x, w, s = quant.make_int8_case(rng, 2, 64, 3)
    y, _ = quant.int8_pc_matmul(x, w, s)
    xs = bf16.bf16_bits_to_f32(x)
    ref = np.zeros((2, 3))
    for m in range(2):
        for n in range(3):
            acc = 0.0
            for k in range(64):
                acc += float(xs[m, k]) * int(w[k, n])
            ref[m, n] = acc * float(s[n])
    np.testing.assert_allclose(y, ref, rtol=1e-12)
    eye = np.eye(8, dtype=np.int8)
    x8 = bf16.randn_bf16(rng, (4, 8))
    y8, _ = quant.int8_pc_matmul(x8, eye, np.ones(8, np.float32))
    np.testing.assert_array_equal(y8, bf16.bf16_bits_to_f32(x8))


# ------------------------------------------ the reference's affine quantizer

@pytest.mark.parametrize("bits", [4, 8])
def test_affine_roundtrip_reference_tolerance(bits):
    # tests/test_quantized.py:418-431
    rng = np.random.default_rng(42)
    w = rng.standard_normal((8, 128)).astype(np.float32) * 0.1
    packed, sc, bi = quant.affine_quantize(w, bits=bits, group_size=64)
    back = quant.affine_dequantize(packed, sc, bi, bits=bits, group_size=64, shape=w.shape)
    atol = 0.02 if bits == 8 else 0.05
    np.testing.assert_allclose(back, w, atol=atol, rtol=0.3)
    # and the max error is at most half a step per group
    step = np.repeat(sc, 64, axis=1)
    assert np.all(np.abs(back - w) <= 0.5 * step + 1e-6)


@pytest.mark.parametrize("bits", [4, 8])
def test_affine_shapes(bits):
    # tests/test_quantized.py:433-447
    packed, sc, bi = quant.affine_quantize(np.ones((16, 128), np.float32), bits=bits, group_size=64)
    if bits == 4:
        assert packed.shape == (16, 16) and packed.dtype == np.uint32
    else:
        assert packed.shape == (16, 128) and packed.dtype == np.uint8
    assert sc.shape == (16, 2) and bi.shape == (16, 2)


def test_affine_zeros():
    # tests/test_quantized.py:449-455
    w = np.zeros((2, 64), np.float32)
    packed, sc, bi = quant.affine_quantize(w, bits=4, group_size=32)
    back = quant.affine_dequantize(packed, sc, bi, bits=4, group_size=32, shape=w.shape)
    np.testing.assert_allclose(back, 0.0, atol=1e-6)


def test_affine_matmul_reference_tolerance():
    # tests/test_quantized.py:461-485 (4-bit, f32 activations)
    rng = np.random.default_rng(42)
    x = rng.standard_normal((8, 128)).astype(np.float32) * 0.1
    w = rng.standard_normal((16, 128)).astype(np.float32) * 0.1
    ref = x @ w.T
    packed, sc, bi = quant.affine_quantize(w, bits=4, group_size=64)
    wd = quant.affine_dequantize(packed, sc, bi, bits=4, group_size=64, shape=w.shape)
    np.testing.assert_allclose(x @ wd.T, ref, atol=0.05, rtol=0.3)


def test_affine_ones_known_answer_through_hot_path_format():
    # tests/test_quantized.py:528-541: ones(1,64) @ ones(2,64).T == [[64, 64]]
    w = np.ones((2, 64), np.float32)
    packed, sc, bi = quant.affine_quantize(w, bits=4, group_size=64)
    p, s, z = quant.affine_to_int4_g64(packed, sc, bi, K=64)
    x = bf16.f32_to_bf16_bits(np.ones((1, 64), np.float32))
    y, yb = quant.int4_g64_matmul(x, p, s, z)
    np.testing.assert_array_equal(y, [[64.0, 64.0]])
    np.testing.assert_array_equal(bf16.bf16_bits_to_f32(yb), [[64.0, 64.0]])


def test_affine_converter_matches_reference_dequant():
    # A weight whose affine code is representable: w = 0.25 * (q - 3)
    rng = np.random.default_rng(5)
    q = rng.integers(0, 16, size=(4, 128))
    q[:, ::64] = 0
    q[:, 1::64] = 15
    w = (0.25 * (q - 3)).astype(np.float32)
    packed, sc, bi = quant.affine_quantize(w, bits=4, group_size=64)
    ref = quant.affine_dequantize(packed, sc, bi, bits=4, group_size=64, shape=w.shape)
    p, s, z = quant.affine_to_int4_g64(packed, sc, bi, K=128)
    mine = quant.int4_g64_dequant(p, s, z)
    np.testing.assert_array_equal(mine.T, ref)


# -------------------------------------------------------------------- GEMM

def test_gemm_identity_ones_and_overflow_case():
    rng = np.random.default_rng(6)
    a = rng.standard_normal((16, 16)).astype(np.float32)
    np.testing.assert_array_equal(gemm.dot_general(a, np.eye(16)), a)
    ones = gemm.dot_general(np.ones((3, 37)), np.ones((37, 5)))
    assert np.all(ones == 37)
    # tests/test_f32_gemm_precision.py:55-60: every product 7e4 * 1/1024.
    c, c32 = gemm.matmul_f32(np.full((8, 1024), 7e4, np.float32), np.full((1024, 8), 1 / 1024, np.float32))
    np.testing.assert_allclose(c32, 7e4, rtol=1e-6)


def test_gemm_k1_signed_zero():
    # ops/binary_ops.mm:904-1004: K == 1 is a multiply and keeps -0.
    c = gemm.dot_general(np.array([[-0.0, 2.0]]).T, np.array([[1.0, -0.0]]))
    assert np.signbit(c[0, 0]) and c[0, 0] == 0
    assert np.signbit(c[1, 1]) and c[1, 1] == 0


def test_dot_general_batch_contract_brute_force():
    rng = np.random.default_rng(7)
    a = rng.standard_normal((2, 3, 4))   # [b, k, m]
    b = rng.standard_normal((4, 2, 3))   # [n, b, k]
    c = gemm.dot_general(a, b, lhs_batch=(0,), rhs_batch=(1,), lhs_contract=(1,), rhs_contract=(2,))
    assert c.shape == (2, 4, 4)
    for bi in range(2):
        for m in range(4):
            for n in range(4):
                s = sum(a[bi, k, m] * b[n, bi, k] for k in range(3))
                assert abs(c[bi, m, n] - s) < 1e-12


def test_rel_err_measure():
    assert gemm.rel_err([1.0, 2.0], [1.0, 2.0]) == 0
    assert gemm.rel_err([1.0, 2.5], [1.0, 2.0]) == 0.25


# ----------------------------------------------------------------- rowops

def _softmax_special():
    # restates tests/test_native_softmax.py:_special
    rng = np.random.default_rng(7)
    x = (rng.standard_normal((8, 40)) * 4).astype(np.float32)
    x[0, 3] = np.nan
    x[1, :] = -np.inf
    x[2, 5] = np.inf
    x[3, 0] = np.nan
    x[3, 1:] = -np.inf
    x[4, :] = 80.0
    x[5, 7] = -np.inf
    return x


def test_softmax_special_rows():
    x = _softmax_special()
    y = rowops.softmax(x)
    for r in range(4):
        assert np.all(np.isnan(y[r])), r
    np.testing.assert_allclose(y[4], 1 / 40)
    assert y[5, 7] == 0
    for r in (5, 6, 7):
        assert abs(y[r].sum() - 1) < 1e-12
        row = x[r].astype(np.float64)
        e = [math.exp(v - max(row)) for v in row]
        np.testing.assert_allclose(y[r], np.array(e) / sum(e), rtol=1e-12)


def test_softmax_bf16_rounding_points():
    x = bf16.f32_to_bf16_bits(np.array([[0.0, 0.0, 0.0, 0.0], [1.0, 1.0, 1.0, 80.0]], np.float32))
    y = bf16.bf16_bits_to_f32(rowops.softmax_bf16(x))
    np.testing.assert_array_equal(y[0], [0.25] * 4)
    assert y[1, 3] == 1.0
    np.testing.assert_allclose(y[1, :3], math.exp(-79.0), rtol=2 ** -7)


def test_rmsnorm_closed_form_and_loop():
    g = np.array([0.5, 1.0, 1.5, 2.0])
    x = np.full((1, 4), -3.0)
    y = rowops.rmsnorm(x, g, eps=0.0)
    np.testing.assert_allclose(y[0], -g)
    rng = np.random.default_rng(8)
    x = rng.standard_normal((3, 9))
    g = rng.uniform(0.5, 1.5, 9)
    y = rowops.rmsnorm(x, g)
    for r in range(3):
        ms = sum(v * v for v in x[r]) / 9
        for c in range(9):
            assert abs(y[r, c] - x[r, c] / math.sqrt(ms + 1e-6) * g[c]) < 1e-12


def _edge(shape, seed):
    # restates tests/test_argreduce_nan.py:_edge
    special_vals = np.array([np.nan, np.inf, -np.inf, 0.0, -0.0, 1.0, -1.0, 3.5], np.float32)
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(shape).astype(np.float32)
    special = rng.random(shape) < 0.7
    x[special] = rng.choice(special_vals, size=int(special.sum()))
    return x


@pytest.mark.parametrize("shape,seed", [((512, 37), 0), ((300, 1), 0), ((8, 2049), 3), ((64, 300), 5)])
def test_argmax_special_values_vs_brute(shape, seed):
    x = _edge(shape, seed)
    got = rowops.argmax(x)
    ref = [rowops.brute_argmax_row(list(row)) for row in x]
    np.testing.assert_array_equal(got, ref)


def test_argmax_known_rows():
    # tests/test_argreduce_nan.py:57-66 with the answers XLA's rule fixes.
    x = np.random.default_rng(1).standard_normal((6, 16)).astype(np.float32)
    x[0] = np.nan
    x[1, 5] = np.nan
    x[1, 9] = np.nan
    x[2] = 2.0
    x[3, :4] = [np.inf, np.nan, -np.inf, np.nan]
    x[4, -1] = np.nan
    got = rowops.argmax(x)
    assert got[:5].tolist() == [0, 5, 0, 1, 15]
    assert got[5] == int(np.argmax(x[5]))
    z = np.array([[-0.0, 0.0], [0.0, -0.0], [-1.0, -0.0]], np.float32)
    assert rowops.argmax(z).tolist() == [0, 0, 1]


def test_argmax_int_ties_lowest_index():
    x = np.array([[5, 9, 9, 1], [-3, -3, -3, -3]], np.int32)
    assert rowops.argmax(x).tolist() == [1, 0]


def test_reduce_sum_max():
    x = np.array([[1.0, np.nan, 2.0], [-0.0, 0.0, -1.0], [-0.0, -0.0, -2.0], [1.0, 2.0, 3.0]])
    m = rowops.reduce_max(x)
    assert np.isnan(m[0])
    assert m[1] == 0 and not np.signbit(m[1])
    assert m[2] == 0 and np.signbit(m[2])
    assert m[3] == 3
    assert rowops.reduce_sum(x[3:]).tolist() == [6.0]


# ----------------------------------------------------------------- eltwise

@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_chain6_spot_values(dtype):
    x = np.array([0.0, -1.0, 2.0, -0.0], np.float32)
    y = eltwise.evaluate(eltwise.CHAIN6, [x], dtype)
    assert y[0] == 0.5 and y[1] == -1.0 and y[3] == 0.5
    if dtype == "f32":
        assert abs(y[2] - math.log1p(math.exp(3.5))) < 1e-6
    else:
        # exp(3.5) = 33.115 rounds to 33.0 in bf16, log1p(33) = 3.5264 -> 3.53125
        assert y[2] == 3.53125


def test_chain6_brute_force_per_element():
    rng = np.random.default_rng(9)
    x = (rng.standard_normal(200) * math.sqrt(2)).astype(np.float32)
    y = eltwise.evaluate(eltwise.CHAIN6, [x], "f32")
    for v, out in zip(x.tolist(), y.tolist()):
        b = float(np.float32(float(np.float32(v * 1.5)) + 0.5))
        d = float(np.float32(math.log1p(float(np.float32(math.exp(b))))))
        ref = max(d, v) if v > 0 else b
        assert abs(out - ref) <= 1e-6 * max(1.0, abs(ref))


def test_eltwise_nan_and_signed_zero_max():
    prog = [("maximum", (0, 1))]
    a = np.array([np.nan, 1.0, -0.0, 0.0], np.float32)
    b = np.array([1.0, np.nan, 0.0, -0.0], np.float32)
    y = eltwise.evaluate(prog, [a, b])
    assert np.isnan(y[0]) and np.isnan(y[1])
    assert y[2] == 0 and not np.signbit(y[2]) and not np.signbit(y[3])


# ------------------------------------------------- the C port (oracle/c)
#
# oracle/c/oracle.c is the checker for the full-size quantized, GEMM and
# argmax GPU tests and the bench's CPU baseline.  It accumulates in f32 (the
# numpy restatements in float64), so it is held to the numpy oracle at a
# relative 1e-5 of each output's magnitude, to brute-force loops, and to
# closed forms that f32 accumulation reproduces exactly.  Shapes cover the
# port's 64-row and 64-column chunking: M > 64 with a ragged last chunk, N not
# a multiple of 64, several K groups, and column slices (n_range / m_range).

def _cport():
    from oracle import cport
    try:
        cport.lib()
    except RuntimeError as e:  # pragma: no cover - the build step makes it
        pytest.fail(str(e))
    return cport


def _close_f32_accum(out, ref, K):
    """f32 accumulation of K products vs float64: |err| <= K * 2^-23 * sum|terms|,
    bounded here by a normwise 1e-5 (K <= 512) and an elementwise check."""
    out = np.asarray(out, np.float64)
    ref = np.asarray(ref, np.float64)
    scale = max(np.max(np.abs(ref)), 1e-30)
    assert np.max(np.abs(out - ref)) <= 1e-5 * scale


@pytest.mark.parametrize("M,K,N", [(70, 192, 100), (130, 128, 65), (1, 64, 8), (65, 256, 129)])
def test_cport_int4_matches_numpy_oracle(M, K, N):
    cport = _cport()
    rng = np.random.default_rng(M * 1000 + K + N)
    x, p, s, z = quant.make_int4_case(rng, M, K, N)
    ref, _ = quant.int4_g64_matmul(x, p, s, z, round_w=True)
    got = cport.int4_g64_matmul(x, p, s, z)
    _close_f32_accum(got, ref, K)


def test_cport_int4_brute_force_and_column_slice():
    cport = _cport()
    rng = np.random.default_rng(31)
    x, p, s, z = quant.make_int4_case(rng, 3, 128, 5)
    got = cport.int4_g64_matmul(x, p, s, z)
    _close_f32_accum(got, _brute_int4(x, p, s, z, round_w=True), 128)
    # Column slice: the columns in [n0, n1) equal the full result, the rest stay 0.
    x, p, s, z = quant.make_int4_case(rng, 70, 128, 200)
    full = cport.int4_g64_matmul(x, p, s, z)
    part = cport.int4_g64_matmul(x, p, s, z, n_range=(37, 101))
    np.testing.assert_array_equal(part[:, 37:101], full[:, 37:101])
    assert not part[:, :37].any() and not part[:, 101:].any()


def test_cport_int4_nibble_order_and_zero_point():
    """A swapped nibble or a dropped zero-point fails these closed forms:
    even k carries q = 1, odd k q = 3 (low nibble = even k), z = 1, s = 0.5,
    x = 1 on even k and 0 on odd k -> every output is 0 (q - z = 0 on even k);
    x = 1 on odd k only -> every output is (K/2) * (3 - 1) * 0.5 = K/2."""
    cport = _cport()
    K, N = 256, 70
    q = np.zeros((K, N), np.uint8)
    q[0::2] = 1
    q[1::2] = 3
    p = quant.pack_int4_k(q)
    assert p[0, 0] == 0x31
    s = np.full((K // 64, N), 0x3F00, np.uint16)   # 0.5
    z = np.ones((K // 64, N), np.uint8)
    x = np.zeros((2, K), np.float32)
    x[0, 0::2] = 1.0
    x[1, 1::2] = 1.0
    y = cport.int4_g64_matmul(bf16.f32_to_bf16_bits(x), p, s, z)
    assert np.all(y[0] == 0.0)
    assert np.all(y[1] == K / 2)


@pytest.mark.parametrize("M,K,N", [(70, 192, 100), (1, 64, 8), (130, 320, 65)])
def test_cport_int8_matches_numpy_oracle(M, K, N):
    cport = _cport()
    rng = np.random.default_rng(M * 7 + K + N)
    x, w, s = quant.make_int8_case(rng, M, K, N)
    ref, _ = quant.int8_pc_matmul(x, w, s)
    _close_f32_accum(cport.int8_pc_matmul(x, w, s), ref, K)
    part = cport.int8_pc_matmul(x, w, s, n_range=(5, N - 3))
    full = cport.int8_pc_matmul(x, w, s)
    np.testing.assert_array_equal(part[:, 5:N - 3], full[:, 5:N - 3])


def test_cport_int8_brute_force_and_identity():
    cport = _cport()
    rng = np.random.default_rng(33)
    x, w, s = quant.make_int8_case(rng, 2, 64, 3)
    xs = bf16.bf16_bits_to_f32(x)
    ref = np.array([[sum(float(xs[m, k]) * int(w[k, n]) for k in range(64)) * float(s[n])
                     for n in range(3)] for m in range(2)])
    _close_f32_accum(cport.int8_pc_matmul(x, w, s), ref, 64)
    # W = I, s = 1: Y = X exactly (a transposed W or a scale on the wrong
    # axis fails this).
    eye = np.eye(80, dtype=np.int8)
    x8 = bf16.randn_bf16(rng, (3, 80))
    y = cport.int8_pc_matmul(x8, eye, np.ones(80, np.float32))
    np.testing.assert_array_equal(y, bf16.bf16_bits_to_f32(x8))
    sc = np.arange(1, 81, dtype=np.float32)
    y = cport.int8_pc_matmul(x8, eye, sc)
    np.testing.assert_array_equal(y, bf16.bf16_bits_to_f32(x8) * sc[None, :])


@pytest.mark.parametrize("M,K,N", [(70, 96, 33), (3, 512, 130)])
def test_cport_gemm_bf16_matches_numpy_oracle(M, K, N):
    cport = _cport()
    rng = np.random.default_rng(M + K + N)
    a = bf16.randn_bf16(rng, (M, K))
    b = bf16.randn_bf16(rng, (K, N))
    ref, _ = gemm.matmul_bf16(a, b)
    _close_f32_accum(cport.gemm_bf16(a, b), ref, K)
    part = cport.gemm_bf16(a, b, m_range=(1, M - 1))
    np.testing.assert_array_equal(part[1:M - 1], cport.gemm_bf16(a, b)[1:M - 1])


def test_cport_gemm_bf16_closed_forms():
    """A @ I == A exactly; ones @ ones == K exactly; a non-square A @ B.T
    transposition mistake changes the shape/values of the asymmetric case."""
    cport = _cport()
    rng = np.random.default_rng(34)
    a = bf16.randn_bf16(rng, (9, 64))
    eye = bf16.f32_to_bf16_bits(np.eye(64, dtype=np.float32))
    np.testing.assert_array_equal(cport.gemm_bf16(a, eye), bf16.bf16_bits_to_f32(a))
    ones_a = bf16.f32_to_bf16_bits(np.ones((4, 300), np.float32))
    ones_b = bf16.f32_to_bf16_bits(np.ones((300, 7), np.float32))
    assert np.all(cport.gemm_bf16(ones_a, ones_b) == 300)
    # Row-index matrix times column-index matrix: C[m, n] = sum_k m * n = K m n.
    K = 16
    am = bf16.f32_to_bf16_bits(np.repeat(np.arange(5, dtype=np.float32)[:, None], K, axis=1))
    bn = bf16.f32_to_bf16_bits(np.repeat(np.arange(3, dtype=np.float32)[None, :], K, axis=0))
    c = cport.gemm_bf16(am, bn)
    np.testing.assert_array_equal(c, K * np.outer(np.arange(5), np.arange(3)))


def test_cport_gemm_f32_pins():
    """The C port's f32 GEMM (the f32 GEMM line's CPU baseline): against
    float64 within the f32 accumulation bound on a ragged shape, a row slice
    equal to the full product's rows, A @ I == A exactly, and the
    row-index x column-index closed form K m n (exact in f32), which a
    transposed operand or a wrong stride fails."""
    cport = _cport()
    rng = np.random.default_rng(35)
    M, K, N = 37, 130, 45
    a = rng.standard_normal((M, K)).astype(np.float32)
    b = rng.standard_normal((K, N)).astype(np.float32)
    _close_f32_accum(cport.gemm_f32(a, b), a.astype(np.float64) @ b.astype(np.float64), K)
    part = cport.gemm_f32(a, b, m_range=(2, M - 3))
    np.testing.assert_array_equal(part[2:M - 3], cport.gemm_f32(a, b)[2:M - 3])
    np.testing.assert_array_equal(cport.gemm_f32(a, np.eye(K, dtype=np.float32)), a)
    Kc = 24
    am = np.repeat(np.arange(6, dtype=np.float32)[:, None], Kc, axis=1)
    bn = np.repeat(np.arange(5, dtype=np.float32)[None, :], Kc, axis=0)
    np.testing.assert_array_equal(cport.gemm_f32(am, bn), Kc * np.outer(np.arange(6), np.arange(5)))


@pytest.mark.parametrize("shape,seed", [((512, 37), 0), ((300, 1), 0), ((8, 2049), 3), ((64, 300), 5)])
def test_cport_argmax_matches_brute(shape, seed):
    cport = _cport()
    x = _edge(shape, seed)
    ref = [rowops.brute_argmax_row(list(row)) for row in x]
    np.testing.assert_array_equal(cport.argmax_f32(x), ref)
    np.testing.assert_array_equal(cport.argmax_f32(x), rowops.argmax(x))


def test_cport_argmax_known_rows():
    cport = _cport()
    x = np.random.default_rng(1).standard_normal((6, 16)).astype(np.float32)
    x[0] = np.nan
    x[1, 5] = np.nan
    x[1, 9] = np.nan
    x[2] = 2.0
    x[3, :4] = [np.inf, np.nan, -np.inf, np.nan]
    x[4, -1] = np.nan
    got = cport.argmax_f32(x)
    assert got[:5].tolist() == [0, 5, 0, 1, 15]
    z = np.array([[-0.0, 0.0], [0.0, -0.0], [-1.0, -0.0]], np.float32)
    assert cport.argmax_f32(z).tolist() == [0, 0, 1]


@pytest.mark.parametrize("shape,seed", [((512, 37), 0), ((8, 2049), 3), ((64, 300), 5)])
def test_cport_argmax_bf16_matches_numpy(shape, seed):
    cport = _cport()
    xb = bf16.f32_to_bf16_bits(_edge(shape, seed))
    xf = bf16.bf16_bits_to_f32(xb)
    np.testing.assert_array_equal(cport.argmax_bf16(xb), rowops.argmax(xf))
    ties = bf16.f32_to_bf16_bits(np.round(np.random.default_rng(seed).standard_normal((32, 512)) * 2) / 2)
    np.testing.assert_array_equal(cport.argmax_bf16(ties), rowops.argmax(bf16.bf16_bits_to_f32(ties)))


def _rows_case(rows, cols, seed):
    x = (np.random.default_rng(seed).standard_normal((rows, cols)) * np.sqrt(2)).astype(np.float32)
    # the reference's special softmax rows (tests/test_native_softmax.py:26-35)
    x[0] = np.nan
    x[1] = -np.inf
    x[2, 3] = np.inf
    x[3] = 80.0
    return x


def test_cport_softmax_f32_matches_numpy_and_special_rows():
    cport = _cport()
    x = _rows_case(40, 1000, 11)
    y = cport.softmax(x)
    ref = rowops.softmax(x)
    assert np.array_equal(np.isnan(y), np.isnan(ref))
    fin = ~np.isnan(ref)
    np.testing.assert_allclose(y[fin], ref[fin], rtol=1e-5, atol=1e-12)
    np.testing.assert_allclose(y[3], 1.0 / 1000, rtol=1e-6)  # constant row: uniform
    np.testing.assert_allclose(y[4:].sum(axis=1), 1.0, rtol=1e-5)
    part = cport.softmax(x, row_range=(5, 9))
    np.testing.assert_array_equal(part[5:9], y[5:9])
    assert not part[:5].any() and not part[9:].any()


def test_cport_softmax_bf16_matches_numpy_rounding_points():
    cport = _cport()
    xb = bf16.f32_to_bf16_bits(_rows_case(40, 1000, 12))
    got = cport.softmax(xb)
    ref = rowops.softmax_bf16(xb)
    gf, rf = bf16.bf16_bits_to_f32(got), bf16.bf16_bits_to_f32(ref)
    assert np.array_equal(np.isnan(gf), np.isnan(rf))
    fin = ~np.isnan(rf)
    # the same rounding points; expf may move a rounding by one bf16 ulp
    np.testing.assert_array_less(np.abs(gf[fin] - rf[fin]), 2.0 ** -7 * np.abs(rf[fin]) + 1e-30)
    assert np.mean(got[fin] == ref[fin]) > 0.99


def test_cport_rmsnorm_matches_numpy():
    cport = _cport()
    rng = np.random.default_rng(13)
    x = (rng.standard_normal((33, 777)) * np.sqrt(2)).astype(np.float32)
    g = rng.uniform(0.5, 1.5, 777).astype(np.float32)
    ref = rowops.rmsnorm(x, g)
    np.testing.assert_allclose(cport.rmsnorm(x, g), ref, rtol=1e-5, atol=1e-7)
    # closed form: a constant row c gives c / sqrt(c^2 + eps) * g
    c = np.full((2, 64), 3.0, np.float32)
    np.testing.assert_allclose(cport.rmsnorm(c, np.ones(64, np.float32)), 3.0 / np.sqrt(9.0 + 1e-6), rtol=1e-6)
    xb, gb = bf16.f32_to_bf16_bits(x), bf16.f32_to_bf16_bits(g)
    got = bf16.bf16_bits_to_f32(cport.rmsnorm(xb, gb))
    refb = rowops.rmsnorm(bf16.bf16_bits_to_f32(xb), bf16.bf16_bits_to_f32(gb))
    np.testing.assert_array_less(np.abs(got - refb), 2.0 ** -8 * np.abs(refb) * 1.01 + 1e-30)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_cport_chain6_matches_numpy(dtype):
    cport = _cport()
    rng = np.random.default_rng(14)
    x = (rng.standard_normal(20000) * np.sqrt(2) * 8).astype(np.float32)
    x[:6] = [0.0, -0.0, np.nan, np.inf, -np.inf, 100.0]
    if dtype == "f32":
        got = cport.chain6(x)
        ref = eltwise.evaluate(eltwise.CHAIN6, [x], "f32")
        assert np.array_equal(np.isnan(got), np.isnan(ref))
        fin = ~np.isnan(ref)
        np.testing.assert_allclose(got[fin], ref[fin], rtol=4e-7, atol=0)
    else:
        xb = bf16.f32_to_bf16_bits(x)
        got = bf16.bf16_bits_to_f32(cport.chain6(xb))
        ref = eltwise.evaluate(eltwise.CHAIN6, [bf16.bf16_bits_to_f32(xb)], "bf16")
        assert np.array_equal(np.isnan(got), np.isnan(ref))
        inf = np.isinf(ref)
        np.testing.assert_array_equal(got[inf], ref[inf])
        fin = np.isfinite(ref)
        np.testing.assert_array_less(np.abs(got[fin] - ref[fin]), 2.0 ** -7 * np.abs(ref[fin]) + 1e-30)
        assert np.mean(got[fin] == ref[fin]) > 0.99


def test_cport_plumbing_matches_float64():
    cport = _cport()
    rng = np.random.default_rng(0)
    n = 96
    a = rng.standard_normal((n, n)).astype(np.float32)
    b = rng.standard_normal((n, n)).astype(np.float32)
    ref = np.tanh(a.astype(np.float64) @ b.astype(np.float64)).sum(axis=1)
    y = cport.plumbing(a, b)
    assert np.max(np.abs(y - ref)) / np.max(np.abs(ref)) <= 1e-5
    # closed form: B = 0 gives tanh(0) = 0 everywhere
    assert not cport.plumbing(a, np.zeros_like(b)).any()
    part = cport.plumbing(a, b, row_range=(10, 20))
    np.testing.assert_array_equal(part[10:20], y[10:20])


# ------------------------------------------------------- decoder layer

def test_decoder_rope_closed_forms():
    from oracle import decoder
    cos, sin = decoder.rope_tables(8, 4)
    x = np.array([1.0, 2.0, 3.0, 4.0])
    # position 0: identity
    np.testing.assert_array_equal(decoder.rope(x, cos[0], sin[0]), x)
    # pair i rotates by angle pos * base^(-2i/D): pos 3, pair 0 by 3 rad, pair 1 by 3/100 rad
    y = decoder.rope(x, cos[3], sin[3])
    np.testing.assert_allclose(y[[0, 2]], [math.cos(3) - 3 * math.sin(3), 3 * math.cos(3) + math.sin(3)])
    np.testing.assert_allclose(y[[1, 3]], [2 * math.cos(.03) - 4 * math.sin(.03), 4 * math.cos(.03) + 2 * math.sin(.03)])
    # a rotation keeps each pair's norm
    np.testing.assert_allclose(y[:2] ** 2 + y[2:] ** 2, x[:2] ** 2 + x[2:] ** 2)


def test_decoder_attention_brute_force_and_closed_forms():
    from oracle import decoder
    rng = np.random.default_rng(40)
    S, D = 9, 4
    q, k, v = rng.standard_normal((S, D)), rng.standard_normal((S, D)), rng.standard_normal((S, D))
    pos = np.arange(S)
    out = decoder.attention_causal_rows(q, pos, k, v, 0.5)
    np.testing.assert_array_equal(out[0], v[0])            # one visible key
    for t in range(S):
        w = [math.exp(0.5 * sum(q[t, d] * k[j, d] for d in range(D))) for j in range(t + 1)]
        ref = [sum(w[j] * v[j, d] for j in range(t + 1)) / sum(w) for d in range(D)]
        np.testing.assert_allclose(out[t], ref, rtol=1e-12)
    # equal keys: uniform weights, the mean of the visible values (a mask
    # that let later keys in would fail this)
    out = decoder.attention_causal_rows(q, pos, np.ones((S, D)), v, 1.0)
    for t in range(S):
        np.testing.assert_allclose(out[t], v[:t + 1].mean(axis=0), rtol=1e-12)


def _tiny_layer_weights(rng, hidden, A, F, zero_scale=False):
    def w(K, N):
        q = rng.integers(0, 16, size=(K, N), dtype=np.uint8)
        s = np.zeros((K // 64, N), np.float32) if zero_scale else rng.uniform(4e-3, 6e-3, (K // 64, N))
        return (quant.pack_int4_k(q), bf16.f32_to_bf16_bits(np.asarray(s, np.float32)),
                rng.integers(0, 16, size=(K // 64, N), dtype=np.uint8))
    g = bf16.f32_to_bf16_bits(rng.uniform(0.5, 1.5, hidden).astype(np.float32))
    g2 = bf16.f32_to_bf16_bits(rng.uniform(0.5, 1.5, hidden).astype(np.float32))
    return {"g_attn": g, "g_mlp": g2, "w_qkv": w(hidden, 3 * A), "w_o": w(A, hidden),
            "w_gate": w(hidden, F), "w_up": w(hidden, F), "w_down": w(F, hidden)}


def test_decoder_layer_zero_weights_is_identity():
    from oracle import decoder
    rng = np.random.default_rng(41)
    x = bf16.round_bf16(rng.standard_normal((6, 128)))
    w = _tiny_layer_weights(rng, 128, 128, 128, zero_scale=True)
    out = decoder.layer_rows(x, np.arange(6), w, heads=1, head_dim=128)
    np.testing.assert_array_equal(out, x)


@pytest.mark.parametrize("exact", [False, True])
def test_decoder_layer_rows_brute_force(exact):
    """The subset evaluation equals a plain whole-sequence evaluation written
    with explicit loops over heads and positions, with the dequantised
    weights rounded to bf16 or (exact_weights) exact."""
    from oracle import decoder
    rng = np.random.default_rng(42)
    S, hidden, H, D, F = 5, 128, 2, 64, 192
    x = bf16.round_bf16(rng.standard_normal((S, hidden)))
    w = _tiny_layer_weights(rng, hidden, H * D, F)
    r = bf16.round_bf16
    names = ("w_qkv", "w_o", "w_gate", "w_up", "w_down")
    deq = {n: quant.int4_g64_dequant(*w[n], round_to_bf16=not exact).astype(np.float64) for n in names}
    g1 = bf16.bf16_bits_to_f32(w["g_attn"]).astype(np.float64)
    g2 = bf16.bf16_bits_to_f32(w["g_mlp"]).astype(np.float64)
    cos, sin = decoder.rope_tables(S, D)
    ref = np.zeros((S, hidden))
    h = np.array([r(x[t] / math.sqrt(np.mean(x[t].astype(np.float64) ** 2) + 1e-6) * g1) for t in range(S)])
    qkv = r(h @ deq["w_qkv"])
    for t in range(S):
        a = np.zeros(H * D)
        for hd in range(H):
            def rot(vec, p):
                half = D // 2
                return np.array([vec[i] * cos[p, i] - vec[i + half] * sin[p, i] for i in range(half)] +
                                [vec[i + half] * cos[p, i] + vec[i] * sin[p, i] for i in range(half)])
            qv = r(rot(qkv[t, hd * D:(hd + 1) * D], t))
            ks = [r(rot(qkv[j, H * D + hd * D:H * D + (hd + 1) * D], j)) for j in range(t + 1)]
            vs = [qkv[j, 2 * H * D + hd * D:2 * H * D + (hd + 1) * D] for j in range(t + 1)]
            sc = np.array([float(qv @ kk) / math.sqrt(D) for kk in ks])
            p = np.exp(sc - sc.max())
            p /= p.sum()
            a[hd * D:(hd + 1) * D] = sum(p[j] * vs[j] for j in range(t + 1))
        x1 = r(x[t] + r(r(a) @ deq["w_o"]))
        h2 = r(x1 / math.sqrt(np.mean(x1.astype(np.float64) ** 2) + 1e-6) * g2)
        gg, uu = r(h2 @ deq["w_gate"]), r(h2 @ deq["w_up"])
        act = r(r(gg * r(1 / (1 + np.exp(-gg.astype(np.float64))))) * uu)
        ref[t] = r(x1 + r(act @ deq["w_down"]))
    pos = np.array([4, 0, 2])
    out = decoder.layer_rows(x, pos, w, heads=H, head_dim=D, exact_weights=exact)
    np.testing.assert_allclose(out, ref[pos], rtol=2 ** -7, atol=1e-6)


def test_decoder_exact_weights_only_change_the_weight_rounding():
    """With power-of-two scales every (q - z) * s is a bf16 value, so the
    exact and bf16-rounded weight conventions give identical layers; with
    general scales they differ (the flag is not ignored)."""
    from oracle import decoder
    rng = np.random.default_rng(44)
    S, hidden, H, D, F = 4, 128, 2, 64, 192
    x = bf16.round_bf16(rng.standard_normal((S, hidden)))
    w = _tiny_layer_weights(rng, hidden, H * D, F)
    pos = np.arange(S)
    general = [decoder.layer_rows(x, pos, w, heads=H, head_dim=D, exact_weights=e) for e in (False, True)]
    assert not np.array_equal(general[0], general[1])
    for n in ("w_qkv", "w_o", "w_gate", "w_up", "w_down"):
        p_, s_, z_ = w[n]
        pow2 = 2.0 ** rng.integers(-9, -6, size=s_.shape)
        w[n] = (p_, bf16.f32_to_bf16_bits(pow2.astype(np.float32)), z_)
    same = [decoder.layer_rows(x, pos, w, heads=H, head_dim=D, exact_weights=e) for e in (False, True)]
    np.testing.assert_array_equal(same[0], same[1])
