"""GPU parity of the last-axis row kernels (softmax, RMSNorm, argmax, sum,
max) against the oracle (oracle/rowops.py), including the special-value
rows and matrices the reference's own tests use
(tests/test_native_softmax.py:26-35, tests/test_argreduce_nan.py:28-66 under
/root/reference, restated in the oracle's tests)."""

import numpy as np
import pytest

from _gpu import (BF16_RTOL, F32_RTOL, assert_rel_close, dev, dev_bf16, f32_sum_bound, host_bf16, host_bf16_bits,
                  need_gpu, torch)
from oracle import bf16 as obf
from oracle import rowops

pytestmark = pytest.mark.gpu

SHAPES = [(4, 40), (8, 8192), (3, 1000), (5, 4097), (2, 20000), (16, 256), (7, 1)]


def _ops():
    need_gpu()
    from mi355x import ops
    return ops


def _x(shape, seed, scale=np.sqrt(2.0)):
    return (np.random.default_rng(seed).standard_normal(shape) * scale).astype(np.float32)


def _softmax_special():
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


def _edge(shape, seed):
    special_vals = np.array([np.nan, np.inf, -np.inf, 0.0, -0.0, 1.0, -1.0, 3.5], np.float32)
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(shape).astype(np.float32)
    special = rng.random(shape) < 0.7
    x[special] = rng.choice(special_vals, size=int(special.sum()))
    return x


@pytest.mark.parametrize("shape", SHAPES)
def test_softmax_f32(shape):
    ops = _ops()
    x = _x(shape, 1)
    y = ops.softmax(dev(x)).cpu().numpy()
    assert_rel_close(y, rowops.softmax(x), F32_RTOL, f"softmax f32 {shape}")


@pytest.mark.parametrize("shape", SHAPES)
def test_softmax_bf16(shape):
    ops = _ops()
    xb = obf.f32_to_bf16_bits(_x(shape, 2))
    y = host_bf16(ops.softmax(dev_bf16(xb)))
    ref = obf.bf16_bits_to_f32(rowops.softmax_bf16(xb))
    assert_rel_close(y, ref, BF16_RTOL, f"softmax bf16 {shape}")


def test_softmax_special_rows():
    ops = _ops()
    x = _softmax_special()
    y = ops.softmax(dev(x)).cpu().numpy()
    ref = rowops.softmax(x)
    for r in range(4):
        assert np.all(np.isnan(y[r])), r
    assert np.all(y[4] == np.float32(1 / 40)) or np.allclose(y[4], 1 / 40, rtol=1e-6)
    assert y[5, 7] == 0
    assert_rel_close(y[5:], ref[5:], F32_RTOL, "softmax special finite rows")


def test_softmax_bf16_special_rows():
    ops = _ops()
    xb = obf.f32_to_bf16_bits(_softmax_special())
    y = host_bf16(ops.softmax(dev_bf16(xb)))
    ref = obf.bf16_bits_to_f32(rowops.softmax_bf16(xb))
    assert np.array_equal(np.isnan(y), np.isnan(ref))
    assert_rel_close(y[5:], ref[5:], BF16_RTOL, "softmax bf16 special")


@pytest.mark.parametrize("shape", SHAPES)
def test_rmsnorm_f32_and_bf16(shape):
    ops = _ops()
    x = _x(shape, 3)
    g = np.random.default_rng(4).uniform(0.5, 1.5, shape[-1]).astype(np.float32)
    y = ops.rmsnorm(dev(x), dev(g)).cpu().numpy()
    assert_rel_close(y, rowops.rmsnorm(x, g), F32_RTOL, f"rmsnorm f32 {shape}")
    xb, gb = obf.f32_to_bf16_bits(x), obf.f32_to_bf16_bits(g)
    yb = host_bf16(ops.rmsnorm(dev_bf16(xb), dev_bf16(gb)))
    ref = rowops.rmsnorm(obf.bf16_bits_to_f32(xb), obf.bf16_bits_to_f32(gb))
    assert_rel_close(yb, ref, BF16_RTOL, f"rmsnorm bf16 {shape}")


@pytest.mark.parametrize("wave", ["1", "0"])
@pytest.mark.parametrize("shape,seed", [((512, 37), 0), ((300, 1), 0), ((8, 2049), 3), ((64, 300), 5),
                                        ((16, 8192), 6), ((4, 20000), 7), ((33, 1576), 8), ((5, 16384), 9),
                                        ((70, 8), 10)])
def test_argmax_special_values_bit_exact(shape, seed, wave, monkeypatch):
    """Both argmax kernels (one wave per row, and MK_ROW_WAVE=0's workgroup
    per row) against the oracle on rows dense with NaN, +-inf and +-0;
    aligned shapes of up to 16 vectors per lane (32 for bf16: 16384
    columns) take the wave kernel, with a partly filled last vector row at
    1576 columns."""
    monkeypatch.setenv("MK_ROW_WAVE", wave)
    ops = _ops()
    x = _edge(shape, seed)
    got = ops.argmax(dev(x)).cpu().numpy()
    np.testing.assert_array_equal(got, rowops.argmax(x))
    xb = obf.f32_to_bf16_bits(x)
    gotb = ops.argmax(dev_bf16(xb)).cpu().numpy()
    np.testing.assert_array_equal(gotb, rowops.argmax(obf.bf16_bits_to_f32(xb)))


def test_argmax_known_rows():
    ops = _ops()
    x = np.random.default_rng(1).standard_normal((6, 16)).astype(np.float32)
    x[0] = np.nan
    x[1, 5] = np.nan
    x[1, 9] = np.nan
    x[2] = 2.0
    x[3, :4] = [np.inf, np.nan, -np.inf, np.nan]
    x[4, -1] = np.nan
    got = ops.argmax(dev(x)).cpu().numpy()
    assert got[:5].tolist() == [0, 5, 0, 1, 15]
    assert got[5] == int(np.argmax(x[5]))
    z = np.array([[-0.0, 0.0], [0.0, -0.0], [-1.0, -0.0]], np.float32)
    assert ops.argmax(dev(z)).cpu().numpy().tolist() == [0, 0, 1]


def test_argmax_bf16_many_ties():
    """bf16 rounding creates many equal maxima: the first one must win."""
    ops = _ops()
    xb = obf.f32_to_bf16_bits(np.round(_x((64, 8192), 9) * 2) / 2)
    got = ops.argmax(dev_bf16(xb)).cpu().numpy()
    np.testing.assert_array_equal(got, rowops.argmax(obf.bf16_bits_to_f32(xb)))


@pytest.mark.parametrize("shape", SHAPES)
def test_reduce_sum_max(shape):
    ops = _ops()
    x = _x(shape, 11)
    s = ops.reduce_lastdim(dev(x), "sum").cpu().numpy()
    # normwise at the stated f32 1e-5; per row within the f32 summation
    # bound gamma_{n-1} * sum |x|.
    assert_rel_close(s, rowops.reduce_sum(x), F32_RTOL, f"sum {shape}",
                     elem=f32_sum_bound(np.abs(x.astype(np.float64)).sum(axis=-1), shape[-1]))
    m = ops.reduce_lastdim(dev(x), "max").cpu().numpy()
    np.testing.assert_array_equal(m, rowops.reduce_max(x).astype(np.float32))


@pytest.mark.parametrize("wave", ["1", "0"])
@pytest.mark.parametrize("shape,seed", [((64, 300), 12), ((33, 1576), 13), ((16, 8192), 14), ((5, 16384), 15)])
def test_reduce_max_min_special_values(shape, seed, wave, monkeypatch):
    """Row max and min of both kernels on rows dense with NaN, +-inf and
    +-0, exactly (max puts +0 above -0, min -0 below +0)."""
    monkeypatch.setenv("MK_ROW_WAVE", wave)
    ops = _ops()
    x = _edge(shape, seed)
    for xs, host in ((dev(x), x), (dev_bf16(obf.f32_to_bf16_bits(x)), None)):
        ref_in = x if host is not None else obf.bf16_bits_to_f32(obf.f32_to_bf16_bits(x))
        for op, ref in (("max", rowops.reduce_max(ref_in)), ("min", -rowops.reduce_max(-ref_in))):
            got = ops.reduce_lastdim(xs, op)
            got = got.cpu().numpy() if host is not None else obf.bf16_bits_to_f32(host_bf16_bits(got))
            ref = ref.astype(np.float32)
            assert np.array_equal(np.isnan(got), np.isnan(ref)), (op, shape)
            ok = ~np.isnan(ref)
            np.testing.assert_array_equal(got[ok], ref[ok], err_msg=f"{op} {shape}")
            np.testing.assert_array_equal(np.signbit(got[ok]), np.signbit(ref[ok]), err_msg=f"{op} sign {shape}")


def test_reduce_max_nan_and_signed_zero():
    ops = _ops()
    x = np.array([[1.0, np.nan, 2.0], [-0.0, 0.0, -1.0], [-0.0, -0.0, -2.0], [1.0, 2.0, 3.0]], np.float32)
    m = ops.reduce_lastdim(dev(x), "max").cpu().numpy()
    assert np.isnan(m[0])
    assert m[1] == 0 and not np.signbit(m[1])
    assert m[2] == 0 and np.signbit(m[2])
    assert m[3] == 3


@pytest.mark.parametrize("op", ["softmax", "argmax", "sum"])
def test_more_rows_than_one_launch_row_each(op):
    """More rows than the launch gives workgroups (2^20): rows stride over the
    grid, and the last rows are computed like the first."""
    _more_rows(op, (1 << 20) + 37)


def test_argmax_more_rows_than_the_wave_grid():
    """argmax over more rows than the one-wave-per-row launch covers (4 x
    2^20 waves): waves stride over rows, and the last rows are computed like
    the first."""
    _more_rows("argmax", 4 * (1 << 20) + 37)


def _more_rows(op, rows):
    ops = _ops()
    cols = 16
    x = _x((rows, cols), 21)
    print(f"rows case {op} {rows}x{cols}", flush=True)
    xd = dev(x)
    if op == "softmax":
        y = ops.softmax(xd).cpu().numpy()
        assert_rel_close(y, rowops.softmax(x), F32_RTOL, "softmax many rows")
    elif op == "argmax":
        np.testing.assert_array_equal(ops.argmax(xd).cpu().numpy(), rowops.argmax(x))
    else:
        y = ops.reduce_lastdim(xd, "sum").cpu().numpy()
        assert_rel_close(y, rowops.reduce_sum(x), F32_RTOL, "sum many rows",
                         elem=f32_sum_bound(np.abs(x.astype(np.float64)).sum(axis=-1), cols))
