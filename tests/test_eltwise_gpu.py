"""GPU parity of the fused elementwise kernel (mk_elementwise) against the
oracle's op-by-op evaluation (oracle/eltwise.py), for the workload's 6-op
chain (mul, add, exp, log1p, max, select) in f32 and bf16 (per-op bf16
rounding) and for single ops with special values."""

import numpy as np
import pytest

from _gpu import BF16_RTOL, dev, dev_bf16, host_bf16, host_bf16_bits, need_gpu, torch
from oracle import bf16 as obf
from oracle import eltwise

pytestmark = pytest.mark.gpu

# CHAIN6 as a register program: slots 0 = x; then one slot per step.
CHAIN6_PROGRAM = [
    ("LOAD", 0, 0, 0, 0, 0.0),
    ("CONST", 1, 0, 0, 0, 1.5), ("MUL", 2, 0, 1, 0, 0.0),
    ("CONST", 1, 0, 0, 0, 0.5), ("ADD", 3, 2, 1, 0, 0.0),
    ("EXP", 4, 3, 0, 0, 0.0),
    ("LOG1P", 5, 4, 0, 0, 0.0),
    ("MAX", 6, 5, 0, 0, 0.0),
    ("CONST", 1, 0, 0, 0, 0.0), ("CMP_GT", 7, 0, 1, 0, 0.0),
    ("SELECT", 8, 7, 6, 3, 0.0),
]


def _ops():
    need_gpu()
    from mi355x import ops
    return ops


@pytest.fixture(params=["jit", "interpreter"], autouse=True)
def ew_path(request, monkeypatch):
    """Run every test on both paths: the generated kernel (default) and the
    precompiled interpreter (MK_EW_JIT=0)."""
    if request.param == "interpreter":
        monkeypatch.setenv("MK_EW_JIT", "0")
    else:
        monkeypatch.delenv("MK_EW_JIT", raising=False)
    return request.param


def _close_f32(out, ref, rtol=1e-5):
    out = np.asarray(out, np.float64)
    ref = np.asarray(ref, np.float64)
    assert np.array_equal(np.isnan(out), np.isnan(ref))
    f = ~np.isnan(ref)
    err = np.abs(out[f] - ref[f])
    tol = rtol * np.abs(ref[f]) + 1e-30
    assert np.all(err <= tol), f"max rel {np.max(err / np.maximum(np.abs(ref[f]), 1e-30)):.3e}"


@pytest.mark.parametrize("n", [1, 7, 8, 1000, 4096 * 3 + 5, 1 << 20])
def test_chain6_f32(n):
    ops = _ops()
    x = (np.random.default_rng(n).standard_normal(n) * np.sqrt(2.0)).astype(np.float32)
    y = ops.elementwise(CHAIN6_PROGRAM, [dev(x)], out_slot=8).cpu().numpy()
    ref = eltwise.evaluate(eltwise.CHAIN6, [x], "f32")
    _close_f32(y, ref)


@pytest.mark.parametrize("n", [8, 1000, 1 << 20])
def test_chain6_bf16(n):
    ops = _ops()
    xb = obf.f32_to_bf16_bits((np.random.default_rng(n + 1).standard_normal(n) * np.sqrt(2.0)).astype(np.float32))
    y = host_bf16(ops.elementwise(CHAIN6_PROGRAM, [dev_bf16(xb)], out_slot=8))
    ref = eltwise.evaluate(eltwise.CHAIN6, [obf.bf16_bits_to_f32(xb)], "bf16")
    rel = np.abs(y - ref) / np.maximum(np.abs(ref), 1e-30)
    assert np.max(rel) <= BF16_RTOL, np.max(rel)
    # With the same per-op rounding points, almost every element is bit-equal.
    assert np.mean(y == ref) > 0.98


def test_binary_ops_and_special_values():
    ops = _ops()
    vals = np.array([0.0, -0.0, 1.0, -1.0, 2.5, np.inf, -np.inf, np.nan], np.float32)
    a = np.repeat(vals, len(vals))
    b = np.tile(vals, len(vals))
    for name, ref_fn in [("ADD", np.add), ("SUB", np.subtract), ("MUL", np.multiply),
                         ("MAX", eltwise._max), ("MIN", eltwise._min)]:
        prog = [("LOAD", 0, 0, 0, 0, 0.0), ("LOAD", 1, 1, 0, 0, 0.0), (name, 2, 0, 1, 0, 0.0)]
        y = ops.elementwise(prog, [dev(a), dev(b)], out_slot=2).cpu().numpy()
        with np.errstate(invalid="ignore"):
            ref = ref_fn(a.astype(np.float64), b.astype(np.float64)).astype(np.float32)
        assert np.array_equal(np.isnan(y), np.isnan(ref)), name
        f = ~np.isnan(ref)
        assert np.array_equal(y[f], ref[f]), name
        assert np.array_equal(np.signbit(y[f]), np.signbit(ref[f])), name


def _exp_inputs():
    f = np.finfo(np.float32)
    dense = np.linspace(-104.0, 89.0, 1 << 21).astype(np.float32)
    # Around the overflow threshold ln(FLT_MAX) = 88.7228391 and the
    # denormal range, one ulp at a time.
    hi = np.nextafter(np.float32(88.72283), np.float32(np.inf)) + np.arange(-64, 64, dtype=np.float32) * np.float32(7.62939453125e-06)
    special = np.array([0.0, -0.0, 1e-30, -1e-30, f.tiny, -87.33655, -103.2789, -103.9721,
                        np.inf, -np.inf, np.nan], np.float32)
    return np.concatenate([dense, hi.astype(np.float32), special])


def _log1p_inputs():
    r = np.random.default_rng(7)
    near_m1 = (-1.0 + np.logspace(-7.2, -0.05, 1 << 18)).astype(np.float32)
    mid = np.linspace(-0.99, 2.0, 1 << 20).astype(np.float32)
    tiny = np.logspace(-44, -1, 1 << 18).astype(np.float32)
    big = np.logspace(-1, 38.5, 1 << 18).astype(np.float32)
    rnd = (r.standard_normal(1 << 18) * 0.05).astype(np.float32)
    special = np.array([0.0, -0.0, -1.0, -1.5, 0.0625, -0.0625, np.nextafter(np.float32(0.0625), np.float32(0)),
                        3.4e38, np.inf, -np.inf, np.nan, 1e-45], np.float32)
    return np.concatenate([near_m1, mid, tiny, -tiny[tiny < 0.9], big, rnd, special])


def _ulp_check_f32(y, x, ref64, max_rel):
    """Every result within max_rel of the float64 value rounded to f32
    (denormal results within 2 ulp of the smallest subnormal); infinities,
    NaNs and signed zeros exactly."""
    ref = ref64.astype(np.float32)
    assert np.array_equal(np.isnan(y), np.isnan(ref)), x[np.isnan(y) != np.isnan(ref)][:8]
    f = ~np.isnan(ref)
    y, ref, xs = y[f], ref[f], x[f]
    inf = np.isinf(ref)
    assert np.array_equal(y[inf], ref[inf]), xs[inf][y[inf] != ref[inf]][:8]
    zero = ref == 0
    assert np.array_equal(np.signbit(y[zero & (xs == 0)]), np.signbit(ref[zero & (xs == 0)]))
    fin = ~inf
    err = np.abs(y[fin].astype(np.float64) - ref64[f][fin])
    tol = np.maximum(max_rel * np.abs(ref64[f][fin]), 2.0 * 1.401298464324817e-45)
    bad = err > tol
    assert not bad.any(), (xs[fin][bad][:8], y[fin][bad][:8], ref[fin][bad][:8])


def _logistic64(x):
    return np.where(x >= 0, 1.0 / (1.0 + np.exp(-np.abs(x))), np.exp(-np.abs(x)) / (1.0 + np.exp(-np.abs(x))))


def _logistic_inputs():
    return np.concatenate([np.linspace(-110.0, 110.0, 1 << 20).astype(np.float32),
                           np.array([0.0, -0.0, -80.0, -80.00001, -87.5, -103.0, 17.0, np.inf, -np.inf, np.nan],
                                    np.float32)])


def test_exp_log1p_accuracy_sweep_f32():
    """mk_exp, mk_log1p and mk_logistic against float64 over dense sweeps:
    within 1e-6 relative (8 f32 ulp; the workload's f32 tolerance is 1e-5)."""
    ops = _ops()
    for name, xs, fn in [("EXP", _exp_inputs(), np.exp), ("LOG1P", _log1p_inputs(), np.log1p),
                         ("LOGISTIC", _logistic_inputs(), _logistic64)]:
        prog = [("LOAD", 0, 0, 0, 0, 0.0), (name, 1, 0, 0, 0, 0.0)]
        y = ops.elementwise(prog, [dev(xs)], out_slot=1).cpu().numpy()
        with np.errstate(all="ignore"):
            ref64 = fn(xs.astype(np.float64))
        _ulp_check_f32(y, xs, ref64, 1e-6)


def test_exp_log1p_accuracy_sweep_bf16():
    """bf16 programs: each result is the float64 value rounded to bf16, or a
    neighbour of it when the exact value lies within 2^-14 of a rounding
    midpoint."""
    ops = _ops()
    for name, xs, fn in [("EXP", _exp_inputs(), np.exp), ("LOG1P", _log1p_inputs(), np.log1p),
                         ("LOGISTIC", _logistic_inputs(), _logistic64)]:
        xb = obf.f32_to_bf16_bits(xs)
        xf = obf.bf16_bits_to_f32(xb)
        prog = [("LOAD", 0, 0, 0, 0, 0.0), (name, 1, 0, 0, 0, 0.0)]
        y = host_bf16(ops.elementwise(prog, [dev_bf16(xb)], out_slot=1))
        with np.errstate(all="ignore"):
            ref = obf.bf16_bits_to_f32(obf.f32_to_bf16_bits(fn(xf.astype(np.float64)).astype(np.float32)))
        assert np.array_equal(np.isnan(y), np.isnan(ref))
        f = ~np.isnan(ref) & ~np.isinf(ref)
        assert np.array_equal(y[np.isinf(ref)], ref[np.isinf(ref)])
        rel = np.abs(y[f] - ref[f]) / np.maximum(np.abs(ref[f]), 1e-38)
        assert np.max(rel) <= 2.0 ** -7, np.max(rel)
        assert np.mean(y[f] == ref[f]) > 0.995


def test_scalar_broadcast_input_and_compare_select():
    ops = _ops()
    x = np.linspace(-3, 3, 4097).astype(np.float32)
    thr = np.array([0.25], np.float32)
    prog = [("LOAD", 0, 0, 0, 0, 0.0), ("LOAD", 1, 1, 0, 0, 0.0), ("CMP_GE", 2, 0, 1, 0, 0.0),
            ("NEG", 3, 0, 0, 0, 0.0), ("SELECT", 4, 2, 0, 3, 0.0)]
    y = ops.elementwise(prog, [dev(x), dev(thr)], out_slot=4).cpu().numpy()
    np.testing.assert_array_equal(y, np.where(x >= 0.25, x, -x))


def test_invalid_program_rejected_on_host():
    ops = _ops()
    from mi355x._lib import MKError
    x = dev(np.ones(16, np.float32))
    with pytest.raises(MKError):
        ops.elementwise([("ADD", 0, 1, 2, 0, 0.0)], [x], out_slot=0)  # reads undefined slots
    with pytest.raises(MKError):
        ops.elementwise([("LOAD", 0, 3, 0, 0, 0.0)], [x], out_slot=0)  # no input 3
