"""End-to-end tests of the plugin runtime on the GPU: StableHLO text of the
workload functions is compiled by the runtime (include/mk_runtime.h),
executed on device buffers through the kernel plan, and checked against
the CPU oracle at the workload's tolerances (integer/index outputs exact,
f32 rel 1e-5, bf16 rel 2e-2).  Also covers the PJRT object semantics the
reference's C-API layer has: buffers own device memory, executions borrow
inputs and return new buffers plus a completion event, error buffers carry
their error (src/pjrt_plugin/api/pjrt_client.cc:254-293, :362-386;
pjrt_executable.cc:245-301; pjrt_buffer.cc:217-247).
"""

import sys
import threading

import numpy as np
import pytest

from mi355x import programs as P
from mi355x import runtime as rt
from oracle import eltwise, gemm, quant, rowops
from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits

from _gpu import BF16_RTOL, F32_RTOL, assert_rel_close

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
    """Compile `text`, execute on `arrays` ((array, type) or array), return host outputs."""
    print(f"[runtime] {text.splitlines()[0]} inputs={[np.shape(a[0] if isinstance(a, tuple) else a) for a in arrays]}",
          flush=True)
    exe = client.compile(text)
    bufs = [client.buffer(*a) if isinstance(a, tuple) else client.buffer(a) for a in arrays]
    outs, done = exe.execute(bufs)
    done.wait()
    res = [o.to_numpy() for o in outs]
    for b in bufs + outs:
        b.close()
    exe.close()
    return res


def bf16(bits):
    return (np.ascontiguousarray(bits, dtype=np.uint16), rt.BF16)


def test_int4_headline_shape(client):
    rng = np.random.default_rng(0)
    M, K, N = 16, 4096, 14336
    x, p, s, z = quant.make_int4_case(rng, M, K, N)
    (y,) = run(client, P.int4_g64_matmul(M, K, N), bf16(x), p, bf16(s), z)
    ref, _ = quant.int4_g64_matmul(x, p, s, z, round_w=False)
    assert y.dtype == np.uint16 and y.shape == (M, N)
    assert_rel_close(bf16_bits_to_f32(y), ref, BF16_RTOL, "int4 runtime")


# 256 rows take the fused many-row kernel, 800 rows dequantise W into the
# executable's workspace and run the bf16 GEMM.
@pytest.mark.parametrize("M,K,N", [(1, 1024, 512), (16, 2048, 1024), (5, 512, 136), (256, 1024, 512),
                                   (800, 512, 384)])
def test_int4_shapes(client, M, K, N):
    rng = np.random.default_rng(M * 7 + N)
    x, p, s, z = quant.make_int4_case(rng, M, K, N)
    (y,) = run(client, P.int4_g64_matmul(M, K, N), bf16(x), p, bf16(s), z)
    ref, _ = quant.int4_g64_matmul(x, p, s, z, round_w=False)
    assert_rel_close(bf16_bits_to_f32(y), ref, BF16_RTOL, f"int4 {M}x{K}x{N}")


@pytest.mark.parametrize("M,K,N", [(16, 4096, 14336), (3, 1024, 520), (256, 1024, 512), (800, 512, 384)])
def test_int8(client, M, K, N):
    rng = np.random.default_rng(1)
    x, w, s = quant.make_int8_case(rng, M, K, N)
    (y,) = run(client, P.int8_pc_matmul(M, K, N), bf16(x), w, s)
    ref, _ = quant.int8_pc_matmul(x, w, s)
    assert_rel_close(bf16_bits_to_f32(y), ref, BF16_RTOL, "int8 runtime")


@pytest.mark.parametrize("M,K,N,batch,pref", [
    (256, 512, 384, None, False), (200, 64, 136, None, True), (128, 64, 256, 4, False), (512, 512, 512, None, False)])
def test_gemm_bf16(client, M, K, N, batch, pref):
    rng = np.random.default_rng(2)
    lead = () if batch is None else (batch,)
    a = f32_to_bf16_bits((rng.standard_normal(lead + (M, K)) / np.sqrt(K)).astype(np.float32))
    b = f32_to_bf16_bits(rng.standard_normal(lead + (K, N)).astype(np.float32))
    (c,) = run(client, P.matmul(M, K, N, batch=batch, preferred_f32=pref), bf16(a), bf16(b))
    ref, _ = gemm.matmul_bf16(a, b, out="f32")
    out = c if pref else bf16_bits_to_f32(c)
    assert c.dtype == (np.float32 if pref else np.uint16)
    assert_rel_close(out, ref, 1e-5 if pref else BF16_RTOL, "gemm bf16 runtime")


def test_gemm_f32(client):
    rng = np.random.default_rng(3)
    a = rng.standard_normal((256, 320)).astype(np.float32)
    b = rng.standard_normal((320, 264)).astype(np.float32)
    (c,) = run(client, P.matmul(256, 320, 264, dt="f32"), a, b)
    assert_rel_close(c, a.astype(np.float64) @ b.astype(np.float64), F32_RTOL, "gemm f32 runtime")


def special_rows(x):
    x = x.copy()
    x[0, 3] = np.nan
    x[1, :] = -np.inf
    x[2, 5] = np.inf
    x[3, :] = 80.0
    return x


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_softmax(client, dt):
    rng = np.random.default_rng(4)
    x = special_rows((rng.standard_normal((64, 1024)) * np.sqrt(2)).astype(np.float32))
    if dt == "f32":
        (y,) = run(client, P.softmax(64, 1024), x)
        assert_rel_close(y, rowops.softmax(x), F32_RTOL, "softmax f32")
    else:
        xb = f32_to_bf16_bits(x)
        (y,) = run(client, P.softmax(64, 1024, "bf16"), bf16(xb))
        ref = bf16_bits_to_f32(rowops.softmax_bf16(xb))
        assert_rel_close(bf16_bits_to_f32(y), ref, BF16_RTOL, "softmax bf16")


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_rmsnorm(client, dt):
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((32, 2048)) * np.sqrt(2)).astype(np.float32)
    g = rng.uniform(0.5, 1.5, 2048).astype(np.float32)
    if dt == "f32":
        (y,) = run(client, P.rmsnorm(32, 2048), x, g)
        assert_rel_close(y, rowops.rmsnorm(x, g), F32_RTOL, "rmsnorm f32")
    else:
        xb, gb = f32_to_bf16_bits(x), f32_to_bf16_bits(g)
        (y,) = run(client, P.rmsnorm(32, 2048, "bf16"), bf16(xb), bf16(gb))
        ref = rowops.rmsnorm(bf16_bits_to_f32(xb), bf16_bits_to_f32(gb))
        assert_rel_close(bf16_bits_to_f32(y), ref, BF16_RTOL, "rmsnorm bf16")


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_argmax_exact(client, dt):
    rng = np.random.default_rng(6)
    x = rng.standard_normal((48, 777)).astype(np.float32)
    x[0, 10] = np.nan
    x[0, 20] = np.nan          # first NaN wins
    x[1, :] = -0.0
    x[1, 5] = 0.0              # -0 == +0: earliest index
    x[2, 100] = x[2, 7] = 50.0  # tie: earliest
    x[3, :] = -np.inf
    if dt == "bf16":
        xb = f32_to_bf16_bits(x)
        (i,) = run(client, P.argmax(48, 777, "bf16"), bf16(xb))
        ref = rowops.argmax(bf16_bits_to_f32(xb))
    else:
        (i,) = run(client, P.argmax(48, 777), x)
        ref = rowops.argmax(x)
    assert i.dtype == np.int32
    np.testing.assert_array_equal(i, ref)
    assert i[0] == 10 and i[1] == 0 and i[2] == 7 and i[3] == 0


@pytest.mark.parametrize("op,dt", [("sum", "f32"), ("max", "f32"), ("sum", "bf16"), ("max", "bf16")])
def test_reduce(client, op, dt):
    rng = np.random.default_rng(7)
    x = rng.standard_normal((40, 3000)).astype(np.float32)
    if dt == "bf16":
        xb = f32_to_bf16_bits(x)
        x = bf16_bits_to_f32(xb)
        (y,) = run(client, P.reduce(40, 3000, op, "bf16"), bf16(xb))
        y = bf16_bits_to_f32(y)
    else:
        (y,) = run(client, P.reduce(40, 3000, op), x)
    if op == "max":
        np.testing.assert_array_equal(y, rowops.reduce_max(x).astype(np.float32))
    else:
        ref = rowops.reduce_sum(x)
        err = np.abs(y - ref) / (np.abs(x).sum(axis=1))  # relative to the sum of magnitudes
        assert err.max() <= (F32_RTOL if dt == "f32" else BF16_RTOL / 2), err.max()


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_chain6(client, dt):
    rng = np.random.default_rng(8)
    x = (rng.standard_normal((64, 4096)) * np.sqrt(2)).astype(np.float32)
    if dt == "bf16":
        xb = f32_to_bf16_bits(x)
        (y,) = run(client, P.chain6(64, 4096, "bf16"), bf16(xb))
        ref = eltwise.evaluate(eltwise.CHAIN6, [bf16_bits_to_f32(xb)], "bf16")
        assert_rel_close(bf16_bits_to_f32(y), ref, BF16_RTOL, "chain6 bf16")
    else:
        (y,) = run(client, P.chain6(64, 4096), x)
        ref = eltwise.evaluate(eltwise.CHAIN6, [x], "f32")
        assert_rel_close(y, ref, F32_RTOL, "chain6 f32")


def test_plumbing_tanh_matmul_sum(client):
    rng = np.random.default_rng(0)
    n = 1024
    a = rng.standard_normal((n, n)).astype(np.float32)
    b = rng.standard_normal((n, n)).astype(np.float32)
    (y,) = run(client, P.plumbing(n), a, b)
    ref = np.tanh(a.astype(np.float64) @ b.astype(np.float64)).sum(axis=1)
    # The stated f32 measure, normwise (max|y - ref| / max|ref| <= 1e-5).
    assert_rel_close(y, ref, F32_RTOL, "plumbing n=1024", elem=False)


# ---- runtime object semantics ------------------------------------------------

@pytest.mark.parametrize("dtype,type_", [(np.float32, None), (np.int32, None), (np.uint8, None), (np.int8, None),
                                         (np.int64, None), (np.float64, None), (np.uint16, rt.BF16)])
def test_buffer_round_trip(client, dtype, type_):
    a = (np.arange(3 * 5 * 7) % 251).astype(dtype).reshape(3, 5, 7)
    b = client.buffer(a, type_) if type_ else client.buffer(a)
    assert b.shape == (3, 5, 7) and b.nbytes == a.nbytes
    np.testing.assert_array_equal(b.to_numpy(), a)
    b.ready_event().wait(1000)
    b.close()


def test_execute_twice_reuses_temporaries(client):
    exe = client.compile(P.plumbing(256))
    rng = np.random.default_rng(9)
    outs = []
    for _ in range(3):
        a = rng.standard_normal((256, 256)).astype(np.float32)
        b = rng.standard_normal((256, 256)).astype(np.float32)
        ba, bb = client.buffer(a), client.buffer(b)
        (o,), done = exe.execute([ba, bb])
        outs.append((o, np.tanh(a.astype(np.float64) @ b).sum(axis=1), ba, bb))
    for o, ref, ba, bb in outs:
        assert_rel_close(o.to_numpy(), ref, F32_RTOL, "plumbing n=256", elem=False)
        for x in (o, ba, bb):
            x.close()
    assert exe.num_steps == 3 and "gemm_f32" in exe.plan
    exe.close()


def test_completion_callback_fires(client):
    exe = client.compile(P.chain6(256, 1024))
    x = client.buffer(np.ones((256, 1024), np.float32))
    (o,), done = exe.execute([x])
    fired = threading.Event()
    errs = []

    def cb(err):
        errs.append(err)
        fired.set()

    done.on_ready(cb)
    assert fired.wait(30)
    assert errs == [None] and done.is_ready()
    ref = eltwise.evaluate(eltwise.CHAIN6, [np.ones((256, 1024), np.float32)], "f32")
    assert_rel_close(o.to_numpy(), ref, F32_RTOL, "chain6 ones")
    for b in (o, x):
        b.close()
    exe.close()


def test_returned_argument_is_an_independent_copy(client):
    text = ("module @m {\n  func.func public @main(%arg0: tensor<8x8xf32>) -> (tensor<8x8xf32>, tensor<8x8xf32>) {\n"
            "    %0 = stablehlo.negate %arg0 : tensor<8x8xf32>\n"
            "    return %arg0, %0 : tensor<8x8xf32>, tensor<8x8xf32>\n  }\n}\n")
    a = np.arange(64, dtype=np.float32).reshape(8, 8)
    x = client.buffer(a)
    exe = client.compile(text)
    (same, neg), done = exe.execute([x])
    x.close()  # the output copy must survive its source
    np.testing.assert_array_equal(same.to_numpy(), a)
    np.testing.assert_array_equal(neg.to_numpy(), -a)
    same.close()
    neg.close()
    exe.close()


def test_error_buffer_propagates(client):
    eb = client.error_buffer(rt.INTERNAL, "upstream failure", rt.F32, (4, 8))
    with pytest.raises(rt.PluginError) as ei:
        eb.to_numpy()
    assert ei.value.code == rt.INTERNAL and "upstream failure" in ei.value.message
    exe = client.compile(P.reduce(4, 8))
    with pytest.raises(rt.PluginError) as ei:
        exe.execute([eb])
    assert ei.value.code == rt.INTERNAL
    eb.close()
    exe.close()


def test_input_type_mismatch_is_invalid_argument(client):
    exe = client.compile(P.reduce(4, 8))
    wrong = client.buffer(np.zeros((4, 9), np.float32))
    with pytest.raises(rt.PluginError) as ei:
        exe.execute([wrong])
    assert ei.value.code == rt.INVALID_ARGUMENT and "tensor<4x9xf32>" in ei.value.message
    with pytest.raises(rt.PluginError):
        exe.execute([])
    wrong.close()
    exe.close()


def test_memory_stats_track_buffers(client):
    used0, limit = client.memory_stats()
    assert limit > 100 * (1 << 30)  # an MI355X has 288 GB of HBM
    b = client.buffer(np.zeros((64, 1 << 20), np.float32))  # 256 MiB
    used1, _ = client.memory_stats()
    assert used1 - used0 >= 256 << 20
    b.close()
    used2, _ = client.memory_stats()
    assert used2 == used0
    assert client.platform_name == "mi355x"


def _reduce_case(rng, shape, specials=True):
    x = (rng.standard_normal(shape) * np.sqrt(2)).astype(np.float32)
    if specials:
        c = shape[-1]
        flat = x.reshape(-1, c)       # rows 0..3 fall in different output rows for every case below
        rows = [0, flat.shape[0] // 3, 2 * flat.shape[0] // 3, flat.shape[0] - 1]
        flat[rows[0], 3 % c] = np.nan  # NaN propagates through min / max / sum
        flat[rows[1], :] = 0.0
        flat[rows[1], 2 % c] = -0.0    # min of a zero row with one -0 is -0, max +0
        flat[rows[2], 5 % c] = np.inf
        flat[rows[3], 6 % c] = -np.inf
    return x


@pytest.mark.parametrize("op", ["min", "max", "sum", "mean"])
@pytest.mark.parametrize("shape,nd", [((64, 48), 1), ((6, 8, 40), 2), ((3, 4, 5, 7), 3)])
def test_reduce_trailing_axes(client, op, shape, nd):
    """jnp.min / max / sum / mean over the trailing axes, f32: min and max
    exact with NaN propagation and -0 < +0; sum and mean at f32 tolerance."""
    rng = np.random.default_rng(len(shape) * 7 + nd)
    x = _reduce_case(rng, shape)
    axes = tuple(range(len(shape) - nd, len(shape)))
    (y,) = run(client, P.reduce_trailing(shape, nd, op), x)
    ref = {"min": np.min, "max": np.max, "sum": np.sum, "mean": np.mean}[op](x.astype(np.float64), axis=axes)
    y = y.reshape(ref.shape)
    assert np.array_equal(np.isnan(y), np.isnan(ref))
    fin = np.isfinite(ref)
    if op in ("min", "max"):
        assert np.array_equal(y[~np.isnan(ref)], ref[~np.isnan(ref)].astype(np.float32))
        # -0 < +0 (StableHLO minimum / maximum; numpy does not order them):
        # a zero minimum is -0 when any zero of the row is -0, a zero
        # maximum is -0 only when every zero of the row is.
        rows = np.moveaxis(x, axes, tuple(range(-nd, 0))).reshape(ref.size, -1)
        neg = np.signbit(rows) & (rows == 0)
        pos = ~np.signbit(rows) & (rows == 0)
        want = neg.any(axis=1) if op == "min" else ~pos.any(axis=1)
        zero = (ref == 0).reshape(-1)
        assert np.array_equal(np.signbit(y.reshape(-1)[zero]), want[zero])
    else:
        assert np.array_equal(y[~fin & ~np.isnan(ref)], ref[~fin & ~np.isnan(ref)])
        assert_rel_close(y[fin], ref[fin], F32_RTOL, f"{op} {shape}")


def test_reduce_min_bf16(client):
    rng = np.random.default_rng(5)
    x = _reduce_case(rng, (32, 64))
    xb = f32_to_bf16_bits(x)
    (y,) = run(client, P.reduce_trailing((32, 64), 1, "min", "bf16"), bf16(xb))
    xf = bf16_bits_to_f32(xb)
    ref = np.min(xf, axis=1)
    yf = bf16_bits_to_f32(y)
    assert np.array_equal(np.isnan(yf), np.isnan(ref))
    ok = ~np.isnan(ref)
    assert np.array_equal(yf[ok], ref[ok])
    zero = ref == 0  # -0 < +0: the zero row holds one -0
    assert np.array_equal(np.signbit(yf[zero]), (np.signbit(xf) & (xf == 0)).any(axis=1)[zero])


@pytest.mark.parametrize("op,init", [("sum", 2.5), ("max", 0.0), ("min", 0.25)])
def test_reduce_non_neutral_init(client, op, init):
    """lax.reduce with an init that is not the body's identity: the init
    joins the reduction once."""
    rng = np.random.default_rng(9)
    x = (rng.standard_normal((16, 40)) * 0.5).astype(np.float32)
    (y,) = run(client, P.reduce_trailing((16, 40), 1, op, "f32", init), x)
    x64 = x.astype(np.float64)
    ref = {"sum": lambda: x64.sum(1) + init, "max": lambda: np.maximum(x64.max(1), init),
           "min": lambda: np.minimum(x64.min(1), init)}[op]()
    if op == "sum":
        assert_rel_close(y, ref, F32_RTOL, "sum init")
    else:
        assert np.array_equal(y, ref.astype(np.float32))
