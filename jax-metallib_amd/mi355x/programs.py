"""StableHLO text of the workload's jitted functions.

Each function returns the module text that ``jax.jit(f).lower(*args).as_text()``
prints for the jnp function in its docstring (pretty-printed StableHLO, the
form jax's MLIR printer emits).  The plugin's compile path reads this text;
these builders give the exact programs at any shape, for tests and the
benchmark, without jax installed.

The quantized formats are this plugin's (the reference's quantized matmul is
not jittable, src/jax_metallib/quantized.py:1077-1152):
  int4 g64: X bf16 [M, K]; P uint8 [K/2, N], element k of column n in byte
            P[k // 2, n], low nibble for even k (the reference's nibble order,
            quantized.py:189-190); scale bf16 [K/64, N]; zero uint8 [K/64, N]
            (values 0..15); Y = X @ ((q - z) * s) as bf16.
  int8 per-channel: W int8 [K, N], scale f32 [N]; Y = X @ (W * s) as bf16.
"""

_HEADER = ('module @{name} attributes {{mhlo.num_partitions = 1 : i32, mhlo.num_replicas = 1 : i32}} {{\n'
           '  func.func public @main({args}) -> ({rets}) {{\n')
_FOOTER = '  }\n}\n'


def _t(shape, dt):
    return "tensor<" + "".join(f"{d}x" for d in shape) + dt + ">"


def _module(name, args, rets, body):
    a = ", ".join(f"%arg{i}: {t}" for i, t in enumerate(args))
    r = ", ".join(f'{t} {{jax.result_info = "{"" if len(rets) == 1 else f"[{i}]"}"}}'
                  for i, t in enumerate(rets))
    lines = "".join(f"    {l}\n" for l in body)
    return _HEADER.format(name=name, args=a, rets=r) + lines + _FOOTER


_NEG_INF = {"f32": "0xFF800000", "bf16": "0xFF80"}


def matmul(M, K, N, dt="bf16", batch=None, preferred_f32=False):
    """jnp.matmul(a, b) (a [batch.., M, K], b [batch.., K, N]);
    preferred_f32: jnp.matmul(a, b, preferred_element_type=jnp.float32)."""
    bd = [] if batch is None else [batch]
    ta, tb = _t(bd + [M, K], dt), _t(bd + [K, N], dt)
    odt = "f32" if preferred_f32 else dt
    tc = _t(bd + [M, N], odt)
    dims = ("batching_dims = [0] x [0], contracting_dims = [2] x [1]" if batch is not None
            else "contracting_dims = [1] x [0]")
    body = [f"%0 = stablehlo.dot_general %arg0, %arg1, {dims}, precision = [DEFAULT, DEFAULT] : "
            f"({ta}, {tb}) -> {tc}", f"return %0 : {tc}"]
    return _module("jit_matmul", [ta, tb], [tc], body)


_MLIR_DT = {"int8": "i8", "uint8": "ui8", "int16": "i16", "uint16": "ui16", "int32": "i32", "uint32": "ui32",
            "int64": "i64", "uint64": "ui64", "float16": "f16", "float32": "f32", "bfloat16": "bf16"}


def dot_general(shape_a, shape_b, dt, out_dt=None, batch=0, contract=(None, None), transpose_b=None,
                self_transpose=False):
    """One stablehlo.dot_general as jax.jit(...).lower().as_text() prints it:
    batch leading batching dims on both sides, contracting dims `contract`
    (default: last of a, first non-batch of b).  transpose_b = a
    permutation applied to b by a stablehlo.transpose first (the operand
    is then the transpose's result); self_transpose: b is the transpose of
    argument 0 (a @ a.T, one argument).  dt / out_dt are numpy dtype names."""
    t = _MLIR_DT[dt]
    to = _MLIR_DT[out_dt or dt]
    ta = _t(shape_a, t)
    tb0 = _t(shape_b, t) if shape_b is not None else None
    lc = contract[0] if contract[0] is not None else len(shape_a) - 1
    body, args = [], [ta] if self_transpose else [ta, tb0]
    bname = "%arg1"
    b_shape = list(shape_b) if shape_b is not None else None
    if self_transpose:
        perm = list(range(len(shape_a)))
        perm[-1], perm[-2] = perm[-2], perm[-1]
        b_shape = [shape_a[p] for p in perm]
        body.append(f"%0 = stablehlo.transpose %arg0, dims = [{', '.join(map(str, perm))}] : ({ta}) -> {_t(b_shape, t)}")
        bname = "%0"
    elif transpose_b is not None:
        b_shape = [shape_b[p] for p in transpose_b]
        body.append(f"%0 = stablehlo.transpose %arg1, dims = [{', '.join(map(str, transpose_b))}] : ({tb0}) -> "
                    f"{_t(b_shape, t)}")
        bname = "%0"
    rc = contract[1] if contract[1] is not None else batch
    a_free = [shape_a[i] for i in range(batch, len(shape_a)) if i != lc]
    b_free = [b_shape[i] for i in range(batch, len(b_shape)) if i != rc]
    out_shape = list(shape_a[:batch]) + a_free + b_free
    tc = _t(out_shape, to)
    dims = []
    if batch:
        bl = ", ".join(str(i) for i in range(batch))
        dims.append(f"batching_dims = [{bl}] x [{bl}]")
    dims.append(f"contracting_dims = [{lc}] x [{rc}]")
    res = "%1" if body else "%0"
    body.append(f"{res} = stablehlo.dot_general %arg0, {bname}, {', '.join(dims)}, precision = [DEFAULT, DEFAULT] : "
                f"({ta}, {_t(b_shape, t)}) -> {tc}")
    body.append(f"return {res} : {tc}")
    return _module("jit_dot", args, [tc], body)


def dot_general_dims(shape_a, shape_b, dt, lc, rc, lb=(), rb=(), out_dt=None):
    """lax.dot_general(a, b, ((lc, rc), (lb, rb))) with any dimension numbers
    (several contracting dims, none, batch dims anywhere), as jax.jit
    lowers it: the result is [batch (in lb order), lhs free, rhs free]."""
    t, to = _MLIR_DT[dt], _MLIR_DT[out_dt or dt]
    ta, tb = _t(shape_a, t), _t(shape_b, t)
    a_free = [shape_a[i] for i in range(len(shape_a)) if i not in lc and i not in lb]
    b_free = [shape_b[i] for i in range(len(shape_b)) if i not in rc and i not in rb]
    tc = _t([shape_a[i] for i in lb] + a_free + b_free, to)
    dims = []
    if lb:
        dims.append(f"batching_dims = [{', '.join(map(str, lb))}] x [{', '.join(map(str, rb))}]")
    dims.append(f"contracting_dims = [{', '.join(map(str, lc))}] x [{', '.join(map(str, rc))}]")
    body = [f"%0 = stablehlo.dot_general %arg0, %arg1, {', '.join(dims)}, precision = [DEFAULT, DEFAULT] : "
            f"({ta}, {tb}) -> {tc}", f"return %0 : {tc}"]
    return _module("jit_dot_general", [ta, tb], [tc], body)


def softmax(R, C, dt="f32"):
    """jax.nn.softmax(x, axis=-1) on x [R, C]."""
    tx, tr, tr1 = _t([R, C], dt), _t([R], dt), _t([R, 1], dt)
    s = _t([], dt)
    body = [
        f"%cst = stablehlo.constant dense<{_NEG_INF[dt]}> : {s}",
        f"%0 = stablehlo.reduce(%arg0 init: %cst) applies stablehlo.maximum across dimensions = [1] : "
        f"({tx}, {s}) -> {tr}",
        f"%cst_0 = stablehlo.constant dense<{_NEG_INF[dt]}> : {s}",
        f"%1 = stablehlo.broadcast_in_dim %cst_0, dims = [] : ({s}) -> {tr}",
        f"%2 = stablehlo.maximum %1, %0 : {tr}",
        f"%3 = stablehlo.broadcast_in_dim %2, dims = [0] : ({tr}) -> {tr1}",
        f"%4 = stablehlo.broadcast_in_dim %3, dims = [0, 1] : ({tr1}) -> {tx}",
        f"%5 = stablehlo.subtract %arg0, %4 : {tx}",
        f"%6 = stablehlo.exponential %5 : {tx}",
    ]
    if dt == "bf16":
        # jnp.sum upcasts bf16 to f32 for the reduction.
        txf, trf = _t([R, C], "f32"), _t([R], "f32")
        body += [
            f"%7 = stablehlo.convert %6 : ({tx}) -> {txf}",
            "%cst_1 = stablehlo.constant dense<0.000000e+00> : tensor<f32>",
            f"%8 = stablehlo.reduce(%7 init: %cst_1) applies stablehlo.add across dimensions = [1] : "
            f"({txf}, tensor<f32>) -> {trf}",
            f"%9 = stablehlo.convert %8 : ({trf}) -> {tr}",
        ]
    else:
        body += [
            "%cst_1 = stablehlo.constant dense<0.000000e+00> : tensor<f32>",
            f"%9 = stablehlo.reduce(%6 init: %cst_1) applies stablehlo.add across dimensions = [1] : "
            f"({tx}, tensor<f32>) -> {tr}",
        ]
    body += [
        f"%10 = stablehlo.broadcast_in_dim %9, dims = [0] : ({tr}) -> {tr1}",
        f"%11 = stablehlo.broadcast_in_dim %10, dims = [0, 1] : ({tr1}) -> {tx}",
        f"%12 = stablehlo.divide %6, %11 : {tx}",
        f"return %12 : {tx}",
    ]
    return _module("jit_softmax", [tx], [tx], body)


def rmsnorm(R, C, dt="f32", eps="9.99999997E-7"):
    """x * jax.lax.rsqrt(jnp.mean(x * x, axis=-1, keepdims=True) + 1e-6) * g
    on x [R, C], g [C]."""
    tx, tg, tr, tr1 = _t([R, C], dt), _t([C], dt), _t([R], "f32"), _t([R, 1], "f32")
    tr1d, t1c = _t([R, 1], dt), _t([1, C], dt)
    body = [f"%0 = stablehlo.multiply %arg0, %arg0 : {tx}"]
    src = "%0"
    if dt == "bf16":
        body.append(f"%c0 = stablehlo.convert %0 : ({tx}) -> {_t([R, C], 'f32')}")
        src = "%c0"
    body += [
        "%cst = stablehlo.constant dense<0.000000e+00> : tensor<f32>",
        f"%1 = stablehlo.reduce({src} init: %cst) applies stablehlo.add across dimensions = [1] : "
        f"({_t([R, C], 'f32')}, tensor<f32>) -> {tr}",
        f"%2 = stablehlo.broadcast_in_dim %1, dims = [0] : ({tr}) -> {tr1}",
        f"%cst_0 = stablehlo.constant dense<{float(C):.6e}> : tensor<f32>",
        f"%3 = stablehlo.broadcast_in_dim %cst_0, dims = [] : (tensor<f32>) -> {tr1}",
        f"%4 = stablehlo.divide %2, %3 : {tr1}",
    ]
    m = "%4"
    if dt == "bf16":
        body.append(f"%c4 = stablehlo.convert %4 : ({tr1}) -> {tr1d}")
        m = "%c4"
    body += [
        f"%cst_1 = stablehlo.constant dense<{eps}> : {_t([], dt)}",
        f"%5 = stablehlo.broadcast_in_dim %cst_1, dims = [] : ({_t([], dt)}) -> {tr1d}",
        f"%6 = stablehlo.add {m}, %5 : {tr1d}",
        f"%7 = stablehlo.rsqrt %6 : {tr1d}",
        f"%8 = stablehlo.broadcast_in_dim %7, dims = [0, 1] : ({tr1d}) -> {tx}",
        f"%9 = stablehlo.multiply %arg0, %8 : {tx}",
        f"%10 = stablehlo.broadcast_in_dim %arg1, dims = [1] : ({tg}) -> {t1c}",
        f"%11 = stablehlo.broadcast_in_dim %10, dims = [0, 1] : ({t1c}) -> {tx}",
        f"%12 = stablehlo.multiply %9, %11 : {tx}",
        f"return %12 : {tx}",
    ]
    return _module("jit_rmsnorm", [tx, tg], [tx], body)


def argmax(R, C, dt="f32"):
    """jnp.argmax(x, axis=-1) on x [R, C] -> int32 [R]."""
    tx, ti, tr, tri = _t([R, C], dt), _t([R, C], "i32"), _t([R], dt), _t([R], "i32")
    s = _t([], dt)
    body = [
        f"%0 = stablehlo.iota dim = 1 : {ti}",
        f"%cst = stablehlo.constant dense<{_NEG_INF[dt]}> : {s}",
        "%c = stablehlo.constant dense<0> : tensor<i32>",
        f"%1:2 = stablehlo.reduce(%arg0 init: %cst), (%0 init: %c) across dimensions = [1] : "
        f"({tx}, {ti}, {s}, tensor<i32>) -> ({tr}, {tri})",
        f" reducer(%arg1: {s}, %arg3: {s}) (%arg2: tensor<i32>, %arg4: tensor<i32>)  {{",
        f"  %2 = stablehlo.compare  GT, %arg1, %arg3,  FLOAT : ({s}, {s}) -> tensor<i1>",
        f"  %3 = stablehlo.compare  NE, %arg1, %arg1,  FLOAT : ({s}, {s}) -> tensor<i1>",
        "  %4 = stablehlo.or %2, %3 : tensor<i1>",
        f"  %5 = stablehlo.compare  EQ, %arg1, %arg3,  FLOAT : ({s}, {s}) -> tensor<i1>",
        "  %6 = stablehlo.compare  LT, %arg2, %arg4,  SIGNED : (tensor<i32>, tensor<i32>) -> tensor<i1>",
        "  %7 = stablehlo.and %5, %6 : tensor<i1>",
        "  %8 = stablehlo.or %4, %7 : tensor<i1>",
        f"  %9 = stablehlo.select %4, %arg1, %arg3 : tensor<i1>, {s}",
        "  %10 = stablehlo.select %8, %arg2, %arg4 : tensor<i1>, tensor<i32>",
        f"  stablehlo.return %9, %10 : {s}, tensor<i32>",
        "}",
        f"return %1#1 : {tri}",
    ]
    return _module("jit_argmax", [tx], [tri], body)


def reduce(R, C, op="sum", dt="f32"):
    """jnp.sum(x, axis=-1) / jnp.max(x, axis=-1) on x [R, C]."""
    tx, tr = _t([R, C], dt), _t([R], dt)
    if op == "max":
        body = [f"%cst = stablehlo.constant dense<{_NEG_INF[dt]}> : {_t([], dt)}",
                f"%0 = stablehlo.reduce(%arg0 init: %cst) applies stablehlo.maximum across dimensions = [1] : "
                f"({tx}, {_t([], dt)}) -> {tr}",
                f"return %0 : {tr}"]
    elif dt == "bf16":
        txf, trf = _t([R, C], "f32"), _t([R], "f32")
        body = [f"%0 = stablehlo.convert %arg0 : ({tx}) -> {txf}",
                "%cst = stablehlo.constant dense<0.000000e+00> : tensor<f32>",
                f"%1 = stablehlo.reduce(%0 init: %cst) applies stablehlo.add across dimensions = [1] : "
                f"({txf}, tensor<f32>) -> {trf}",
                f"%2 = stablehlo.convert %1 : ({trf}) -> {tr}",
                f"return %2 : {tr}"]
    else:
        body = ["%cst = stablehlo.constant dense<0.000000e+00> : tensor<f32>",
                f"%0 = stablehlo.reduce(%arg0 init: %cst) applies stablehlo.add across dimensions = [1] : "
                f"({tx}, tensor<f32>) -> {tr}",
                f"return %0 : {tr}"]
    return _module(f"jit_{op}", [tx], [tr], body)


_POS_INF = {"f32": "0x7F800000", "bf16": "0x7F80"}


def reduce_trailing(shape, ndims, op="sum", dt="f32", init=None):
    """jnp.sum / jnp.max / jnp.min / jnp.mean of x over its last `ndims`
    axes (op "sum" / "max" / "min" / "mean"), or, with `init`, lax.reduce
    with that init value and the op's body (add / max / min).  f32 only for
    "mean" (jnp.mean of f32 divides the f32 sum by the count)."""
    rank = len(shape)
    dims = list(range(rank - ndims, rank))
    out = list(shape[:rank - ndims])
    tx, tr, ts = _t(shape, dt), _t(out, dt), _t([], dt)
    body_op = {"sum": "add", "mean": "add", "max": "maximum", "min": "minimum"}[op]
    if init is not None:
        cst = f"{float(init):.6e}"
    elif op in ("sum", "mean"):
        cst = "0.000000e+00"
    else:
        cst = (_NEG_INF if op == "max" else _POS_INF)[dt]
    body = [f"%cst = stablehlo.constant dense<{cst}> : {ts}",
            f"%0 = stablehlo.reduce(%arg0 init: %cst) applies stablehlo.{body_op} across dimensions = "
            f"[{', '.join(map(str, dims))}] : ({tx}, {ts}) -> {tr}"]
    res = "%0"
    if op == "mean":
        count = 1
        for d in dims:
            count *= shape[d]
        body += [f"%cst_0 = stablehlo.constant dense<{float(count):.6e}> : {ts}",
                 f"%1 = stablehlo.broadcast_in_dim %cst_0, dims = [] : ({ts}) -> {tr}",
                 f"%2 = stablehlo.divide %0, %1 : {tr}"]
        res = "%2"
    body.append(f"return {res} : {tr}")
    return _module(f"jit_{op}", [tx], [tr], body)


def chain6(R, C, dt="f32"):
    """The workload's 6-op chain on x [R, C]:
    a = x * 1.5; b = a + 0.5; y = jnp.where(x > 0, jnp.maximum(jnp.log1p(jnp.exp(b)), x), b)."""
    tx, tp, s = _t([R, C], dt), _t([R, C], "i1"), _t([], dt)
    body = [
        f"%cst = stablehlo.constant dense<1.500000e+00> : {s}",
        f"%0 = stablehlo.broadcast_in_dim %cst, dims = [] : ({s}) -> {tx}",
        f"%1 = stablehlo.multiply %arg0, %0 : {tx}",
        f"%cst_0 = stablehlo.constant dense<5.000000e-01> : {s}",
        f"%2 = stablehlo.broadcast_in_dim %cst_0, dims = [] : ({s}) -> {tx}",
        f"%3 = stablehlo.add %1, %2 : {tx}",
        f"%4 = stablehlo.exponential %3 : {tx}",
        f"%5 = stablehlo.log_plus_one %4 : {tx}",
        f"%6 = stablehlo.maximum %5, %arg0 : {tx}",
        f"%cst_1 = stablehlo.constant dense<0.000000e+00> : {s}",
        f"%7 = stablehlo.broadcast_in_dim %cst_1, dims = [] : ({s}) -> {tx}",
        f"%8 = stablehlo.compare  GT, %arg0, %7,  FLOAT : ({tx}, {tx}) -> {tp}",
        f"%9 = stablehlo.select %8, %6, %3 : {tp}, {tx}",
        f"return %9 : {tx}",
    ]
    return _module("jit_chain6", [tx], [tx], body)


def int4_g64_matmul(M, K, N):
    """def f(x, p, s, z):
           q = jnp.stack([p & 15, p >> 4], axis=1).reshape(K, N)
           w = (q.astype(f32) - jnp.repeat(z, 64, 0).astype(f32)) * jnp.repeat(s, 64, 0).astype(f32)
           return jnp.dot(x.astype(f32), w).astype(bf16)"""
    G = K // 64
    tx, tp, ts, tz = _t([M, K], "bf16"), _t([K // 2, N], "ui8"), _t([G, N], "bf16"), _t([G, N], "ui8")
    tp3, tc = _t([K // 2, 1, N], "ui8"), _t([K // 2, 2, N], "ui8")
    tq, tqf = _t([K, N], "ui8"), _t([K, N], "f32")
    tz3, tzb, ts3, tsb = _t([G, 1, N], "ui8"), _t([G, 64, N], "ui8"), _t([G, 1, N], "bf16"), _t([G, 64, N], "bf16")
    tsk, txf, ty, tyf = _t([K, N], "bf16"), _t([M, K], "f32"), _t([M, N], "bf16"), _t([M, N], "f32")
    body = [
        "%c = stablehlo.constant dense<15> : tensor<ui8>",
        f"%0 = stablehlo.broadcast_in_dim %c, dims = [] : (tensor<ui8>) -> {tp}",
        f"%1 = stablehlo.and %arg1, %0 : {tp}",
        "%c_0 = stablehlo.constant dense<4> : tensor<ui8>",
        f"%2 = stablehlo.broadcast_in_dim %c_0, dims = [] : (tensor<ui8>) -> {tp}",
        f"%3 = stablehlo.shift_right_logical %arg1, %2 : {tp}",
        f"%4 = stablehlo.broadcast_in_dim %1, dims = [0, 2] : ({tp}) -> {tp3}",
        f"%5 = stablehlo.broadcast_in_dim %3, dims = [0, 2] : ({tp}) -> {tp3}",
        f"%6 = stablehlo.concatenate %4, %5, dim = 1 : ({tp3}, {tp3}) -> {tc}",
        f"%7 = stablehlo.reshape %6 : ({tc}) -> {tq}",
        f"%8 = stablehlo.reshape %arg3 : ({tz}) -> {tz3}",
        f"%9 = stablehlo.broadcast_in_dim %8, dims = [0, 1, 2] : ({tz3}) -> {tzb}",
        f"%10 = stablehlo.reshape %9 : ({tzb}) -> {tq}",
        f"%11 = stablehlo.reshape %arg2 : ({ts}) -> {ts3}",
        f"%12 = stablehlo.broadcast_in_dim %11, dims = [0, 1, 2] : ({ts3}) -> {tsb}",
        f"%13 = stablehlo.reshape %12 : ({tsb}) -> {tsk}",
        f"%14 = stablehlo.convert %7 : ({tq}) -> {tqf}",
        f"%15 = stablehlo.convert %10 : ({tq}) -> {tqf}",
        f"%16 = stablehlo.subtract %14, %15 : {tqf}",
        f"%17 = stablehlo.convert %13 : ({tsk}) -> {tqf}",
        f"%18 = stablehlo.multiply %16, %17 : {tqf}",
        f"%19 = stablehlo.convert %arg0 : ({tx}) -> {txf}",
        f"%20 = stablehlo.dot_general %19, %18, contracting_dims = [1] x [0], precision = [DEFAULT, DEFAULT] : "
        f"({txf}, {tqf}) -> {tyf}",
        f"%21 = stablehlo.convert %20 : ({tyf}) -> {ty}",
        f"return %21 : {ty}",
    ]
    return _module("jit_int4_g64_matmul", [tx, tp, ts, tz], [ty], body)


def int8_pc_matmul(M, K, N):
    """def f(x, w, s):
           return jnp.dot(x.astype(f32), w.astype(f32) * s[None, :]).astype(bf16)"""
    tx, tw, ts = _t([M, K], "bf16"), _t([K, N], "i8"), _t([N], "f32")
    twf, t1n, txf, ty, tyf = _t([K, N], "f32"), _t([1, N], "f32"), _t([M, K], "f32"), _t([M, N], "bf16"), _t([M, N], "f32")
    body = [
        f"%0 = stablehlo.convert %arg1 : ({tw}) -> {twf}",
        f"%1 = stablehlo.broadcast_in_dim %arg2, dims = [1] : ({ts}) -> {t1n}",
        f"%2 = stablehlo.broadcast_in_dim %1, dims = [0, 1] : ({t1n}) -> {twf}",
        f"%3 = stablehlo.multiply %0, %2 : {twf}",
        f"%4 = stablehlo.convert %arg0 : ({tx}) -> {txf}",
        f"%5 = stablehlo.dot_general %4, %3, contracting_dims = [1] x [0], precision = [DEFAULT, DEFAULT] : "
        f"({txf}, {twf}) -> {tyf}",
        f"%6 = stablehlo.convert %5 : ({tyf}) -> {ty}",
        f"return %6 : {ty}",
    ]
    return _module("jit_int8_pc_matmul", [tx, tw, ts], [ty], body)


def qmm_epilogue(M, K, N, fmt="int4", op="add"):
    """def f(aux, x, *w):  # aux bf16 [M, N]; (x, *w) as int4_g64_matmul / int8_pc_matmul
           y = qmm(x, *w)
           return aux + y                              # op "add"
           return aux * jax.nn.sigmoid(aux) * y        # op "swiglu" (silu(aux) * y)"""
    t = int4_g64_matmul(M, K, N) if fmt == "int4" else int8_pc_matmul(M, K, N)
    ty = _t([M, N], "bf16")
    last = "%21" if fmt == "int4" else "%6"
    t = t.replace("func.func public @main(", f"func.func public @main(%aux: {ty}, ", 1)
    if op == "add":
        body = f"    %e0 = stablehlo.add %aux, {last} : {ty}\n    return %e0 : {ty}"
    else:
        body = (f"    %e0 = stablehlo.logistic %aux : {ty}\n    %e1 = stablehlo.multiply %aux, %e0 : {ty}\n"
                f"    %e2 = stablehlo.multiply %e1, {last} : {ty}\n    return %e2 : {ty}")
    return t.replace(f"    return {last} : {ty}", body)


def plumbing(n=1024):
    """jnp.tanh(a @ b).sum(axis=1) on f32 [n, n]."""
    t, tr = _t([n, n], "f32"), _t([n], "f32")
    body = [
        f"%0 = stablehlo.dot_general %arg0, %arg1, contracting_dims = [1] x [0], precision = [DEFAULT, DEFAULT] : "
        f"({t}, {t}) -> {t}",
        f"%1 = stablehlo.tanh %0 : {t}",
        "%cst = stablehlo.constant dense<0.000000e+00> : tensor<f32>",
        f"%2 = stablehlo.reduce(%1 init: %cst) applies stablehlo.add across dimensions = [1] : "
        f"({t}, tensor<f32>) -> {tr}",
        f"return %2 : {tr}",
    ]
    return _module("jit_plumbing", [t, t], [tr], body)


class _Body:
    """SSA body builder: each call appends `%<n> = <rhs>` and returns %<n>."""

    def __init__(self):
        self.lines = []

    def __call__(self, rhs):
        name = f"%{len(self.lines)}"
        self.lines.append(f"{name} = {rhs}")
        return name

    def const(self, value, dt):
        return self(f"stablehlo.constant dense<{value}> : {_t([], dt)}")

    def bcast(self, x, tx, dims, ty):
        return self(f"stablehlo.broadcast_in_dim {x}, dims = [{', '.join(map(str, dims))}] : ({tx}) -> {ty}")

    def splat(self, value, dt, shape):
        return self.bcast(self.const(value, dt), _t([], dt), [], _t(shape, dt))

    def bin(self, op, a, b, t):
        return self(f"stablehlo.{op} {a}, {b} : {t}")

    def un(self, op, a, t):
        return self(f"stablehlo.{op} {a} : {t}")

    def cvt(self, x, tx, ty):
        return self(f"stablehlo.convert {x} : ({tx}) -> {ty}")

    def reshape(self, x, tx, ty):
        return self(f"stablehlo.reshape {x} : ({tx}) -> {ty}")

    def transpose(self, x, tx, perm, ty):
        return self(f"stablehlo.transpose {x}, dims = [{', '.join(map(str, perm))}] : ({tx}) -> {ty}")

    def slice(self, x, tx, ranges, ty):
        return self(f"stablehlo.slice {x} [{', '.join(f'{a}:{b}' for a, b in ranges)}] : ({tx}) -> {ty}")

    def reduce(self, x, tx, init, ts, op, dims, tr):
        return self(f"stablehlo.reduce({x} init: {init}) applies stablehlo.{op} across dimensions = "
                    f"[{', '.join(map(str, dims))}] : ({tx}, {ts}) -> {tr}")


def _rmsnorm_bf16(e, x, g, R, C, eps):
    """x * rsqrt(mean(x * x, -1, keepdims=True) + eps) * g on bf16 x [R, C]
    (jnp.mean sums in f32 and divides there)."""
    tx, txf, tr, tr1, tr1b = _t([R, C], "bf16"), _t([R, C], "f32"), _t([R], "f32"), _t([R, 1], "f32"), _t([R, 1], "bf16")
    sq = e.cvt(e.bin("multiply", x, x, tx), tx, txf)
    ss = e.reduce(sq, txf, e.const("0.000000e+00", "f32"), "tensor<f32>", "add", [1], tr)
    mean = e.bin("divide", e.bcast(ss, tr, [0], tr1), e.splat(f"{float(C):.6e}", "f32", [R, 1]), tr1)
    r = e.un("rsqrt", e.bin("add", e.cvt(mean, tr1, tr1b), e.splat(eps, "bf16", [R, 1]), tr1b), tr1b)
    xr = e.bin("multiply", x, e.bcast(r, tr1b, [0, 1], tx), tx)
    gb = e.bcast(e.bcast(g, _t([C], "bf16"), [1], _t([1, C], "bf16")), _t([1, C], "bf16"), [0, 1], tx)
    return e.bin("multiply", xr, gb, tx)


def _int4_mm(e, x, p, s, z, M, K, N):
    """x @ ((q - z) * s) as bf16 for the int4 g64 weight (p, s, z), written
    like int4_g64_matmul's function."""
    G = K // 64
    tp, ts, tz = _t([K // 2, N], "ui8"), _t([G, N], "bf16"), _t([G, N], "ui8")
    tp3, tc, tq, tqf = _t([K // 2, 1, N], "ui8"), _t([K // 2, 2, N], "ui8"), _t([K, N], "ui8"), _t([K, N], "f32")
    lo = e.bin("and", p, e.splat("15", "ui8", [K // 2, N]), tp)
    hi = e.bin("shift_right_logical", p, e.splat("4", "ui8", [K // 2, N]), tp)
    cat = e(f"stablehlo.concatenate {e.bcast(lo, tp, [0, 2], tp3)}, {e.bcast(hi, tp, [0, 2], tp3)}, dim = 1 : "
            f"({tp3}, {tp3}) -> {tc}")
    q = e.reshape(cat, tc, tq)
    zr = e.reshape(e.bcast(e.reshape(z, tz, _t([G, 1, N], "ui8")), _t([G, 1, N], "ui8"), [0, 1, 2],
                           _t([G, 64, N], "ui8")), _t([G, 64, N], "ui8"), tq)
    sr = e.reshape(e.bcast(e.reshape(s, ts, _t([G, 1, N], "bf16")), _t([G, 1, N], "bf16"), [0, 1, 2],
                           _t([G, 64, N], "bf16")), _t([G, 64, N], "bf16"), _t([K, N], "bf16"))
    w = e.bin("multiply", e.bin("subtract", e.cvt(q, tq, tqf), e.cvt(zr, tq, tqf), tqf),
              e.cvt(sr, _t([K, N], "bf16"), tqf), tqf)
    xf = e.cvt(x, _t([M, K], "bf16"), _t([M, K], "f32"))
    y = e(f"stablehlo.dot_general {xf}, {w}, contracting_dims = [1] x [0], precision = [DEFAULT, DEFAULT] : "
          f"({_t([M, K], 'f32')}, {tqf}) -> {_t([M, N], 'f32')}")
    return e.cvt(y, _t([M, N], "f32"), _t([M, N], "bf16"))


def _int8_mm(e, x, w, s, M, K, N):
    """x @ (w * s[None, :]) as bf16 for the int8 per-channel weight (w, s),
    written like int8_pc_matmul's function."""
    tw, twf, t1n = _t([K, N], "i8"), _t([K, N], "f32"), _t([1, N], "f32")
    wf = e.bin("multiply", e.cvt(w, tw, twf), e.bcast(e.bcast(s, _t([N], "f32"), [1], t1n), t1n, [0, 1], twf), twf)
    xf = e.cvt(x, _t([M, K], "bf16"), _t([M, K], "f32"))
    y = e(f"stablehlo.dot_general {xf}, {wf}, contracting_dims = [1] x [0], precision = [DEFAULT, DEFAULT] : "
          f"({_t([M, K], 'f32')}, {twf}) -> {_t([M, N], 'f32')}")
    return e.cvt(y, _t([M, N], "f32"), _t([M, N], "bf16"))


def swiglu_mlp(M, K, N, fmt="int4"):
    """The decoder's gated projection pair on its own:

        def f(x, *wg, *wu):  # x bf16 [M, K]; wg, wu as int4_g64_matmul / int8_pc_matmul
            return jax.nn.silu(qmm(x, *wg)) * qmm(x, *wu)"""
    e = _Body()
    ty = _t([M, N], "bf16")
    if fmt == "int4":
        G = K // 64
        wt = [_t([K // 2, N], "ui8"), _t([G, N], "bf16"), _t([G, N], "ui8")]
        g = _int4_mm(e, "%arg0", "%arg1", "%arg2", "%arg3", M, K, N)
        u = _int4_mm(e, "%arg0", "%arg4", "%arg5", "%arg6", M, K, N)
    else:
        wt = [_t([K, N], "i8"), _t([N], "f32")]
        g = _int8_mm(e, "%arg0", "%arg1", "%arg2", M, K, N)
        u = _int8_mm(e, "%arg0", "%arg3", "%arg4", M, K, N)
    act = e.bin("multiply", e.bin("multiply", g, e.un("logistic", g, ty), ty), u, ty)
    return _module("jit_swiglu_mlp", [_t([M, K], "bf16")] + wt + wt, [ty], e.lines + [f"return {act} : {ty}"])


def _softmax_bf16(e, x, shape):
    """jax.nn.softmax(x, axis=-1) on bf16 x of any rank (the sum upcast to f32)."""
    r = len(shape)
    tx, txf = _t(shape, "bf16"), _t(shape, "f32")
    rows, rows1 = shape[:-1], shape[:-1] + [1]
    tr, trf, tr1 = _t(rows, "bf16"), _t(rows, "f32"), _t(rows1, "bf16")
    lead = list(range(r - 1))
    m = e.reduce(x, tx, e.const(_NEG_INF["bf16"], "bf16"), "tensor<bf16>", "maximum", [r - 1], tr)
    m = e.bin("maximum", e.splat(_NEG_INF["bf16"], "bf16", rows), m, tr)
    mb = e.bcast(e.bcast(m, tr, lead, tr1), tr1, list(range(r)), tx)
    ex = e.un("exponential", e.bin("subtract", x, mb, tx), tx)
    sm = e.reduce(e.cvt(ex, tx, txf), txf, e.const("0.000000e+00", "f32"), "tensor<f32>", "add", [r - 1], trf)
    sb = e.bcast(e.bcast(e.cvt(sm, trf, tr), tr, lead, tr1), tr1, list(range(r)), tx)
    return e.bin("divide", ex, sb, tx)


def causal_attention(B, H, S, D, mask="GE", transpose_k=True):
    """def f(q, k, v):  # bf16 [B, H, S, D]
           sc = (q @ jnp.swapaxes(k, -1, -2)) * D ** -0.5   # or einsum("bhqd,bhkd->bhqk")
           m = jnp.arange(S)[:, None] >= jnp.arange(S)[None, :]
           p = jax.nn.softmax(jnp.where(m, sc, -jnp.inf), axis=-1)
           return (p @ v).transpose(0, 2, 1, 3)             # [B, S, H, D]
    mask: the comparison of row and column index (GE is causal);
    transpose_k=False contracts k on its last axis instead of transposing."""
    e = _Body()
    t4, tkT, ts = _t([B, H, S, D], "bf16"), _t([B, H, D, S], "bf16"), _t([B, H, S, S], "bf16")
    if transpose_k:
        kT = e.transpose("%arg1", t4, [0, 1, 3, 2], tkT)
        sc = e(f"stablehlo.dot_general %arg0, {kT}, batching_dims = [0, 1] x [0, 1], contracting_dims = [3] x [2], "
               f"precision = [DEFAULT, DEFAULT] : ({t4}, {tkT}) -> {ts}")
    else:
        sc = e(f"stablehlo.dot_general %arg0, %arg1, batching_dims = [0, 1] x [0, 1], contracting_dims = [3] x [3], "
               f"precision = [DEFAULT, DEFAULT] : ({t4}, {t4}) -> {ts}")
    sc = e.bin("multiply", sc, e.splat(f"{D ** -0.5:.6e}", "bf16", [B, H, S, S]), ts)
    ti, tm = _t([S], "i32"), _t([S, S], "i32")
    io = e(f"stablehlo.iota dim = 0 : {ti}")
    r = e.bcast(e.bcast(io, ti, [0], _t([S, 1], "i32")), _t([S, 1], "i32"), [0, 1], tm)
    c = e.bcast(e.bcast(io, ti, [1], _t([1, S], "i32")), _t([1, S], "i32"), [0, 1], tm)
    m = e(f"stablehlo.compare  {mask}, {r}, {c},  SIGNED : ({tm}, {tm}) -> {_t([S, S], 'i1')}")
    mb = e.bcast(m, _t([S, S], "i1"), [2, 3], _t([B, H, S, S], "i1"))
    x = e(f"stablehlo.select {mb}, {sc}, {e.splat(_NEG_INF['bf16'], 'bf16', [B, H, S, S])} : "
          f"{_t([B, H, S, S], 'i1')}, {ts}")
    p = _softmax_bf16(e, x, [B, H, S, S])
    o = e(f"stablehlo.dot_general {p}, %arg2, batching_dims = [0, 1] x [0, 1], contracting_dims = [3] x [2], "
          f"precision = [DEFAULT, DEFAULT] : ({ts}, {t4}) -> {t4}")
    tout = _t([B, S, H, D], "bf16")
    out = e.transpose(o, t4, [0, 2, 1, 3], tout)
    return _module("jit_attention", [t4, t4, t4], [tout], e.lines + [f"return {out} : {tout}"])


def decoder_layer(B, S, hidden, heads, head_dim, ffn, eps="9.99999997E-7"):
    """One Llama-style decoder layer as jax.jit lowers it (bf16 activations,
    int4 g64 projections), the reference's transformer-layer benchmark
    (benchmarks/vs_cpu.py:603-626) with RMSNorm, rotate-half RoPE, a causal
    mask and SwiGLU:

        def layer(x, g1, wqkv, wo, g2, wg, wu, wd, cos, sin):  # w* = (p, s, z)
            T, A = B * S, H * D
            qkv = int4mm(rmsnorm(x, g1), *wqkv).reshape(B, S, 3, H, D)
            q, k, v = qkv[:, :, 0], qkv[:, :, 1], qkv[:, :, 2]
            c, s = cos[None, :, None, :], sin[None, :, None, :]
            def rope(t):
                t = t.astype(f32); t0, t1 = t[..., :D // 2], t[..., D // 2:]
                return jnp.concatenate([t0 * c - t1 * s, t1 * c + t0 * s], -1).astype(bf16)
            q, k, v = (t.transpose(0, 2, 1, 3) for t in (rope(q), rope(k), v))
            sc = (q @ jnp.swapaxes(k, -1, -2)) * D ** -0.5
            mask = jnp.arange(S)[:, None] >= jnp.arange(S)[None, :]
            p = jax.nn.softmax(jnp.where(mask, sc, -jnp.inf), axis=-1)
            a = (p @ v).transpose(0, 2, 1, 3).reshape(T, A)
            x1 = x + int4mm(a, *wo)
            h2 = rmsnorm(x1, g2)
            return x1 + int4mm(jax.nn.silu(int4mm(h2, *wg)) * int4mm(h2, *wu), *wd)

    with rmsnorm and int4mm the functions of rmsnorm(dt="bf16") and
    int4_g64_matmul.  Arguments: x bf16 [B*S, hidden]; g_attn bf16 [hidden];
    w_qkv (3 arrays); w_o; g_mlp; w_gate; w_up; w_down; cos, sin f32
    [S, head_dim/2].  The qkv columns are q | k | v, each heads x head_dim."""
    e = _Body()
    args, out = _decoder_args_and_layers(e, 1, B, S, hidden, heads, head_dim, ffn, eps)
    tx = _t([B * S, hidden], "bf16")
    return _module("jit_layer", args, [tx], e.lines + [f"return {out} : {tx}"])


def decoder_stack(layers, B, S, hidden, heads, head_dim, ffn, eps="9.99999997E-7"):
    """The decoder forward of `layers` layers as one jitted function
    (jax.jit of ``for w in weights: x = layer(x, *w, cos, sin)``): arguments
    x, then each layer's 17 weight arrays in decoder_layer's order, then cos
    and sin; returns the last layer's output [B*S, hidden] bf16."""
    e = _Body()
    args, out = _decoder_args_and_layers(e, layers, B, S, hidden, heads, head_dim, ffn, eps)
    tx = _t([B * S, hidden], "bf16")
    return _module("jit_decoder", args, [tx], e.lines + [f"return {out} : {tx}"])


def decoder_stack_scan(layers, B, S, hidden, heads, head_dim, ffn, eps="9.99999997E-7"):
    """The decoder forward written with lax.scan over stacked layer weights
    (the usual way to write a layer stack):

        def f(x, *stacked_w, cos, sin):     # each weight array [layers, ...]
            def step(x, w):
                return layer(x, *w, cos, sin), None
            return jax.lax.scan(step, x, stacked_w)[0]

    lowered as jax lowers a scan: a stablehlo.while whose carry is (counter,
    x, stacked weights), a cond of counter < layers, and a body that wraps a
    negative index (select(i < 0, i + layers, i)), takes each layer's weights
    with dynamic_slice + reshape, runs the layer and returns counter + 1.
    Arguments: x, the 17 stacked weight arrays in decoder_layer's order,
    cos, sin; returns the last layer's output [B*S, hidden] bf16."""
    e = _Body()
    H, D, T, A, F = heads, head_dim, B * S, heads * head_dim, ffn
    Dh = D // 2

    def w3(K, N):
        return [([K // 2, N], "ui8"), ([K // 64, N], "bf16"), ([K // 64, N], "ui8")]

    per_layer = ([([hidden], "bf16")] + w3(hidden, 3 * A) + w3(A, hidden) + [([hidden], "bf16")] +
                 w3(hidden, F) + w3(hidden, F) + w3(F, hidden))
    stacked = [_t([layers] + d, dt) for d, dt in per_layer]
    tx = _t([T, hidden], "bf16")
    ti = _t([], "i32")
    args = [tx] + stacked + [_t([S, Dh], "f32"), _t([S, Dh], "f32")]
    cos_arg, sin_arg = f"%arg{1 + len(per_layer)}", f"%arg{2 + len(per_layer)}"
    th, t4 = _t([B, S, H, Dh], "f32"), _t([1, S, 1, Dh], "f32")
    c = e.bcast(e.reshape(cos_arg, _t([S, Dh], "f32"), t4), t4, [0, 1, 2, 3], th)
    s = e.bcast(e.reshape(sin_arg, _t([S, Dh], "f32"), t4), t4, [0, 1, 2, 3], th)
    zero = e.const(0, "i32")
    names = ["%iterArg", "%iterArg_0"] + [f"%iterArg_{i + 1}" for i in range(len(per_layer))]
    inits = [zero, "%arg0"] + [f"%arg{i + 1}" for i in range(len(per_layer))]
    types = [ti, tx] + stacked
    loop = f"%{len(e.lines)}"
    e.lines.append(f"{loop}:{len(names)} = stablehlo.while(" +
                   ", ".join(f"{a} = {b}" for a, b in zip(names, inits)) + ") : " + ", ".join(types))
    e.lines.append("cond {")
    n_layers = e.const(layers, "i32")
    more = e(f"stablehlo.compare  LT, %iterArg, {n_layers},  SIGNED : ({ti}, {ti}) -> {_t([], 'i1')}")
    e.lines.append(f"stablehlo.return {more} : {_t([], 'i1')}")
    e.lines.append("} do {")
    c0 = e.const(0, "i32")
    neg = e(f"stablehlo.compare  LT, %iterArg, {c0},  SIGNED : ({ti}, {ti}) -> {_t([], 'i1')}")
    wrapped = e.bin("add", "%iterArg", e.const(layers, "i32"), ti)
    idx = e(f"stablehlo.select {neg}, {wrapped}, %iterArg : {_t([], 'i1')}, {ti}")
    w = []
    for k, (d, dt) in enumerate(per_layer):
        starts = ", ".join([idx] + [c0] * len(d))
        t1 = _t([1] + d, dt)
        ds = e(f"stablehlo.dynamic_slice {names[2 + k]}, {starts}, sizes = [{', '.join(map(str, [1] + d))}] : "
               f"({stacked[k]}, {', '.join([ti] * (len(d) + 1))}) -> {t1}")
        w.append(e.reshape(ds, t1, _t(d, dt)))
    x_new = _decoder_layer_ops(e, "%iterArg_0", w, c, s, B, S, hidden, H, D, F, eps)
    nxt = e.bin("add", "%iterArg", e.const(1, "i32"), ti)
    e.lines.append(f"stablehlo.return {nxt}, {x_new}, " + ", ".join(names[2:]) + " : " + ", ".join(types))
    e.lines.append("}")
    return _module("jit_decoder_scan", args, [tx], e.lines + [f"return {loop}#1 : {tx}"])


def counted_loop(trips, n=8, cond="LT", step=1, start=0):
    """A fori_loop the plugin unrolls: def f(x): return lax.fori_loop(start,
    trips, lambda i, x: x * 2 + i.astype(f32), x) on f32 [n], lowered as a
    stablehlo.while over (counter, x) with the given comparison and counter
    step (a non-counted or too long loop is an error at compile)."""
    e = _Body()
    tx, ti = _t([n], "f32"), _t([], "i32")
    c0 = e.const(start, "i32")
    loop = f"%{len(e.lines)}"
    e.lines.append(f"{loop}:2 = stablehlo.while(%iterArg = {c0}, %iterArg_0 = %arg0) : {ti}, {tx}")
    e.lines.append("cond {")
    lim = e.const(trips, "i32")
    more = e(f"stablehlo.compare  {cond}, %iterArg, {lim},  SIGNED : ({ti}, {ti}) -> {_t([], 'i1')}")
    e.lines.append(f"stablehlo.return {more} : {_t([], 'i1')}")
    e.lines.append("} do {")
    two = e.splat("2.000000e+00", "f32", [n])
    fi = e.bcast(e.cvt("%iterArg", ti, _t([], "f32")), _t([], "f32"), [], tx)
    y = e.bin("add", e.bin("multiply", "%iterArg_0", two, tx), fi, tx)
    nxt = e.bin("add", "%iterArg", e.const(step, "i32"), ti)
    e.lines.append(f"stablehlo.return {nxt}, {y} : {ti}, {tx}")
    e.lines.append("}")
    return _module("jit_loop", [tx], [tx], e.lines + [f"return {loop}#1 : {tx}"])


def _decoder_args_and_layers(e, layers, B, S, hidden, heads, head_dim, ffn, eps):
    """Argument types (x, per layer g_attn w_qkv(3) w_o(3) g_mlp w_gate(3)
    w_up(3) w_down(3), cos, sin) and the ops of `layers` layers into e;
    returns (arg types, name of the last output)."""
    H, D, T, A, F = heads, head_dim, B * S, heads * head_dim, ffn
    Dh = D // 2

    def w3(K, N):
        return [_t([K // 2, N], "ui8"), _t([K // 64, N], "bf16"), _t([K // 64, N], "ui8")]

    per_layer = ([_t([hidden], "bf16")] + w3(hidden, 3 * A) + w3(A, hidden) + [_t([hidden], "bf16")] +
                 w3(hidden, F) + w3(hidden, F) + w3(F, hidden))
    args = [_t([T, hidden], "bf16")] + per_layer * layers + [_t([S, Dh], "f32"), _t([S, Dh], "f32")]
    cos_arg, sin_arg = f"%arg{1 + 17 * layers}", f"%arg{2 + 17 * layers}"
    th, t4 = _t([B, S, H, Dh], "f32"), _t([1, S, 1, Dh], "f32")
    c = e.bcast(e.reshape(cos_arg, _t([S, Dh], "f32"), t4), t4, [0, 1, 2, 3], th)
    s = e.bcast(e.reshape(sin_arg, _t([S, Dh], "f32"), t4), t4, [0, 1, 2, 3], th)
    x = "%arg0"
    for l in range(layers):
        base = 1 + 17 * l
        a = [f"%arg{base + i}" for i in range(17)]
        x = _decoder_layer_ops(e, x, a, c, s, B, S, hidden, H, D, F, eps)
    return args, x


def _decoder_layer_ops(e, x, a, c, s, B, S, hidden, H, D, F, eps):
    """One layer's ops: x [B*S, hidden]; a = the layer's 17 argument names;
    c, s the broadcast RoPE tables [B, S, H, D/2]."""
    T, A, Dh = B * S, H * D, D // 2
    g1, wqkv, wo, g2, wg, wu, wd = a[0], a[1:4], a[4:7], a[7], a[8:11], a[11:14], a[14:17]
    tb = _t([B, S, H, D], "bf16")
    h = _rmsnorm_bf16(e, x, g1, T, hidden, eps)
    qkv = e.reshape(_int4_mm(e, h, *wqkv, T, hidden, 3 * A), _t([T, 3 * A], "bf16"), _t([B, S, 3, H, D], "bf16"))
    parts = []
    for j in range(3):
        sl = e.slice(qkv, _t([B, S, 3, H, D], "bf16"), [(0, B), (0, S), (j, j + 1), (0, H), (0, D)],
                     _t([B, S, 1, H, D], "bf16"))
        parts.append(e.reshape(sl, _t([B, S, 1, H, D], "bf16"), tb))
    q, k, v = parts
    th, tf = _t([B, S, H, Dh], "f32"), _t([B, S, H, D], "f32")

    def rope(t):
        tf_ = e.cvt(t, tb, tf)
        t0 = e.slice(tf_, tf, [(0, B), (0, S), (0, H), (0, Dh)], th)
        t1 = e.slice(tf_, tf, [(0, B), (0, S), (0, H), (Dh, D)], th)
        lo = e.bin("subtract", e.bin("multiply", t0, c, th), e.bin("multiply", t1, s, th), th)
        hi = e.bin("add", e.bin("multiply", t1, c, th), e.bin("multiply", t0, s, th), th)
        cat = e(f"stablehlo.concatenate {lo}, {hi}, dim = 3 : ({th}, {th}) -> {tf}")
        return e.cvt(cat, tf, tb)

    tbh = _t([B, H, S, D], "bf16")
    qt = e.transpose(rope(q), tb, [0, 2, 1, 3], tbh)
    kt = e.transpose(rope(k), tb, [0, 2, 1, 3], tbh)
    vt = e.transpose(v, tb, [0, 2, 1, 3], tbh)
    tkT, tsc = _t([B, H, D, S], "bf16"), _t([B, H, S, S], "bf16")
    kT = e.transpose(kt, tbh, [0, 1, 3, 2], tkT)
    sc = e(f"stablehlo.dot_general {qt}, {kT}, batching_dims = [0, 1] x [0, 1], contracting_dims = [3] x [2], "
           f"precision = [DEFAULT, DEFAULT] : ({tbh}, {tkT}) -> {tsc}")
    sc = e.bin("multiply", sc, e.splat(f"{D ** -0.5:.6e}", "bf16", [B, H, S, S]), tsc)
    ti, ti1, tm = _t([S], "i32"), _t([S, 1], "i32"), _t([S, S], "i32")
    io = e(f"stablehlo.iota dim = 0 : {ti}")
    r_ = e.bcast(e.bcast(io, ti, [0], ti1), ti1, [0, 1], tm)
    c_ = e.bcast(e.bcast(io, ti, [1], _t([1, S], "i32")), _t([1, S], "i32"), [0, 1], tm)
    mask = e(f"stablehlo.compare  GE, {r_}, {c_},  SIGNED : ({tm}, {tm}) -> {_t([S, S], 'i1')}")
    maskb = e.bcast(mask, _t([S, S], "i1"), [2, 3], _t([B, H, S, S], "i1"))
    sc = e(f"stablehlo.select {maskb}, {sc}, {e.splat(_NEG_INF['bf16'], 'bf16', [B, H, S, S])} : "
           f"{_t([B, H, S, S], 'i1')}, {tsc}")
    p = _softmax_bf16(e, sc, [B, H, S, S])
    o = e(f"stablehlo.dot_general {p}, {vt}, batching_dims = [0, 1] x [0, 1], contracting_dims = [3] x [2], "
          f"precision = [DEFAULT, DEFAULT] : ({tsc}, {tbh}) -> {tbh}")
    att = e.reshape(e.transpose(o, tbh, [0, 2, 1, 3], tb), tb, _t([T, A], "bf16"))
    tx = _t([T, hidden], "bf16")
    x1 = e.bin("add", x, _int4_mm(e, att, *wo, T, A, hidden), tx)
    h2 = _rmsnorm_bf16(e, x1, g2, T, hidden, eps)
    tfb = _t([T, F], "bf16")
    gt = _int4_mm(e, h2, *wg, T, hidden, F)
    up = _int4_mm(e, h2, *wu, T, hidden, F)
    act = e.bin("multiply", e.bin("multiply", gt, e.un("logistic", gt, tfb), tfb), up, tfb)
    return e.bin("add", x1, _int4_mm(e, act, *wd, T, F, hidden), tx)
