"""ctypes loader for the C restatement ``oracle/c/oracle.c`` (test infrastructure only)."""

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "lib", "liboracle_c.so")
        if not os.path.exists(path):
            raise RuntimeError(f"{path} missing: run oracle/build_oracle.sh (or __graft_entry__.build())")
        L = ctypes.CDLL(path)
        p = ctypes.c_void_p
        i64 = ctypes.c_int64
        L.orc_threads.argtypes = [ctypes.c_int]
        L.orc_threads.restype = ctypes.c_int
        L.orc_int4_g64_matmul.argtypes = [p, p, p, p, i64, i64, i64, i64, i64, p]
        L.orc_int8_pc_matmul.argtypes = [p, p, p, i64, i64, i64, i64, i64, p]
        L.orc_gemm_bf16.argtypes = [p, p, i64, i64, i64, i64, i64, p]
        L.orc_gemm_f32.argtypes = [p, p, i64, i64, i64, i64, i64, p]
        L.orc_argmax_f32.argtypes = [p, i64, i64, p]
        L.orc_argmax_bf16.argtypes = [p, i64, i64, p]
        L.orc_softmax_f32.argtypes = [p, i64, i64, i64, p]
        L.orc_softmax_bf16.argtypes = [p, i64, i64, i64, p]
        L.orc_rmsnorm_f32.argtypes = [p, p, i64, ctypes.c_float, i64, i64, p]
        L.orc_rmsnorm_bf16.argtypes = [p, p, i64, ctypes.c_float, i64, i64, p]
        L.orc_chain6_f32.argtypes = [p, i64, p]
        L.orc_chain6_bf16.argtypes = [p, i64, p]
        L.orc_plumbing_f32.argtypes = [p, p, i64, i64, i64, p]
        _LIB = L
    return _LIB


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def threads(n=0):
    """Set (n > 0) and return the OpenMP thread count the port uses."""
    return lib().orc_threads(n)


def int4_g64_matmul(x_bits, packed, s_bits, z, n_range=None):
    M, K = x_bits.shape
    N = packed.shape[1]
    n0, n1 = n_range or (0, N)
    y = np.zeros((M, N), dtype=np.float32)
    arrs = [np.ascontiguousarray(a) for a in (x_bits, packed, s_bits, z)]
    lib().orc_int4_g64_matmul(*[_ptr(a) for a in arrs], M, K, N, n0, n1, _ptr(y))
    return y


def int8_pc_matmul(x_bits, w, s, n_range=None):
    M, K = x_bits.shape
    N = w.shape[1]
    n0, n1 = n_range or (0, N)
    y = np.zeros((M, N), dtype=np.float32)
    arrs = [np.ascontiguousarray(a) for a in (x_bits, w, s)]
    lib().orc_int8_pc_matmul(*[_ptr(a) for a in arrs], M, K, N, n0, n1, _ptr(y))
    return y


def gemm_bf16(a_bits, b_bits, m_range=None):
    M, K = a_bits.shape
    N = b_bits.shape[1]
    m0, m1 = m_range or (0, M)
    c = np.zeros((M, N), dtype=np.float32)
    a = np.ascontiguousarray(a_bits)
    b = np.ascontiguousarray(b_bits)
    lib().orc_gemm_bf16(_ptr(a), _ptr(b), M, K, N, m0, m1, _ptr(c))
    return c


def gemm_f32(a, b, m_range=None):
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    M, K = a.shape
    N = b.shape[1]
    m0, m1 = m_range or (0, M)
    c = np.zeros((M, N), dtype=np.float32)
    lib().orc_gemm_f32(_ptr(a), _ptr(b), M, K, N, m0, m1, _ptr(c))
    return c


def argmax_f32(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, cols = x.shape
    out = np.zeros(rows, dtype=np.int32)
    lib().orc_argmax_f32(_ptr(x), rows, cols, _ptr(out))
    return out


def argmax_bf16(x_bits):
    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    rows, cols = x.shape
    out = np.zeros(rows, dtype=np.int32)
    lib().orc_argmax_bf16(_ptr(x), rows, cols, _ptr(out))
    return out


def _out_like(x, row_range):
    """Output array: rows outside row_range stay zero; without a range every
    row is written, so no fill is needed."""
    return np.empty_like(x) if row_range is None else np.zeros_like(x)


def _rows(x, row_range):
    rows = x.shape[0]
    return row_range or (0, rows)


def softmax(x, row_range=None):
    """f32 softmax over the last axis (f32 in, f32 out) or, for uint16 input,
    bf16 softmax on bit patterns (bf16 bits out).  Rows outside row_range
    are left zero."""
    if x.dtype != np.uint16:
        x = np.asarray(x, dtype=np.float32)
    x = np.ascontiguousarray(x)
    r0, r1 = _rows(x, row_range)
    y = _out_like(x, row_range)
    fn = lib().orc_softmax_bf16 if x.dtype == np.uint16 else lib().orc_softmax_f32
    fn(_ptr(x), x.shape[1], r0, r1, _ptr(y))
    return y


def rmsnorm(x, g, eps=1e-6, row_range=None):
    """RMSNorm over the last axis: f32 (float32 x, g) or bf16 bits (uint16 x, g)."""
    x = np.ascontiguousarray(x)
    g = np.ascontiguousarray(g)
    r0, r1 = _rows(x, row_range)
    if x.dtype == np.uint16:
        y = _out_like(x, row_range)
        lib().orc_rmsnorm_bf16(_ptr(x), _ptr(g), x.shape[1], eps, r0, r1, _ptr(y))
    else:
        x = np.ascontiguousarray(x, dtype=np.float32)
        g = np.ascontiguousarray(g, dtype=np.float32)
        y = _out_like(x, row_range)
        lib().orc_rmsnorm_f32(_ptr(x), _ptr(g), x.shape[1], eps, r0, r1, _ptr(y))
    return y


def chain6(x):
    """The workload's 6-op elementwise chain: f32, or bf16 bits for uint16 input."""
    x = np.ascontiguousarray(x)
    if x.dtype == np.uint16:
        y = np.empty_like(x)
        lib().orc_chain6_bf16(_ptr(x), x.size, _ptr(y))
    else:
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.empty_like(x)
        lib().orc_chain6_f32(_ptr(x), x.size, _ptr(y))
    return y


def plumbing(a, b, row_range=None):
    """tanh(A @ B).sum(axis=1) in f32 for rows in row_range (others zero)."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    n = a.shape[0]
    r0, r1 = row_range or (0, n)
    y = np.zeros(n, dtype=np.float32)
    lib().orc_plumbing_f32(_ptr(a), _ptr(b), n, r0, r1, _ptr(y))
    return y
