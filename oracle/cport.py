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
        L.orc_argmax_f32.argtypes = [p, i64, i64, p]
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


def argmax_f32(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, cols = x.shape
    out = np.zeros(rows, dtype=np.int32)
    lib().orc_argmax_f32(_ptr(x), rows, cols, _ptr(out))
    return out
