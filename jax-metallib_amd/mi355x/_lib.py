"""ctypes binding of the plugin's C-ABI (include/mk_kernels.h, include/mk_runtime.h).

The library is built in-tree by ``jax-metallib_amd/build.py`` (or
``__graft_entry__.build()``).  Loading fails loudly when it is missing: the
plugin has no CPU fallback.
"""

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(os.path.dirname(HERE), "lib")
KERNELS_SO = os.path.join(LIB_DIR, "libmk_kernels.so")

MK_OK, MK_EINVAL, MK_EUNSUPPORTED, MK_EWORKSPACE, MK_ELAUNCH = 0, 1, 2, 3, 4
MK_QFMT_INT4_G64, MK_QFMT_INT8_PC = 0, 1
MK_DT_F32, MK_DT_BF16 = 0, 1
MK_EPI_NONE, MK_EPI_ADD, MK_EPI_SWIGLU, MK_EPI_SWIGLU_PAIRS = 0, 1, 2, 3
# bf16 GEMM routes (MK_GEMM_ROUTE_*)
GEMM_ROUTES = {"default": 0, "ring": 1, "pipe": 2, "persist": 3, "short": 4, "reg256": 5, "generic256": 6,
               "generic128": 7}
MK_REDUCE_SUM, MK_REDUCE_MAX, MK_REDUCE_MIN = 0, 1, 2
EW_OPS = ["LOAD", "CONST", "ADD", "SUB", "MUL", "DIV", "MAX", "MIN", "POW", "NEG", "ABS", "EXP", "LOG",
          "LOG1P", "EXPM1", "TANH", "RSQRT", "SQRT", "LOGISTIC", "FLOOR", "CEIL", "CMP_EQ", "CMP_NE",
          "CMP_LT", "CMP_LE", "CMP_GT", "CMP_GE", "SELECT", "ROUND_BF16"]
EW = {name: i for i, name in enumerate(EW_OPS)}
MK_EW_IN_DEFAULT, MK_EW_IN_F32, MK_EW_IN_BF16 = 0, 1, 2  # LOAD's b: the input's element type
MK_EW_KEEP_F32 = 64  # or'ed into an op: an unrounded f32 result in a bf16 program


class EwInstr(ctypes.Structure):
    """mk_ew_instr (include/mk_kernels.h)."""
    _fields_ = [("op", ctypes.c_int32), ("dst", ctypes.c_int32), ("a", ctypes.c_int32),
                ("b", ctypes.c_int32), ("c", ctypes.c_int32), ("imm", ctypes.c_float)]

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int

# name -> (restype, argtypes); mirrors include/mk_kernels.h
SIGNATURES = {
    "mk_last_error": (ctypes.c_char_p, []),
    "mk_version": (ctypes.c_char_p, []),
    "mk_qmatmul_workspace_bytes": (_i64, [_i32, _i64, _i64, _i64]),
    "mk_qmatmul_epilogue_supported": (_i32, [_i32, _i64, _i64, _i64, _i32]),
    "mk_dot_general": (_i32, [_i32, _i32, _i32, _p, _p, _p, _i64, _i64, _i64, _i64, ctypes.POINTER(_i64),
                              ctypes.POINTER(_i64), _p]),
    "mk_int4g64_matmul_bf16": (_i32, [_p, _p, _p, _p, _p, _i64, _i64, _i64, _p, _i64, _p]),
    "mk_int4g64_matmul_bf16_noalloc": (_i32, [_p, _p, _p, _p, _p, _i64, _i64, _i64, _p]),
    "mk_int8pc_matmul_bf16": (_i32, [_p, _p, _p, _p, _i64, _i64, _i64, _p, _i64, _p]),
    "mk_gemm_bf16": (_i32, [_p, _p, _p, _i64, _i64, _i64, _i64, _i32, _p]),
    "mk_gemm_bf16_epilogue": (_i32, [_p, _p, _p, _p, _i32, _i64, _i64, _i64, _i64, _p]),
    "mk_gemm_bf16_nt": (_i32, [_p, _p, _p, _p, _i32, _i64, _i64, _i64, _i64, _p]),
    "mk_gemm_bf16_route": (_i32, [_p, _p, _p, _p, _i32, _i64, _i64, _i64, _i64, _i32, _i32, _p]),
    "mk_gemm_bf16_route_fits": (_i32, [_i32, _i64, _i64, _i64, _i32, _i32]),
    "mk_gemm_bf16_autotune": (_i32, [_p, _p, _p, _p, _i32, _i64, _i64, _i64, _i64, _i32, _p,
                                     ctypes.POINTER(_i32), ctypes.POINTER(ctypes.c_float)]),
    "mk_gemm_tuned_route": (_i32, [_i64, _i64, _i64, _i64, _i32, _i32]),
    "mk_gemm_autotune_save": (_i32, [ctypes.c_char_p]),
    "mk_gemm_autotune_load": (_i32, [ctypes.c_char_p]),
    "mk_gemm_autotune_clear": (None, []),
    "mk_gemm_autotune_header": (ctypes.c_char_p, []),
    "mk_int4g64_matmul_epilogue_bf16": (_i32, [_p, _p, _p, _p, _p, _p, _i32, _i64, _i64, _i64, _p, _i64, _p]),
    "mk_int8pc_matmul_epilogue_bf16": (_i32, [_p, _p, _p, _p, _p, _i32, _i64, _i64, _i64, _p, _i64, _p]),
    "mk_qmatmul_swiglu_pair_workspace_bytes": (_i64, [_i32, _i64, _i64, _i64]),
    "mk_int4g64_matmul_swiglu_pair_bf16": (_i32, [_p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _p, _i64, _p]),
    "mk_int8pc_matmul_swiglu_pair_bf16": (_i32, [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _p, _i64, _p]),
    "mk_gemm_f32": (_i32, [_p, _p, _p, _i64, _i64, _i64, _i64, _p]),
    "mk_softmax_lastdim": (_i32, [_i32, _p, _p, _i64, _i64, _p]),
    "mk_rope_qkv_split_bf16": (_i32, [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i32, _p]),
    "mk_attention_causal_bf16": (_i32, [_p, _p, _p, _p, _i64, _i64, _i64, _i64, ctypes.c_float, _p]),
    "mk_softmax_causal_bf16": (_i32, [_p, _p, _i64, _i64, ctypes.c_float, _p]),
    "mk_merge_heads_bf16": (_i32, [_p, _p, _i64, _i64, _i64, _i64, _p]),
    "mk_rmsnorm_lastdim": (_i32, [_i32, _p, _p, _p, _i64, _i64, ctypes.c_float, _p]),
    "mk_argmax_lastdim": (_i32, [_i32, _p, _p, _i64, _i64, _p]),
    "mk_reduce_lastdim": (_i32, [_i32, _i32, _p, _p, _i64, _i64, _p]),
    "mk_elementwise": (_i32, [_i32, _p, _i32, _p, _p, _i32, _i32, _p, _i64, _p]),
    "mk_strided_copy": (_i32, [_p, _p, _i32, _i32, _p, _p, _i64, _p, _i64, _p]),
    "mk_iota": (_i32, [_p, _i32, _i32, _p, _i32, _p]),
    "mk_elementwise_prepare": (_i32, [_i32, _p, _i32, _i32, _i32]),
}

_cb = ctypes.CFUNCTYPE(None, _p, _p)
_pp = ctypes.POINTER(_p)

# name -> (restype, argtypes); mirrors include/mk_runtime.h (opaque handles as void*)
RUNTIME_SIGNATURES = {
    "mkrt_error_destroy": (None, [_p]),
    "mkrt_error_message": (ctypes.c_char_p, [_p]),
    "mkrt_error_code": (_i32, [_p]),
    "mkrt_client_create": (_p, [_pp]),
    "mkrt_client_destroy": (None, [_p]),
    "mkrt_client_platform_name": (ctypes.c_char_p, [_p]),
    "mkrt_client_memory_stats": (_p, [_p, ctypes.POINTER(_i64), ctypes.POINTER(_i64)]),
    "mkrt_buffer_from_host": (_p, [_p, _p, _i32, ctypes.POINTER(_i64), _i32, _pp, _pp]),
    "mkrt_buffer_to_host": (_p, [_p, _p, _i64, _pp]),
    "mkrt_buffer_type": (_i32, [_p]),
    "mkrt_buffer_ndims": (_i32, [_p]),
    "mkrt_buffer_dims": (ctypes.POINTER(_i64), [_p]),
    "mkrt_buffer_bytes": (_i64, [_p]),
    "mkrt_buffer_ready_event": (_p, [_p, _pp]),
    "mkrt_buffer_create_error": (_p, [_p, _i32, ctypes.c_char_p, _i32, ctypes.POINTER(_i64), _i32, _pp]),
    "mkrt_buffer_destroy": (None, [_p]),
    "mkrt_buffer_from_host_strided": (_p, [_p, _p, _i32, ctypes.POINTER(_i64), _i32, ctypes.POINTER(_i64), _i32,
                                           _pp, _pp]),
    "mkrt_buffer_copy_raw_to_host": (_p, [_p, _p, _i64, _i64, _pp]),
    "mkrt_buffer_create_view": (_p, [_p, _p, _i32, ctypes.POINTER(_i64), _i32, _p, _p, _pp]),
    "mkrt_buffer_create_uninitialized": (_p, [_p, _i32, ctypes.POINTER(_i64), _i32, _pp]),
    "mkrt_buffer_copy": (_p, [_p, _pp]),
    "mkrt_buffer_delete": (None, [_p]),
    "mkrt_buffer_is_deleted": (_i32, [_p]),
    "mkrt_buffer_device_pointer": (_p, [_p]),
    "mkrt_compile": (_p, [_p, ctypes.c_char_p, _i64, ctypes.c_char_p, _pp]),
    "mkrt_bytecode_to_text": (_p, [ctypes.c_char_p, _i64, ctypes.c_char_p, _i64, ctypes.POINTER(_i64)]),
    "mkrt_compile_check": (_p, [ctypes.c_char_p, _i64, ctypes.c_char_p, ctypes.c_char_p, _i64,
                                ctypes.POINTER(_i32)]),
    "mkrt_executable_num_inputs": (_i32, [_p]),
    "mkrt_executable_num_outputs": (_i32, [_p]),
    "mkrt_executable_output_type": (_i32, [_p, _i32]),
    "mkrt_executable_output_ndims": (_i32, [_p, _i32]),
    "mkrt_executable_output_dims": (ctypes.POINTER(_i64), [_p, _i32]),
    "mkrt_executable_program": (_p, [_p, ctypes.POINTER(_i64)]),
    "mkrt_executable_num_steps": (_i32, [_p]),
    "mkrt_executable_plan": (ctypes.c_char_p, [_p]),
    "mkrt_execute": (_p, [_p, _pp, _i32, _pp, _pp]),
    "mkrt_executable_destroy": (None, [_p]),
    "mkrt_executable_serialize": (_p, [_p, _pp]),
    "mkrt_serialize_program": (_p, [ctypes.c_char_p, _i64, ctypes.c_char_p, _pp]),
    "mkrt_serialized_data": (_p, [_p]),
    "mkrt_serialized_size": (_i64, [_p]),
    "mkrt_serialized_destroy": (None, [_p]),
    "mkrt_deserialize": (_p, [_p, ctypes.c_char_p, _i64, _pp]),
    "mkrt_serialized_inspect": (_p, [ctypes.c_char_p, _i64, ctypes.POINTER(_i64), ctypes.POINTER(_i32)]),
    "mkrt_executable_fingerprint": (ctypes.c_char_p, [_p]),
    "mkrt_jit_cache_stats": (None, [ctypes.POINTER(_i64), ctypes.POINTER(_i64), ctypes.POINTER(_i64)]),
    "mkrt_event_create": (_p, [_pp]),
    "mkrt_event_set": (_p, [_p, _i32, ctypes.c_char_p]),
    "mkrt_event_is_ready": (_i32, [_p]),
    "mkrt_event_error": (_p, [_p]),
    "mkrt_event_await": (_p, [_p, _i64]),
    "mkrt_event_on_ready": (_p, [_p, _cb, _p]),
    "mkrt_event_destroy": (None, [_p]),
}
EVENT_CALLBACK = _cb

_LIB = None


class MKError(RuntimeError):
    """A kernel entry point returned a non-zero MK_E* status."""

    def __init__(self, code, msg):
        super().__init__(f"[MK error {code}] {msg}")
        self.code = code


def lib():
    """The loaded kernel library (raises if it has not been built)."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(KERNELS_SO):
            raise RuntimeError(
                f"{KERNELS_SO} is missing: build it with `python jax-metallib_amd/build.py` "
                "(the plugin has no CPU fallback)")
        L = ctypes.CDLL(KERNELS_SO)
        for name, (res, args) in list(SIGNATURES.items()) + list(RUNTIME_SIGNATURES.items()):
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = L
    return _LIB


def check(status):
    """Raise MKError for a non-zero status, with mk_last_error()'s message."""
    if status != MK_OK:
        raise MKError(status, lib().mk_last_error().decode())
    return status
