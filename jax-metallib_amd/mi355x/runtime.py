"""Python view of the plugin runtime (include/mk_runtime.h).

The object model is PJRT's, as the reference's C-API layer implements it
(src/pjrt_plugin/api/): a Client owns one device and its stream; Buffers are
device arrays created from host data or returned by an execution; an
Executable is StableHLO text compiled to a kernel plan; Events signal
completion and may carry an error.  Every call goes to the native library;
there is no CPU fallback.

bf16 host data is passed as uint16 bit patterns with ``type=BF16``.
"""

import ctypes

import numpy as np

from . import _lib

# PJRT_Buffer_Type values.
PRED, S8, S16, S32, S64, U8, U16, U32, U64, F16, F32, F64, BF16 = range(1, 14)
_NP = {PRED: np.bool_, S8: np.int8, S16: np.int16, S32: np.int32, S64: np.int64, U8: np.uint8,
       U16: np.uint16, U32: np.uint32, U64: np.uint64, F16: np.float16, F32: np.float32,
       F64: np.float64, BF16: np.uint16}
_FROM_NP = {np.dtype(v): k for k, v in _NP.items() if k != BF16}

# PJRT_Error_Code values used by the runtime.
OK, INVALID_ARGUMENT, DEADLINE_EXCEEDED, FAILED_PRECONDITION = 0, 3, 4, 9
RESOURCE_EXHAUSTED, UNIMPLEMENTED, INTERNAL, UNAVAILABLE = 8, 12, 13, 14

_p = ctypes.c_void_p
_live_callbacks = {}  # id -> ctypes callback kept alive until it runs


class PluginError(RuntimeError):
    """An mkrt_error: a PJRT error code and message."""

    def __init__(self, code, message):
        super().__init__(f"[code {code}] {message}")
        self.code = code
        self.message = message


def _raise(err):
    """Turn an owned mkrt_error* into PluginError (freeing it); None passes."""
    if not err:
        return
    L = _lib.lib()
    code = L.mkrt_error_code(err)
    msg = L.mkrt_error_message(err).decode()
    L.mkrt_error_destroy(err)
    raise PluginError(code, msg)


def compile_check(text):
    """Parse and plan StableHLO text without a device -> (plan text, steps)."""
    L = _lib.lib()
    data = text.encode() if isinstance(text, str) else bytes(text)
    buf = ctypes.create_string_buffer(1 << 16)
    n = ctypes.c_int(0)
    _raise(L.mkrt_compile_check(data, len(data), b"mlir", buf, len(buf), ctypes.byref(n)))
    return buf.value.decode(), n.value


def bytecode_to_text(blob):
    """MLIR bytecode (a StableHLO portable artifact) -> the MLIR text the
    compile path reads (the reference's bytecodeToText,
    core/stablehlo_parser.mm:597)."""
    L = _lib.lib()
    data = bytes(blob)
    size = ctypes.c_int64(0)
    _raise(L.mkrt_bytecode_to_text(data, len(data), None, 0, ctypes.byref(size)))
    buf = ctypes.create_string_buffer(size.value + 1)
    _raise(L.mkrt_bytecode_to_text(data, len(data), buf, len(buf), ctypes.byref(size)))
    return buf.raw[:size.value].decode()


def _take_serialized(handle):
    """bytes of an owned mkrt_serialized (freeing it)."""
    L = _lib.lib()
    try:
        n = L.mkrt_serialized_size(handle)
        return ctypes.string_at(L.mkrt_serialized_data(handle), n)
    finally:
        L.mkrt_serialized_destroy(handle)


def serialize_program(text):
    """Serialized executable of StableHLO text, without a device: the program
    plus the compiled code objects of its fused elementwise programs."""
    data = text.encode() if isinstance(text, str) else bytes(text)
    h = _p()
    _raise(_lib.lib().mkrt_serialize_program(data, len(data), b"mlir", ctypes.byref(h)))
    return _take_serialized(h.value)


def inspect_serialized(blob):
    """(program bytes, code objects) of a serialized executable; raises
    PluginError(INVALID_ARGUMENT) for malformed data."""
    n, k = ctypes.c_int64(0), ctypes.c_int(0)
    _raise(_lib.lib().mkrt_serialized_inspect(bytes(blob), len(blob), ctypes.byref(n), ctypes.byref(k)))
    return n.value, k.value


def jit_cache_stats():
    """Process totals of the elementwise JIT: (compiles, disk hits, memory hits)."""
    c, d, m = ctypes.c_int64(0), ctypes.c_int64(0), ctypes.c_int64(0)
    _lib.lib().mkrt_jit_cache_stats(ctypes.byref(c), ctypes.byref(d), ctypes.byref(m))
    return c.value, d.value, m.value


class Event:
    """A completion event (PJRT_Event)."""

    def __init__(self, handle):
        self._h = handle

    @classmethod
    def create(cls):
        h = _p()
        _raise(_lib.lib().mkrt_event_create(ctypes.byref(h)))
        return cls(h.value)

    def set(self, code=OK, message=""):
        _raise(_lib.lib().mkrt_event_set(self._h, code, message.encode()))

    def is_ready(self):
        return bool(_lib.lib().mkrt_event_is_ready(self._h))

    def error(self):
        """None when ready without error; raises PluginError otherwise."""
        _raise(_lib.lib().mkrt_event_error(self._h))

    def wait(self, timeout_ms=-1):
        _raise(_lib.lib().mkrt_event_await(self._h, int(timeout_ms)))

    def on_ready(self, fn):
        """fn(error_or_None) runs once, on the completing thread or inline."""
        L = _lib.lib()

        def tramp(err, _user):
            _live_callbacks.pop(id(cb), None)
            e = None
            if err:
                e = PluginError(L.mkrt_error_code(err), L.mkrt_error_message(err).decode())
                L.mkrt_error_destroy(err)
            fn(e)

        cb = _lib.EVENT_CALLBACK(tramp)
        _live_callbacks[id(cb)] = cb
        _raise(L.mkrt_event_on_ready(self._h, cb, None))

    def close(self):
        if self._h:
            _lib.lib().mkrt_event_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Buffer:
    """A device array owned by the caller (PJRT_Buffer)."""

    def __init__(self, handle, client):
        self._h = handle
        self._client = client  # keeps the client alive while the buffer lives

    @property
    def type(self):
        return _lib.lib().mkrt_buffer_type(self._h)

    @property
    def shape(self):
        L = _lib.lib()
        n = L.mkrt_buffer_ndims(self._h)
        d = L.mkrt_buffer_dims(self._h)
        return tuple(d[i] for i in range(n))

    @property
    def nbytes(self):
        return _lib.lib().mkrt_buffer_bytes(self._h)

    def ready_event(self):
        h = _p()
        _raise(_lib.lib().mkrt_buffer_ready_event(self._h, ctypes.byref(h)))
        return Event(h.value)

    def to_numpy(self):
        """Wait for the producer and copy to host (bf16 comes back as uint16 bits)."""
        out = np.empty(self.shape, dtype=_NP[self.type])
        _raise(_lib.lib().mkrt_buffer_to_host(self._h, out.ctypes.data_as(_p), out.nbytes, None))
        return out

    def close(self):
        if self._h:
            _lib.lib().mkrt_buffer_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Executable:
    """Compiled StableHLO (PJRT_LoadedExecutable)."""

    def __init__(self, handle, client):
        self._h = handle
        self._client = client

    @property
    def num_inputs(self):
        return _lib.lib().mkrt_executable_num_inputs(self._h)

    @property
    def num_outputs(self):
        return _lib.lib().mkrt_executable_num_outputs(self._h)

    @property
    def num_steps(self):
        return _lib.lib().mkrt_executable_num_steps(self._h)

    @property
    def plan(self):
        return _lib.lib().mkrt_executable_plan(self._h).decode()

    @property
    def fingerprint(self):
        """16 hex digits identifying the program (PJRT_Executable_Fingerprint)."""
        return _lib.lib().mkrt_executable_fingerprint(self._h).decode()

    def serialize(self):
        """Serialized form (PJRT_Executable_Serialize): bytes for Client.deserialize."""
        h = _p()
        _raise(_lib.lib().mkrt_executable_serialize(self._h, ctypes.byref(h)))
        return _take_serialized(h.value)

    def execute(self, inputs):
        """Run on borrowed input Buffers -> (list of new Buffers, completion Event)."""
        n_in = len(inputs)
        arr_in = (_p * max(1, n_in))(*[b._h for b in inputs])
        n_out = self.num_outputs
        arr_out = (_p * max(1, n_out))()
        done = _p()
        _raise(_lib.lib().mkrt_execute(self._h, arr_in, n_in, arr_out, ctypes.byref(done)))
        return [Buffer(arr_out[i], self._client) for i in range(n_out)], Event(done.value)

    def close(self):
        if self._h:
            _lib.lib().mkrt_executable_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Client:
    """One MI355X device (PJRT_Client)."""

    def __init__(self):
        h = _p()
        _raise(_lib.lib().mkrt_client_create(ctypes.byref(h)))
        self._h = h.value

    @property
    def platform_name(self):
        return _lib.lib().mkrt_client_platform_name(self._h).decode()

    def memory_stats(self):
        a, b = ctypes.c_int64(0), ctypes.c_int64(0)
        _raise(_lib.lib().mkrt_client_memory_stats(self._h, ctypes.byref(a), ctypes.byref(b)))
        return a.value, b.value

    def buffer(self, array, type=None):
        """Synchronous host-to-device copy of a numpy array."""
        a = np.ascontiguousarray(array)
        t = type if type is not None else _FROM_NP[a.dtype]
        dims = (ctypes.c_int64 * max(1, a.ndim))(*a.shape)
        h, ev = _p(), _p()
        _raise(_lib.lib().mkrt_buffer_from_host(self._h, a.ctypes.data_as(_p), t, dims, a.ndim,
                                                ctypes.byref(h), ctypes.byref(ev)))
        Event(ev.value).close()
        return Buffer(h.value, self)

    def error_buffer(self, code, message, type, shape):
        dims = (ctypes.c_int64 * max(1, len(shape)))(*shape)
        h = _p()
        _raise(_lib.lib().mkrt_buffer_create_error(self._h, code, message.encode(), type, dims,
                                                   len(shape), ctypes.byref(h)))
        return Buffer(h.value, self)

    def compile(self, text):
        data = text.encode() if isinstance(text, str) else bytes(text)
        h = _p()
        _raise(_lib.lib().mkrt_compile(self._h, data, len(data), b"mlir", ctypes.byref(h)))
        return Executable(h.value, self)

    def deserialize(self, blob):
        """Executable from Executable.serialize bytes (PJRT_Executable_DeserializeAndLoad)."""
        data = bytes(blob)
        h = _p()
        _raise(_lib.lib().mkrt_deserialize(self._h, data, len(data), ctypes.byref(h)))
        return Executable(h.value, self)

    def close(self):
        if self._h:
            _lib.lib().mkrt_client_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
