/*
 * mk_runtime.h -- the plugin's runtime API: client, device buffers,
 * executables compiled from StableHLO text, completion events and owned
 * errors, on one MI355X.
 *
 * This is the object model and call contract of the reference's PJRT C-API
 * layer, restated as plain C: every entry point mirrors one PJRT callback
 * (cited below) with the same argument meaning, ownership and error
 * behaviour.  The PJRT function table itself (GetPjrtApi,
 * src/pjrt_plugin/api/pjrt_api.cc:324-329) is a thin adapter over these
 * calls; it needs the exact pjrt_c_api.h of the jaxlib it is loaded into,
 * which this build does not have (see the integration notes).
 *
 * Conventions (from the reference, src/pjrt_plugin/api/):
 *   - calls return NULL on success or an owned mkrt_error (free it with
 *     mkrt_error_destroy), as PJRT callbacks return PJRT_Error*
 *     (pjrt_handles.h:75, pjrt_memory.cc:22-57);
 *   - error codes are PJRT_Error_Code values (absl status numbering);
 *   - element types are PJRT_Buffer_Type values;
 *   - objects are created by the runtime and destroyed by the caller;
 *     execute borrows its inputs and returns new output buffers, each
 *     owning its device memory, plus one completion event
 *     (pjrt_executable.cc:245-301);
 *   - destroying a buffer waits for the work producing it
 *     (core/mps_buffer.mm:656-662).
 */
#ifndef MK_RUNTIME_H_
#define MK_RUNTIME_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* PJRT_Error_Code (absl::StatusCode numbering). */
enum {
  MKRT_OK = 0,
  MKRT_CANCELLED = 1,
  MKRT_UNKNOWN = 2,
  MKRT_INVALID_ARGUMENT = 3,
  MKRT_DEADLINE_EXCEEDED = 4,
  MKRT_NOT_FOUND = 5,
  MKRT_ALREADY_EXISTS = 6,
  MKRT_PERMISSION_DENIED = 7,
  MKRT_RESOURCE_EXHAUSTED = 8,
  MKRT_FAILED_PRECONDITION = 9,
  MKRT_ABORTED = 10,
  MKRT_OUT_OF_RANGE = 11,
  MKRT_UNIMPLEMENTED = 12,
  MKRT_INTERNAL = 13,
  MKRT_UNAVAILABLE = 14
};

/* PJRT_Buffer_Type values for the types this plugin handles. */
enum {
  MKRT_PRED = 1,
  MKRT_S8 = 2,
  MKRT_S16 = 3,
  MKRT_S32 = 4,
  MKRT_S64 = 5,
  MKRT_U8 = 6,
  MKRT_U16 = 7,
  MKRT_U32 = 8,
  MKRT_U64 = 9,
  MKRT_F16 = 10,
  MKRT_F32 = 11,
  MKRT_F64 = 12,
  MKRT_BF16 = 13
};

typedef struct mkrt_error mkrt_error;
typedef struct mkrt_client mkrt_client;
typedef struct mkrt_buffer mkrt_buffer;
typedef struct mkrt_executable mkrt_executable;
typedef struct mkrt_event mkrt_event;

/* Errors (PJRT_Error_Destroy / _Message / _GetCode, pjrt_memory.cc:59-104). */
void mkrt_error_destroy(mkrt_error* err);
const char* mkrt_error_message(const mkrt_error* err);
int mkrt_error_code(const mkrt_error* err);

/* Client (PJRT_Client_Create / _Destroy / _PlatformName,
 * pjrt_client.cc:34-82; platform name pjrt_api.cc:18).  One HIP device
 * (ordinal 0), one stream, a caching device allocator. */
mkrt_error* mkrt_client_create(mkrt_client** out);
void mkrt_client_destroy(mkrt_client* client);
const char* mkrt_client_platform_name(const mkrt_client* client);
/* PJRT_Device_MemoryStats (pjrt_device.cc:110-140). */
mkrt_error* mkrt_client_memory_stats(mkrt_client* client, int64_t* bytes_in_use, int64_t* bytes_limit);

/* Buffers (PJRT_Client_BufferFromHostBuffer pjrt_client.cc:254-293: a
 * synchronous copy whose done-with-host event is already ready;
 * PJRT_Buffer_ToHostBuffer pjrt_buffer.cc:217-234: waits for the producer). */
mkrt_error* mkrt_buffer_from_host(mkrt_client* client, const void* data, int type, const int64_t* dims,
                                  int ndims, mkrt_buffer** out, mkrt_event** done_with_host);
mkrt_error* mkrt_buffer_to_host(mkrt_buffer* buf, void* dst, int64_t dst_bytes, mkrt_event** done);
int mkrt_buffer_type(const mkrt_buffer* buf);
int mkrt_buffer_ndims(const mkrt_buffer* buf);
const int64_t* mkrt_buffer_dims(const mkrt_buffer* buf);
int64_t mkrt_buffer_bytes(const mkrt_buffer* buf);
/* PJRT_Buffer_ReadyEvent (pjrt_buffer.cc:241-247). */
mkrt_error* mkrt_buffer_ready_event(mkrt_buffer* buf, mkrt_event** out);
/* PJRT_Client_CreateErrorBuffer (pjrt_client.cc:362-386): a buffer whose
 * ready event carries the error; reading it returns that error. */
mkrt_error* mkrt_buffer_create_error(mkrt_client* client, int code, const char* message, int type,
                                     const int64_t* dims, int ndims, mkrt_buffer** out);
/* PJRT_Buffer_Destroy: waits for the producer, then returns the memory to
 * the client's allocator. */
void mkrt_buffer_destroy(mkrt_buffer* buf);

/* PJRT_Client_BufferFromHostBuffer with byte strides (pjrt_client.cc:254-293,
 * core/mps_client.mm:133-176): one byte stride per dimension; a non-dense
 * host array is gathered into row-major order before the upload.  NULL
 * strides (or num_strides 0) mean dense row-major. */
mkrt_error* mkrt_buffer_from_host_strided(mkrt_client* client, const void* data, int type, const int64_t* dims,
                                          int ndims, const int64_t* byte_strides, int num_strides,
                                          mkrt_buffer** out, mkrt_event** done_with_host);
/* PJRT_Buffer_CopyRawToHost (pjrt_buffer.cc:148-169): `size` bytes from
 * byte `offset` of the buffer's row-major storage; waits for the producer. */
mkrt_error* mkrt_buffer_copy_raw_to_host(mkrt_buffer* buf, void* dst, int64_t offset, int64_t size,
                                         mkrt_event** done);
/* PJRT_Client_CreateViewOfDeviceBuffer (pjrt_client.cc:295-332): a buffer
 * over device memory the caller owns; on destroy or delete the runtime
 * drains its stream and calls on_release(device_ptr, user) instead of
 * freeing (on_release may be NULL). */
typedef void (*mkrt_release_callback)(void* device_ptr, void* user);
mkrt_error* mkrt_buffer_create_view(mkrt_client* client, void* device_ptr, int type, const int64_t* dims,
                                    int ndims, mkrt_release_callback on_release, void* user, mkrt_buffer** out);
/* PJRT_Client_CreateUninitializedBuffer (pjrt_client.cc:334-360). */
mkrt_error* mkrt_buffer_create_uninitialized(mkrt_client* client, int type, const int64_t* dims, int ndims,
                                             mkrt_buffer** out);
/* PJRT_Buffer_CopyToDevice / _CopyToMemory (pjrt_buffer.cc:112-146): a new
 * buffer holding a device-side copy, ready when the copy has run. */
mkrt_error* mkrt_buffer_copy(mkrt_buffer* buf, mkrt_buffer** out);
/* PJRT_Buffer_Delete / _IsDeleted (pjrt_buffer.cc:100-110): the device memory
 * is released (after its producer), the handle stays valid; executing on or
 * reading a deleted buffer is an error. */
void mkrt_buffer_delete(mkrt_buffer* buf);
int mkrt_buffer_is_deleted(const mkrt_buffer* buf);
/* PJRT_Buffer_OpaqueDeviceMemoryDataPointer / _UnsafePointer: the device
 * address (NULL once deleted, or for an error buffer). */
void* mkrt_buffer_device_pointer(const mkrt_buffer* buf);

/* Compile (PJRT_Client_Compile, pjrt_client.cc:178-244).  `format` "mlir"
 * takes StableHLO as MLIR bytecode (the portable artifact jaxlib's PJRT
 * client sends, vhlo dialect) or in MLIR text form (as jax's
 * lowered.as_text() prints it);
 * unsupported ops fail here with a message listing them
 * (pjrt_client.cc:211-220).  The execution plan is built on the first
 * execute (core/mps_executable.mm:9152, BuildExecutionPlan :7627). */
mkrt_error* mkrt_compile(mkrt_client* client, const char* code, int64_t code_bytes, const char* format,
                         mkrt_executable** out);
/* Parse and plan only, without a device: the same compile-time support
 * check (unsupported ops fail with UNIMPLEMENTED listing them,
 * pjrt_client.cc:211-220), plus the plan trace written into plan_text
 * (truncated to plan_text_bytes, NUL-terminated) and the step count. */
mkrt_error* mkrt_compile_check(const char* code, int64_t code_bytes, const char* format, char* plan_text,
                               int64_t plan_text_bytes, int* num_steps);
/* MLIR bytecode (the portable artifact compile takes) as MLIR text, as the
 * reference's bytecodeToText does (core/stablehlo_parser.mm:597): written
 * into text (truncated to text_bytes, NUL-terminated); text_size receives
 * the full length.  Malformed bytes are INVALID_ARGUMENT, content outside
 * what the reader decodes UNIMPLEMENTED. */
mkrt_error* mkrt_bytecode_to_text(const char* data, int64_t size, char* text, int64_t text_bytes,
                                  int64_t* text_size);
int mkrt_executable_num_inputs(const mkrt_executable* exe);
int mkrt_executable_num_outputs(const mkrt_executable* exe);
/* Output signature (PJRT_Executable_OutputElementTypes / _OutputDimensions,
 * pjrt_executable.cc:94-125) and the program as MLIR text
 * (PJRT_Executable_OptimizedProgram, :127-158; a program compiled from
 * bytecode gives its decoded text, as the reference prints its module). */
int mkrt_executable_output_type(const mkrt_executable* exe, int i);
int mkrt_executable_output_ndims(const mkrt_executable* exe, int i);
const int64_t* mkrt_executable_output_dims(const mkrt_executable* exe, int i);
const char* mkrt_executable_program(const mkrt_executable* exe, int64_t* size);
/* Number of kernel launches per execute and a one-line-per-step plan
 * description ("" before the first execute) -- the plan trace. */
int mkrt_executable_num_steps(const mkrt_executable* exe);
const char* mkrt_executable_plan(const mkrt_executable* exe);
/* PJRT_LoadedExecutable_Execute (pjrt_executable.cc:245-301): inputs are
 * borrowed; `outputs` receives num_outputs new buffers; `done` (optional)
 * receives the completion event of the whole execution. */
mkrt_error* mkrt_execute(mkrt_executable* exe, mkrt_buffer* const* inputs, int num_inputs,
                         mkrt_buffer** outputs, mkrt_event** done);
void mkrt_executable_destroy(mkrt_executable* exe);

/* ------------------------------------------------------------------------
 * Serialization and the compile cache.
 *
 * mkrt_executable_serialize replaces PJRT_Executable_Serialize
 * (api/pjrt_executable.cc:169-187) and mkrt_deserialize replaces
 * PJRT_Executable_DeserializeAndLoad (:303-340).  The reference serializes
 * the program (a VHLO portable artifact, core/mps_executable.mm:7127-7143)
 * and recompiles it on load.  Here the serialized form carries the
 * StableHLO text plus the gfx950 code objects of the executable's fused
 * elementwise programs, so a deserialized executable compiles nothing on
 * its first execute.  Layout (little-endian):
 *   "MKEX" | u32 version (2) | u32 flags (0) | u64 tag bytes | tag |
 *   u64 program bytes | program | u32 code objects | per object:
 *   u64 source bytes | source | u64 code bytes | code
 * The tag names the hiprtc version and compile options of the code objects;
 * a deserialize under another tag recompiles the elementwise programs
 * instead of loading the embedded objects.
 * Errors as the reference's: empty or malformed data -> INVALID_ARGUMENT;
 * a program that does not compile -> its compile error.
 *
 * The elementwise code objects are also cached on disk, one file per
 * object under MK_CACHE_DIR (default $HOME/.cache/mi355x-mk), keyed by
 * source, compile options and hiprtc version; MK_DISABLE_CACHE_PERSIST=1
 * turns that off.  This is the counterpart of the reference's persisted
 * autotune cache (core/mps_executable.mm:3270-3420,
 * JAX_METALLIB_AUTOTUNE_CACHE_DIR / JAX_METALLIB_DISABLE_AUTOTUNE_CACHE_PERSIST).
 * ---------------------------------------------------------------------- */
typedef struct mkrt_serialized mkrt_serialized;
mkrt_error* mkrt_executable_serialize(const mkrt_executable* exe, mkrt_serialized** out);
/* The same from program text, without a client or device (parse, plan and
 * compile the elementwise programs). */
mkrt_error* mkrt_serialize_program(const char* code, int64_t code_bytes, const char* format,
                                   mkrt_serialized** out);
const void* mkrt_serialized_data(const mkrt_serialized* s);
int64_t mkrt_serialized_size(const mkrt_serialized* s);
void mkrt_serialized_destroy(mkrt_serialized* s);
mkrt_error* mkrt_deserialize(mkrt_client* client, const void* bytes, int64_t size, mkrt_executable** out);
/* Header and table check without a device: program size and code-object
 * count, or INVALID_ARGUMENT for malformed data. */
mkrt_error* mkrt_serialized_inspect(const void* bytes, int64_t size, int64_t* program_bytes,
                                    int* num_code_objects);
/* PJRT_Executable_Fingerprint (pjrt_executable.cc:189-196 returns one
 * constant string for every executable): here 16 hex digits of FNV-1a 64
 * over the program text, equal for equal programs. */
const char* mkrt_executable_fingerprint(const mkrt_executable* exe);
/* Process totals of the elementwise JIT: hiprtc compiles, disk-cache hits,
 * memory-cache hits. */
void mkrt_jit_cache_stats(int64_t* compiles, int64_t* disk_hits, int64_t* memory_hits);

/* Events (pjrt_event.cc, core/completion_event.h).  await waits at most
 * timeout_ms (< 0: the MK_COMPLETION_TIMEOUT_MS environment value, default
 * 30000) and returns DEADLINE_EXCEEDED when it elapses (the work is left
 * pending); a ready event with an error returns a copy of that error.
 * event_error before the event is ready returns FAILED_PRECONDITION
 * (pjrt_event.cc:32-44).  on_ready runs the callback once, on the
 * completing thread or inline when already ready (pjrt_event.cc:81-98); the
 * callback receives an owned error or NULL. */
typedef void (*mkrt_event_callback)(mkrt_error* err, void* user);
mkrt_error* mkrt_event_create(mkrt_event** out);
mkrt_error* mkrt_event_set(mkrt_event* ev, int code, const char* message);
int mkrt_event_is_ready(const mkrt_event* ev);
mkrt_error* mkrt_event_error(const mkrt_event* ev);
mkrt_error* mkrt_event_await(mkrt_event* ev, int64_t timeout_ms);
mkrt_error* mkrt_event_on_ready(mkrt_event* ev, mkrt_event_callback cb, void* user);
void mkrt_event_destroy(mkrt_event* ev);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif  /* MK_RUNTIME_H_ */
