// The PJRT C API of the plugin: GetPjrtApi and its function table
// (reference: src/pjrt_plugin/api/pjrt_api.cc:160-329), each callback a thin
// adapter over the runtime C-ABI (include/mk_runtime.h).  Built into
// libmk_pjrt.so, whose only exported symbol is GetPjrtApi; jaxlib's PJRT
// client dlopens it through the jax_plugins registration.
//
// Object model (the reference's, api/pjrt_*.cc):
//   PJRT_Client      one mkrt_client: one MI355X, one stream; one device,
//                    one memory ("device"), one topology
//   PJRT_Buffer      one mkrt_buffer (owns or views device memory)
//   PJRT_Event       one mkrt_event
//   PJRT_Executable  a shared handle on one mkrt_executable; every
//                    LoadedExecutable_GetExecutable returns a new handle the
//                    caller destroys, so repeated calls never double-free
//   PJRT_Error       a heap object whose first member is the static
//                    function table (API >= 0.107 layout)
// Every callback checks its arguments' struct_size against the prefix it
// reads and returns INVALID_ARGUMENT for a null or short argument struct.
#include <stdio.h>
#include <string.h>

#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "mk_runtime.h"
#include "pjrt_c_api_mi355x.h"

namespace {

constexpr char kPlatformName[] = "mi355x";
constexpr char kPlatformVersion[] = "mi355x-pjrt 0.2 (gfx950, HIP)";
constexpr char kDeviceKind[] = "AMD Instinct MI355X";
constexpr char kMemoryKind[] = "device";

// ---------------------------------------------------------------- errors

struct ErrorImpl : PJRT_Error {
  PJRT_Error_Code code;
  std::string message;
};

void error_destroy(PJRT_Error* e) { delete static_cast<ErrorImpl*>(e); }
void error_message(const PJRT_Error* e, const char** m, size_t* n) {
  const ErrorImpl* x = static_cast<const ErrorImpl*>(e);
  *m = x->message.c_str();
  *n = x->message.size();
}
PJRT_Error_Code error_code(const PJRT_Error* e) { return static_cast<const ErrorImpl*>(e)->code; }
void error_payloads(const PJRT_Error*, PJRT_Error_PayloadVisitor, void*) {}  // no payloads are attached

const PJRT_Error_FunctionTable kErrorTable = {PJRT_Error_FunctionTable_STRUCT_SIZE,
                                              PJRT_Error_STRUCT_SIZE,
                                              nullptr,
                                              error_destroy,
                                              error_message,
                                              error_code,
                                              error_payloads};

PJRT_Error* make_error(PJRT_Error_Code code, const std::string& msg) {
  ErrorImpl* e = new ErrorImpl;
  e->vtable = &kErrorTable;
  e->code = code;
  e->message = msg;
  return e;
}

// An owned mkrt_error becomes an owned PJRT_Error (the codes share the absl
// numbering); NULL stays NULL.
PJRT_Error* take(mkrt_error* e) {
  if (!e) return nullptr;
  PJRT_Error* p = make_error(static_cast<PJRT_Error_Code>(mkrt_error_code(e)), mkrt_error_message(e));
  mkrt_error_destroy(e);
  return p;
}

#define CHECK_ARGS(args, Type)                                                                    \
  do {                                                                                            \
    if (!(args) || (args)->struct_size < Type##_STRUCT_SIZE)                                      \
      return make_error(PJRT_Error_Code_INVALID_ARGUMENT,                                         \
                        std::string(#Type ": null argument struct or struct_size below ") +      \
                            std::to_string((size_t)Type##_STRUCT_SIZE));                          \
  } while (0)

// --------------------------------------------------------- handle types

struct MemoryImpl : PJRT_Memory {
  PJRT_Client* client = nullptr;
  PJRT_Device* device = nullptr;
  std::mutex mu;
  std::map<const void*, std::pair<void*, void (*)(void*)>> user_data;
  ~MemoryImpl() {
    for (auto& kv : user_data)
      if (kv.second.second && kv.second.first) kv.second.second(kv.second.first);
  }
};

void* memory_get_user_data(PJRT_Memory* m, const void* key) {
  MemoryImpl* x = static_cast<MemoryImpl*>(m);
  std::lock_guard<std::mutex> g(x->mu);
  auto it = x->user_data.find(key);
  return it == x->user_data.end() ? nullptr : it->second.first;
}

void memory_set_user_data(PJRT_Memory* m, const void* key, void* data, void (*dtor)(void*)) {
  MemoryImpl* x = static_cast<MemoryImpl*>(m);
  std::pair<void*, void (*)(void*)> old{nullptr, nullptr};
  {
    std::lock_guard<std::mutex> g(x->mu);
    auto it = x->user_data.find(key);
    if (it != x->user_data.end()) {
      old = it->second;
      x->user_data.erase(it);
    }
    if (data) x->user_data[key] = {data, dtor};
  }
  // The previous value's destructor runs outside the lock (it may re-enter).
  if (old.first && old.second) old.second(old.first);
}

const PJRT_Memory_FunctionTable kMemoryTable = {PJRT_Memory_FunctionTable_STRUCT_SIZE, nullptr,
                                                PJRT_Memory_STRUCT_SIZE, memory_get_user_data,
                                                memory_set_user_data};

}  // namespace

struct PJRT_DeviceDescription {
  int id = 0;
};

struct PJRT_Device {
  PJRT_Client* client = nullptr;
  PJRT_DeviceDescription desc;
  PJRT_Memory* memory = nullptr;
};

struct PJRT_TopologyDescription {
  PJRT_Client* client = nullptr;  // null: created by TopologyDescription_Create
  PJRT_DeviceDescription desc;
  PJRT_DeviceDescription* descs[1] = {&desc};
};

struct PJRT_Client {
  mkrt_client* rt = nullptr;
  PJRT_Device device;
  MemoryImpl memory;
  PJRT_TopologyDescription topology;
  PJRT_Device* devices[1] = {&device};
  PJRT_Memory* memories[1] = {&memory};
};

struct PJRT_Buffer {
  PJRT_Client* client = nullptr;
  mkrt_buffer* b = nullptr;
  std::vector<int64_t> strides;  // dense row-major byte strides (GetMemoryLayout)
  int external_refs = 0;
};

namespace {
// One mkrt_event, destroyed with its last holder (the PJRT_Event handle and,
// for CopyRawToHostFuture, the pending future).
struct EventHolder {
  mkrt_event* ev = nullptr;
  explicit EventHolder(mkrt_event* e) : ev(e) {}
  ~EventHolder() { mkrt_event_destroy(ev); }
};
}  // namespace

struct PJRT_Event {
  std::shared_ptr<EventHolder> h;
  mkrt_event* ev() const { return h->ev; }
};

namespace {

struct ExeState {
  PJRT_Client* client = nullptr;
  mkrt_executable* exe = nullptr;
  std::string name;
  std::vector<PJRT_Buffer_Type> out_types;
  std::vector<int64_t> out_dims;
  std::vector<size_t> out_ranks;
  std::vector<const char*> out_kinds, in_kinds;
  std::vector<size_t> out_kind_sizes, in_kind_sizes;
  ~ExeState() { mkrt_executable_destroy(exe); }
};

}  // namespace

struct PJRT_Executable {
  std::shared_ptr<ExeState> st;
};

struct PJRT_LoadedExecutable {
  std::shared_ptr<ExeState> st;
  bool deleted = false;
};

namespace {

PJRT_Event* wrap_event(mkrt_event* e) {
  PJRT_Event* p = new PJRT_Event;
  p->h = std::make_shared<EventHolder>(e);
  return p;
}

// An event already complete, carrying `err` (owned) when non-null.
PJRT_Event* done_event(mkrt_error* err) {
  mkrt_event* e = nullptr;
  mkrt_event_create(&e);
  mkrt_event_set(e, err ? mkrt_error_code(err) : MKRT_OK, err ? mkrt_error_message(err) : "");
  if (err) mkrt_error_destroy(err);
  return wrap_event(e);
}

PJRT_Buffer* wrap_buffer(PJRT_Client* c, mkrt_buffer* b) {
  PJRT_Buffer* p = new PJRT_Buffer;
  p->client = c;
  p->b = b;
  const int nd = mkrt_buffer_ndims(b);
  const int64_t* d = mkrt_buffer_dims(b);
  p->strides.assign(nd, 0);
  const int64_t nel = nd ? 1 : 0;
  (void)nel;
  int64_t stride = mkrt_buffer_bytes(b);
  int64_t numel = 1;
  for (int i = 0; i < nd; ++i) numel *= d[i];
  stride = numel > 0 ? stride / numel : 0;  // element bytes
  for (int i = nd - 1; i >= 0; --i) {
    p->strides[i] = stride;
    stride *= d[i];
  }
  return p;
}

// A device layout the runtime can hold: absent, or dense row-major given as
// strides or as a tiled layout with descending minor_to_major and no tiles.
bool row_major_layout(const PJRT_Buffer_MemoryLayout* l, const int64_t* dims, size_t nd, int64_t elem_bytes) {
  if (!l) return true;
  if (l->type == PJRT_Buffer_MemoryLayout_Type_Tiled) {
    if (l->tiled.num_tiles != 0) return false;
    if (l->tiled.minor_to_major_size != nd) return false;
    for (size_t i = 0; i < nd; ++i)
      if (l->tiled.minor_to_major[i] != (int64_t)(nd - 1 - i)) return false;
    return true;
  }
  if (l->strides.num_byte_strides != nd) return false;
  int64_t expect = elem_bytes;
  for (size_t i = nd; i-- > 0;) {
    if (dims[i] > 1 && l->strides.byte_strides[i] != expect) return false;
    expect *= dims[i];
  }
  return true;
}

int64_t elem_bytes(int t) {
  switch (t) {
    case PJRT_Buffer_Type_PRED: case PJRT_Buffer_Type_S8: case PJRT_Buffer_Type_U8: return 1;
    case PJRT_Buffer_Type_S16: case PJRT_Buffer_Type_U16: case PJRT_Buffer_Type_F16: case PJRT_Buffer_Type_BF16:
      return 2;
    case PJRT_Buffer_Type_S32: case PJRT_Buffer_Type_U32: case PJRT_Buffer_Type_F32: return 4;
    case PJRT_Buffer_Type_S64: case PJRT_Buffer_Type_U64: case PJRT_Buffer_Type_F64: return 8;
    default: return 0;
  }
}

std::string module_name(const char* text, int64_t n) {
  // "module @jit_f ..." -> "jit_f" (the executable's name, as jax names it).
  const std::string s(text, (size_t)(n > 4096 ? 4096 : n));
  const size_t m = s.find("module @");
  if (m == std::string::npos) return "main";
  size_t e = m + 8;
  while (e < s.size() && (isalnum((unsigned char)s[e]) || s[e] == '_' || s[e] == '.' || s[e] == '$')) ++e;
  return e > m + 8 ? s.substr(m + 8, e - (m + 8)) : std::string("main");
}

std::shared_ptr<ExeState> new_state(PJRT_Client* c, mkrt_executable* exe) {
  auto st = std::make_shared<ExeState>();
  st->client = c;
  st->exe = exe;
  int64_t n = 0;
  const char* text = mkrt_executable_program(exe, &n);
  st->name = module_name(text, n);
  const int no = mkrt_executable_num_outputs(exe);
  for (int i = 0; i < no; ++i) {
    st->out_types.push_back(static_cast<PJRT_Buffer_Type>(mkrt_executable_output_type(exe, i)));
    const int nd = mkrt_executable_output_ndims(exe, i);
    const int64_t* d = mkrt_executable_output_dims(exe, i);
    st->out_dims.insert(st->out_dims.end(), d, d + nd);
    st->out_ranks.push_back((size_t)nd);
    st->out_kinds.push_back(kMemoryKind);
    st->out_kind_sizes.push_back(sizeof(kMemoryKind) - 1);
  }
  const int ni = mkrt_executable_num_inputs(exe);
  st->in_kinds.assign(ni, kMemoryKind);
  st->in_kind_sizes.assign(ni, sizeof(kMemoryKind) - 1);
  return st;
}

PJRT_Error* load(PJRT_Client* c, mkrt_executable* exe, PJRT_LoadedExecutable** out) {
  PJRT_LoadedExecutable* le = new PJRT_LoadedExecutable;
  le->st = new_state(c, exe);
  *out = le;
  return nullptr;
}

// A DeviceAssignmentProto for one replica and one computation on device 0
// (proto/device_assignment.proto:19-27, the reference's serialized value at
// api/pjrt_executable.cc:358-378), in protobuf wire format:
//   field 1 replica_count = 1        08 01
//   field 2 computation_count = 1    10 01
//   field 3 computation_devices      1A 03  { field 1 replica_device_ids,
//                                             packed: 0A 01 00 }
const char kDeviceAssignment[] = {0x08, 0x01, 0x10, 0x01, 0x1A, 0x03, 0x0A, 0x01, 0x00};

struct SerializedBlob {
  std::string bytes;
};

// ------------------------------------------------------------- callbacks

void Error_Destroy(PJRT_Error_Destroy_Args* args) {
  if (!args || !args->error) return;
  args->error->vtable->destroy(args->error);
}

void Error_Message(PJRT_Error_Message_Args* args) {
  if (!args) return;
  args->message = nullptr;
  args->message_size = 0;
  if (args->error) args->error->vtable->message(args->error, &args->message, &args->message_size);
}

PJRT_Error* Error_GetCode(PJRT_Error_GetCode_Args* args) {
  CHECK_ARGS(args, PJRT_Error_GetCode_Args);
  args->code = args->error ? args->error->vtable->get_code(args->error) : PJRT_Error_Code_OK;
  return nullptr;
}

PJRT_Error* Error_ForEachPayload(PJRT_Error_ForEachPayload_Args* args) {
  CHECK_ARGS(args, PJRT_Error_ForEachPayload_Args);
  if (args->error) args->error->vtable->for_each_payload(args->error, args->visitor, args->user_arg);
  return nullptr;
}

PJRT_Error* Plugin_Initialize(PJRT_Plugin_Initialize_Args* args) {
  CHECK_ARGS(args, PJRT_Plugin_Initialize_Args);
  return nullptr;
}

PJRT_Error* Plugin_Attributes(PJRT_Plugin_Attributes_Args* args) {
  CHECK_ARGS(args, PJRT_Plugin_Attributes_Args);
  args->attributes = nullptr;
  args->num_attributes = 0;
  return nullptr;
}

// ----------------------------------------------------------------- events

PJRT_Error* Event_Destroy(PJRT_Event_Destroy_Args* args) {
  CHECK_ARGS(args, PJRT_Event_Destroy_Args);
  delete args->event;
  return nullptr;
}

PJRT_Error* Event_IsReady(PJRT_Event_IsReady_Args* args) {
  CHECK_ARGS(args, PJRT_Event_IsReady_Args);
  if (!args->event) return make_error(PJRT_Error_Code_INVALID_ARGUMENT, "Event_IsReady: null event");
  args->is_ready = mkrt_event_is_ready(args->event->ev()) != 0;
  return nullptr;
}

PJRT_Error* Event_Error(PJRT_Event_Error_Args* args) {
  CHECK_ARGS(args, PJRT_Event_Error_Args);
  if (!args->event) return make_error(PJRT_Error_Code_INVALID_ARGUMENT, "Event_Error: null event");
  return take(mkrt_event_error(args->event->ev()));
}

PJRT_Error* Event_Await(PJRT_Event_Await_Args* args) {
  CHECK_ARGS(args, PJRT_Event_Await_Args);
  if (!args->event) return make_error(PJRT_Error_Code_INVALID_ARGUMENT, "Event_Await: null event");
  return take(mkrt_event_await(args->event->ev(), -1));
}

struct OnReadyTrampoline {
  PJRT_Event_OnReadyCallback cb;
  void* user;
};

void on_ready_trampoline(mkrt_error* err, void* user) {
  OnReadyTrampoline* t = static_cast<OnReadyTrampoline*>(user);
  t->cb(take(err), t->user);
  delete t;
}

PJRT_Error* Event_OnReady(PJRT_Event_OnReady_Args* args) {
  CHECK_ARGS(args, PJRT_Event_OnReady_Args);
  if (!args->event || !args->callback)
    return make_error(PJRT_Error_Code_INVALID_ARGUMENT, "Event_OnReady: null event or callback");
  OnReadyTrampoline* t = new OnReadyTrampoline{args->callback, args->user_arg};
  mkrt_error* e = mkrt_event_on_ready(args->event->ev(), on_ready_trampoline, t);
  if (e) delete t;
  return take(e);
}

PJRT_Error* Event_Create(PJRT_Event_Create_Args* args) {
  CHECK_ARGS(args, PJRT_Event_Create_Args);
  mkrt_event* e = nullptr;
  if (PJRT_Error* err = take(mkrt_event_create(&e))) return err;
  args->event = wrap_event(e);
  return nullptr;
}

PJRT_Error* Event_Set(PJRT_Event_Set_Args* args) {
  CHECK_ARGS(args, PJRT_Event_Set_Args);
  if (!args->event) return make_error(PJRT_Error_Code_INVALID_ARGUMENT, "Event_Set: null event");
  const std::string msg(args->error_message ? args->error_message : "",
                        args->error_message ? args->error_message_size : 0);
  return take(mkrt_event_set(args->event->ev(), args->error_code, msg.c_str()));
}

// ----------------------------------------------------------------- client

PJRT_Error* Client_Create(PJRT_Client_Create_Args* args) {
  CHECK_ARGS(args, PJRT_Client_Create_Args);
  args->client = nullptr;
  mkrt_client* rt = nullptr;
  if (PJRT_Error* e = take(mkrt_client_create(&rt))) return e;
  PJRT_Client* c = new PJRT_Client;
  c->rt = rt;
  c->device.client = c;
  c->device.memory = &c->memory;
  c->memory.vtable = &kMemoryTable;
  c->memory.client = c;
  c->memory.device = &c->device;
  c->topology.client = c;
  args->client = c;
  return nullptr;
}

PJRT_Error* Client_Destroy(PJRT_Client_Destroy_Args* args) {
  CHECK_ARGS(args, PJRT_Client_Destroy_Args);
  if (args->client) {
    mkrt_client_destroy(args->client->rt);
    delete args->client;
  }
  return nullptr;
}

#define NEED_CLIENT(c, what) \
  if (!(c)) return make_error(PJRT_Error_Code_INVALID_ARGUMENT, what ": null client")

PJRT_Error* Client_PlatformName(PJRT_Client_PlatformName_Args* args) {
  CHECK_ARGS(args, PJRT_Client_PlatformName_Args);
  args->platform_name = kPlatformName;
  args->platform_name_size = sizeof(kPlatformName) - 1;
  return nullptr;
}

PJRT_Error* Client_ProcessIndex(PJRT_Client_ProcessIndex_Args* args) {
  CHECK_ARGS(args, PJRT_Client_ProcessIndex_Args);
  args->process_index = 0;
  return nullptr;
}

PJRT_Error* Client_PlatformVersion(PJRT_Client_PlatformVersion_Args* args) {
  CHECK_ARGS(args, PJRT_Client_PlatformVersion_Args);
  args->platform_version = kPlatformVersion;
  args->platform_version_size = sizeof(kPlatformVersion) - 1;
  return nullptr;
}

PJRT_Error* Client_TopologyDescription(PJRT_Client_TopologyDescription_Args* args) {
  CHECK_ARGS(args, PJRT_Client_TopologyDescription_Args);
  NEED_CLIENT(args->client, "Client_TopologyDescription");
  args->topology = &args->client->topology;
  return nullptr;
}

PJRT_Error* Client_Devices(PJRT_Client_Devices_Args* args) {
  CHECK_ARGS(args, PJRT_Client_Devices_Args);
  NEED_CLIENT(args->client, "Client_Devices");
  args->devices = args->client->devices;
  args->num_devices = 1;
  return nullptr;
}

PJRT_Error* Client_AddressableDevices(PJRT_Client_AddressableDevices_Args* args) {
  CHECK_ARGS(args, PJRT_Client_AddressableDevices_Args);
  NEED_CLIENT(args->client, "Client_AddressableDevices");
  args->addressable_devices = args->client->devices;
  args->num_addressable_devices = 1;
  return nullptr;
}

PJRT_Error* Client_LookupDevice(PJRT_Client_LookupDevice_Args* args) {
  CHECK_ARGS(args, PJRT_Client_LookupDevice_Args);
  NEED_CLIENT(args->client, "Client_LookupDevice");
  if (args->id != 0) {
    args->device = nullptr;
    return make_error(PJRT_Error_Code_INVALID_ARGUMENT,
                      "Client_LookupDevice: no device with id " + std::to_string(args->id) + " (one device, id 0)");
  }
  args->device = &args->client->device;
  return nullptr;
}

PJRT_Error* Client_LookupAddressableDevice(PJRT_Client_LookupAddressableDevice_Args* args) {
  CHECK_ARGS(args, PJRT_Client_LookupAddressableDevice_Args);
  NEED_CLIENT(args->client, "Client_LookupAddressableDevice");
  if (args->local_hardware_id != 0) {
    args->addressable_device = nullptr;
    return make_error(PJRT_Error_Code_INVALID_ARGUMENT, "Client_LookupAddressableDevice: no device with local id " +
                                                            std::to_string(args->local_hardware_id));
  }
  args->addressable_device = &args->client->device;
  return nullptr;
}

PJRT_Error* Client_AddressableMemories(PJRT_Client_AddressableMemories_Args* args) {
  CHECK_ARGS(args, PJRT_Client_AddressableMemories_Args);
  NEED_CLIENT(args->client, "Client_AddressableMemories");
  args->addressable_memories = args->client->memories;
  args->num_addressable_memories = 1;
  return nullptr;
}

// Program formats (api/pjrt_client.cc:195-201): "mlir" carries StableHLO as
// MLIR (the text form is read; VHLO bytecode fails with UNIMPLEMENTED
// naming the text form), "hlo" carries StableHLO text as well.
const char* runtime_format(const PJRT_Program* p, std::string* fmt) {
  fmt->assign(p->format ? p->format : "", p->format ? p->format_size : 0);
  if (*fmt == "mlir" || *fmt == "hlo" || *fmt == "hlo_with_config") return "mlir";
  return nullptr;
}

PJRT_Error* Client_Compile(PJRT_Client_Compile_Args* args) {
  CHECK_ARGS(args, PJRT_Client_Compile_Args);
  NEED_CLIENT(args->client, "Client_Compile");
  args->executable = nullptr;
  if (!args->program || (!args->program->code && args->program->code_size))
    return make_error(PJRT_Error_Code_INVALID_ARGUMENT, "Client_Compile: null program");
  std::string fmt;
  const char* rf = runtime_format(args->program, &fmt);
  if (!rf) return make_error(PJRT_Error_Code_INVALID_ARGUMENT, "Client_Compile: unknown program format '" + fmt + "'");
  // compile_options (a serialized CompileOptionsProto) carries nothing this
  // single-device plugin acts on; the reference ignores it too.
  mkrt_executable* exe = nullptr;
  if (PJRT_Error* e = take(mkrt_compile(args->client->rt, args->program->code, (int64_t)args->program->code_size, rf,
                                        &exe)))
    return e;
  return load(args->client, exe, &args->executable);
}

PJRT_Error* Client_DefaultDeviceAssignment(PJRT_Client_DefaultDeviceAssignment_Args* args) {
  CHECK_ARGS(args, PJRT_Client_DefaultDeviceAssignment_Args);
  if (args->num_replicas != 1 || args->num_partitions != 1)
    return make_error(PJRT_Error_Code_INVALID_ARGUMENT,
                      "DefaultDeviceAssignment: one device; asked for " + std::to_string(args->num_replicas) +
                          " replicas x " + std::to_string(args->num_partitions) + " partitions");
  if (!args->default_assignment || args->default_assignment_size < 1)
    return make_error(PJRT_Error_Code_INVALID_ARGUMENT, "DefaultDeviceAssignment: no room for the assignment");
  args->default_assignment[0] = 0;
  return nullptr;
}

PJRT_Error* Client_BufferFromHostBuffer(PJRT_Client_BufferFromHostBuffer_Args* args) {
  CHECK_ARGS(args, PJRT_Client_BufferFromHostBuffer_Args);
  NEED_CLIENT(args->client, "BufferFromHostBuffer");
  args->buffer = nullptr;
  args->done_with_host_buffer = nullptr;
  if (args->num_dims > 64 || (args->num_dims && !args->dims))
    return make_error(PJRT_Error_Code_INVALID_ARGUMENT, "BufferFromHostBuffer: bad dims");
  const int64_t eb = elem_bytes(args->type);
  if (!eb)
    return make_error(PJRT_Error_Code_UNIMPLEMENTED,
                      "BufferFromHostBuffer: element type " + std::to_string((int)args->type) + " is not supported");
  if (!row_major_layout(args->device_layout, args->dims, args->num_dims, eb))
    return make_error(PJRT_Error_Code_UNIMPLEMENTED, "BufferFromHostBuffer: only row-major device layouts");
  if (args->device && args->device != &args->client->device)
    return make_error(PJRT_Error_Code_INVALID_ARGUMENT, "BufferFromHostBuffer: device of another client");
  if (args->memory && args->memory != &args->client->memory)
    return make_error(PJRT_Error_Code_INVALID_ARGUMENT, "BufferFromHostBuffer: memory of another client");
  mkrt_buffer* b = nullptr;
  mkrt_event* done = nullptr;
  // Every host-buffer semantic is served by a synchronous copy: the host
  // array is no longer needed when the call returns.
  if (PJRT_Error* e = take(mkrt_buffer_from_host_strided(args->client->rt, args->data, args->type, args->dims,
                                                         (int)args->num_dims, args->byte_strides,
                                                         (int)args->num_byte_strides, &b, &done)))
    return e;
  args->buffer = wrap_buffer(args->client, b);
  args->done_with_host_buffer = wrap_event(done);
  return nullptr;
}

PJRT_Error* Client_CreateViewOfDeviceBuffer(PJRT_Client_CreateViewOfDeviceBuffer_Args* args) {
  CHECK_ARGS(args, PJRT_Client_CreateViewOfDeviceBuffer_Args);
  NEED_CLIENT(args->client, "CreateViewOfDeviceBuffer");
  args->buffer = nullptr;
  const int64_t eb = elem_bytes(args->element_type);
  if (!eb) return make_error(PJRT_Error_Code_UNIMPLEMENTED, "CreateViewOfDeviceBuffer: element type not supported");
  if (args->num_dims > 64 || (args->num_dims && !args->dims))
    return make_error(PJRT_Error_Code_INVALID_ARGUMENT, "CreateViewOfDeviceBuffer: bad dims");
  if (!row_major_layout(args->layout, args->dims, args->num_dims, eb))
    return make_error(PJRT_Error_Code_UNIMPLEMENTED, "CreateViewOfDeviceBuffer: only row-major layouts");
  mkrt_buffer* b = nullptr;
  if (PJRT_Error* e = take(mkrt_buffer_create_view(args->client->rt, args->device_buffer_ptr, args->element_type,
                                                   args->dims, (int)args->num_dims,
                                                   (mkrt_release_callback)args->on_delete_callback,
                                                   args->on_delete_callback_arg, &b)))
    return e;
  args->buffer = wrap_buffer(args->client, b);
  return nullptr;
}

PJRT_Error* Client_CreateUninitializedBuffer(PJRT_Client_CreateUninitializedBuffer_Args* args) {
  CHECK_ARGS(args, PJRT_Client_CreateUninitializedBuffer_Args);
  NEED_CLIENT(args->client, "CreateUninitializedBuffer");
  args->buffer = nullptr;
  const int64_t eb = elem_bytes(args->shape_element_type);
  if (!eb) return make_error(PJRT_Error_Code_UNIMPLEMENTED, "CreateUninitializedBuffer: element type not supported");
  if (args->shape_num_dims > 64 || (args->shape_num_dims && !args->shape_dims))
    return make_error(PJRT_Error_Code_INVALID_ARGUMENT, "CreateUninitializedBuffer: bad dims");
  if (!row_major_layout(args->shape_layout, args->shape_dims, args->shape_num_dims, eb))
    return make_error(PJRT_Error_Code_UNIMPLEMENTED, "CreateUninitializedBuffer: only row-major layouts");
  mkrt_buffer* b = nullptr;
  if (PJRT_Error* e = take(mkrt_buffer_create_uninitialized(args->client->rt, args->shape_element_type,
                                                            args->shape_dims, (int)args->shape_num_dims, &b)))
    return e;
  args->buffer = wrap_buffer(args->client, b);
  return nullptr;
}

PJRT_Error* Client_CreateErrorBuffer(PJRT_Client_CreateErrorBuffer_Args* args) {
  CHECK_ARGS(args, PJRT_Client_CreateErrorBuffer_Args);
  NEED_CLIENT(args->client, "CreateErrorBuffer");
  args->buffer = nullptr;
  if (args->shape_num_dims > 64 || (args->shape_num_dims && !args->shape_dims))
    return make_error(PJRT_Error_Code_INVALID_ARGUMENT, "CreateErrorBuffer: bad dims");
  const std::string msg(args->error_message ? args->error_message : "",
                        args->error_message ? args->error_message_size : 0);
  mkrt_buffer* b = nullptr;
  if (PJRT_Error* e = take(mkrt_buffer_create_error(args->client->rt, args->error_code, msg.c_str(),
                                                    args->shape_element_type, args->shape_dims,
                                                    (int)args->shape_num_dims, &b)))
    return e;
  args->buffer = wrap_buffer(args->client, b);
  return nullptr;
}

// -------------------------------------------------------- device metadata

PJRT_Error* DeviceDescription_Id(PJRT_DeviceDescription_Id_Args* args) {
  CHECK_ARGS(args, PJRT_DeviceDescription_Id_Args);
  args->id = args->device_description ? args->device_description->id : 0;
  return nullptr;
}

PJRT_Error* DeviceDescription_ProcessIndex(PJRT_DeviceDescription_ProcessIndex_Args* args) {
  CHECK_ARGS(args, PJRT_DeviceDescription_ProcessIndex_Args);
  args->process_index = 0;
  return nullptr;
}

PJRT_Error* DeviceDescription_Attributes(PJRT_DeviceDescription_Attributes_Args* args) {
  CHECK_ARGS(args, PJRT_DeviceDescription_Attributes_Args);
  args->num_attributes = 0;
  args->attributes = nullptr;
  return nullptr;
}

PJRT_Error* DeviceDescription_Kind(PJRT_DeviceDescription_Kind_Args* args) {
  CHECK_ARGS(args, PJRT_DeviceDescription_Kind_Args);
  args->device_kind = kDeviceKind;
  args->device_kind_size = sizeof(kDeviceKind) - 1;
  return nullptr;
}

PJRT_Error* DeviceDescription_DebugString(PJRT_DeviceDescription_DebugString_Args* args) {
  CHECK_ARGS(args, PJRT_DeviceDescription_DebugString_Args);
  static const char s[] = "MI355X:0";
  args->debug_string = s;
  args->debug_string_size = sizeof(s) - 1;
  return nullptr;
}

PJRT_Error* DeviceDescription_ToString(PJRT_DeviceDescription_ToString_Args* args) {
  CHECK_ARGS(args, PJRT_DeviceDescription_ToString_Args);
  static const char s[] = "MI355XDevice(id=0)";
  args->to_string = s;
  args->to_string_size = sizeof(s) - 1;
  return nullptr;
}

PJRT_Error* Device_GetDescription(PJRT_Device_GetDescription_Args* args) {
  CHECK_ARGS(args, PJRT_Device_GetDescription_Args);
  if (!args->device) return make_error(PJRT_Error_Code_INVALID_ARGUMENT, "Device_GetDescription: null device");
  args->device_description = &args->device->desc;
  return nullptr;
}

PJRT_Error* Device_IsAddressable(PJRT_Device_IsAddressable_Args* args) {
  CHECK_ARGS(args, PJRT_Device_IsAddressable_Args);
  args->is_addressable = true;
  return nullptr;
}

PJRT_Error* Device_LocalHardwareId(PJRT_Device_LocalHardwareId_Args* args) {
  CHECK_ARGS(args, PJRT_Device_LocalHardwareId_Args);
  args->local_hardware_id = 0;
  return nullptr;
}

PJRT_Error* Device_AddressableMemories(PJRT_Device_AddressableMemories_Args* args) {
  CHECK_ARGS(args, PJRT_Device_AddressableMemories_Args);
  if (!args->device) return make_error(PJRT_Error_Code_INVALID_ARGUMENT, "Device_AddressableMemories: null device");
  args->memories = args->device->client->memories;
  args->num_memories = 1;
  return nullptr;
}

PJRT_Error* Device_DefaultMemory(PJRT_Device_DefaultMemory_Args* args) {
  CHECK_ARGS(args, PJRT_Device_DefaultMemory_Args);
  if (!args->device) return make_error(PJRT_Error_Code_INVALID_ARGUMENT, "Device_DefaultMemory: null device");
  args->memory = args->device->memory;
  return nullptr;
}

PJRT_Error* Device_MemoryStats(PJRT_Device_MemoryStats_Args* args) {
  // Callers built against an older header pass the prefix up to
  // peak_pool_bytes_is_set (api/pjrt_device.cc:131-137).
  if (!args || args->struct_size < PJRT_STRUCT_SIZE(PJRT_Device_MemoryStats_Args, peak_pool_bytes_is_set))
    return make_error(PJRT_Error_Code_INVALID_ARGUMENT, "Device_MemoryStats: null or short argument struct");
  if (!args->device) return make_error(PJRT_Error_Code_INVALID_ARGUMENT, "Device_MemoryStats: null device");
  int64_t in_use = 0, limit = 0;
  if (PJRT_Error* e = take(mkrt_client_memory_stats(args->device->client->rt, &in_use, &limit))) return e;
  args->bytes_in_use = in_use;
  args->peak_bytes_in_use_is_set = false;
  args->num_allocs_is_set = false;
  args->largest_alloc_size_is_set = false;
  args->bytes_limit = limit;
  args->bytes_limit_is_set = true;
  args->bytes_reserved_is_set = false;
  args->peak_bytes_reserved_is_set = false;
  args->bytes_reservable_limit_is_set = false;
  args->largest_free_block_bytes_is_set = false;
  args->pool_bytes_is_set = false;
  args->peak_pool_bytes_is_set = false;
  if (args->struct_size >= PJRT_Device_MemoryStats_Args_STRUCT_SIZE) args->peak_allocated_bytes_is_set = false;
  return nullptr;
}

// ----------------------------------------------------------------- memory

PJRT_Error* Memory_Id(PJRT_Memory_Id_Args* args) {
  CHECK_ARGS(args, PJRT_Memory_Id_Args);
  args->id = 0;
  return nullptr;
}

PJRT_Error* Memory_Kind(PJRT_Memory_Kind_Args* args) {
  CHECK_ARGS(args, PJRT_Memory_Kind_Args);
  args->kind = kMemoryKind;
  args->kind_size = sizeof(kMemoryKind) - 1;
  return nullptr;
}

PJRT_Error* Memory_Kind_Id(PJRT_Memory_Kind_Id_Args* args) {
  CHECK_ARGS(args, PJRT_Memory_Kind_Id_Args);
  args->kind_id = 0;
  return nullptr;
}

PJRT_Error* Memory_DebugString(PJRT_Memory_DebugString_Args* args) {
  CHECK_ARGS(args, PJRT_Memory_DebugString_Args);
  static const char s[] = "MI355X HBM3E (device memory)";
  args->debug_string = s;
  args->debug_string_size = sizeof(s) - 1;
  return nullptr;
}

PJRT_Error* Memory_ToString(PJRT_Memory_ToString_Args* args) {
  CHECK_ARGS(args, PJRT_Memory_ToString_Args);
  static const char s[] = "MemorySpace(kind=device, id=0)";
  args->to_string = s;
  args->to_string_size = sizeof(s) - 1;
  return nullptr;
}

PJRT_Error* Memory_AddressableByDevices(PJRT_Memory_AddressableByDevices_Args* args) {
  CHECK_ARGS(args, PJRT_Memory_AddressableByDevices_Args);
  MemoryImpl* m = static_cast<MemoryImpl*>(args->memory);
  if (!m) return make_error(PJRT_Error_Code_INVALID_ARGUMENT, "Memory_AddressableByDevices: null memory");
  args->devices = m->client->devices;
  args->num_devices = 1;
  return nullptr;
}

// ------------------------------------------------------------- executables

#define NEED_EXE(x, what) \
  if (!(x) || !(x)->st) return make_error(PJRT_Error_Code_INVALID_ARGUMENT, what ": null executable")

PJRT_Error* Executable_Destroy(PJRT_Executable_Destroy_Args* args) {
  CHECK_ARGS(args, PJRT_Executable_Destroy_Args);
  delete args->executable;
  return nullptr;
}

PJRT_Error* Executable_Name(PJRT_Executable_Name_Args* args) {
  CHECK_ARGS(args, PJRT_Executable_Name_Args);
  NEED_EXE(args->executable, "Executable_Name");
  args->executable_name = args->executable->st->name.c_str();
  args->executable_name_size = args->executable->st->name.size();
  return nullptr;
}

PJRT_Error* Executable_NumReplicas(PJRT_Executable_NumReplicas_Args* args) {
  CHECK_ARGS(args, PJRT_Executable_NumReplicas_Args);
  args->num_replicas = 1;
  return nullptr;
}

PJRT_Error* Executable_NumPartitions(PJRT_Executable_NumPartitions_Args* args) {
  CHECK_ARGS(args, PJRT_Executable_NumPartitions_Args);
  args->num_partitions = 1;
  return nullptr;
}

PJRT_Error* Executable_NumOutputs(PJRT_Executable_NumOutputs_Args* args) {
  CHECK_ARGS(args, PJRT_Executable_NumOutputs_Args);
  NEED_EXE(args->executable, "Executable_NumOutputs");
  args->num_outputs = args->executable->st->out_types.size();
  return nullptr;
}

PJRT_Error* Executable_SizeOfGeneratedCodeInBytes(PJRT_Executable_SizeOfGeneratedCodeInBytes_Args* args) {
  CHECK_ARGS(args, PJRT_Executable_SizeOfGeneratedCodeInBytes_Args);
  args->size_in_bytes = 0;  // the kernels are precompiled into the library
  return nullptr;
}

PJRT_Error* Executable_GetCostAnalysis(PJRT_Executable_GetCostAnalysis_Args* args) {
  CHECK_ARGS(args, PJRT_Executable_GetCostAnalysis_Args);
  args->num_properties = 0;
  args->properties = nullptr;
  return nullptr;
}

PJRT_Error* Executable_OutputMemoryKinds(PJRT_Executable_OutputMemoryKinds_Args* args) {
  CHECK_ARGS(args, PJRT_Executable_OutputMemoryKinds_Args);
  NEED_EXE(args->executable, "Executable_OutputMemoryKinds");
  const ExeState& s = *args->executable->st;
  args->num_outputs = s.out_kinds.size();
  args->memory_kinds = s.out_kinds.data();
  args->memory_kind_sizes = s.out_kind_sizes.data();
  return nullptr;
}

PJRT_Error* Executable_ParameterMemoryKinds(PJRT_Executable_ParameterMemoryKinds_Args* args) {
  CHECK_ARGS(args, PJRT_Executable_ParameterMemoryKinds_Args);
  NEED_EXE(args->executable, "Executable_ParameterMemoryKinds");
  const ExeState& s = *args->executable->st;
  args->num_parameters = s.in_kinds.size();
  args->memory_kinds = s.in_kinds.data();
  args->memory_kind_sizes = s.in_kind_sizes.data();
  return nullptr;
}

PJRT_Error* Executable_OutputElementTypes(PJRT_Executable_OutputElementTypes_Args* args) {
  CHECK_ARGS(args, PJRT_Executable_OutputElementTypes_Args);
  NEED_EXE(args->executable, "Executable_OutputElementTypes");
  ExeState& s = *args->executable->st;
  args->output_types = s.out_types.data();
  args->num_output_types = s.out_types.size();
  return nullptr;
}

PJRT_Error* Executable_OutputDimensions(PJRT_Executable_OutputDimensions_Args* args) {
  CHECK_ARGS(args, PJRT_Executable_OutputDimensions_Args);
  NEED_EXE(args->executable, "Executable_OutputDimensions");
  const ExeState& s = *args->executable->st;
  args->num_outputs = s.out_ranks.size();
  args->dims = s.out_dims.data();
  args->dim_sizes = s.out_ranks.data();
  return nullptr;
}

PJRT_Error* Executable_OptimizedProgram(PJRT_Executable_OptimizedProgram_Args* args) {
  CHECK_ARGS(args, PJRT_Executable_OptimizedProgram_Args);
  NEED_EXE(args->executable, "Executable_OptimizedProgram");
  if (!args->program) return make_error(PJRT_Error_Code_INVALID_ARGUMENT, "OptimizedProgram: null program");
  if (args->program->struct_size < PJRT_Program_STRUCT_SIZE)
    return make_error(PJRT_Error_Code_INVALID_ARGUMENT, "OptimizedProgram: short PJRT_Program");
  int64_t n = 0;
  const char* text = mkrt_executable_program(args->executable->st->exe, &n);
  static const char fmt[] = "mlir";
  args->program->format = fmt;
  args->program->format_size = sizeof(fmt) - 1;
  // A null code pointer asks for the size; otherwise code_size is the room.
  if (!args->program->code) {
    args->program->code_size = (size_t)n;
    return nullptr;
  }
  if (args->program->code_size < (size_t)n)
    return make_error(PJRT_Error_Code_INVALID_ARGUMENT, "OptimizedProgram: code buffer of " +
                                                            std::to_string(args->program->code_size) +
                                                            " bytes, program needs " + std::to_string(n));
  memcpy(args->program->code, text, (size_t)n);
  args->program->code_size = (size_t)n;
  return nullptr;
}

void delete_serialized(PJRT_SerializedExecutable* s) { delete reinterpret_cast<SerializedBlob*>(s); }

PJRT_Error* Executable_Serialize(PJRT_Executable_Serialize_Args* args) {
  CHECK_ARGS(args, PJRT_Executable_Serialize_Args);
  NEED_EXE(args->executable, "Executable_Serialize");
  mkrt_serialized* ser = nullptr;
  if (PJRT_Error* e = take(mkrt_executable_serialize(args->executable->st->exe, &ser))) return e;
  SerializedBlob* blob = new SerializedBlob;
  blob->bytes.assign(static_cast<const char*>(mkrt_serialized_data(ser)), (size_t)mkrt_serialized_size(ser));
  mkrt_serialized_destroy(ser);
  args->serialized_bytes = blob->bytes.data();
  args->serialized_bytes_size = blob->bytes.size();
  args->serialized_executable = reinterpret_cast<PJRT_SerializedExecutable*>(blob);
  args->serialized_executable_deleter = delete_serialized;
  return nullptr;
}

PJRT_Error* Executable_Fingerprint(PJRT_Executable_Fingerprint_Args* args) {
  CHECK_ARGS(args, PJRT_Executable_Fingerprint_Args);
  NEED_EXE(args->executable, "Executable_Fingerprint");
  const char* fp = mkrt_executable_fingerprint(args->executable->st->exe);
  args->executable_fingerprint = fp;
  args->executable_fingerprint_size = strlen(fp);
  return nullptr;
}

PJRT_Error* Executable_DeserializeAndLoad(PJRT_Executable_DeserializeAndLoad_Args* args) {
  CHECK_ARGS(args, PJRT_Executable_DeserializeAndLoad_Args);
  NEED_CLIENT(args->client, "DeserializeAndLoad");
  args->loaded_executable = nullptr;
  if (!args->serialized_executable || args->serialized_executable_size == 0)
    return make_error(PJRT_Error_Code_INVALID_ARGUMENT, "DeserializeAndLoad: empty serialized data");
  mkrt_executable* exe = nullptr;
  if (PJRT_Error* e = take(mkrt_deserialize(args->client->rt, args->serialized_executable,
                                            (int64_t)args->serialized_executable_size, &exe)))
    return e;
  return load(args->client, exe, &args->loaded_executable);
}

PJRT_Error* LoadedExecutable_Destroy(PJRT_LoadedExecutable_Destroy_Args* args) {
  CHECK_ARGS(args, PJRT_LoadedExecutable_Destroy_Args);
  delete args->executable;
  return nullptr;
}

PJRT_Error* LoadedExecutable_GetExecutable(PJRT_LoadedExecutable_GetExecutable_Args* args) {
  CHECK_ARGS(args, PJRT_LoadedExecutable_GetExecutable_Args);
  NEED_EXE(args->loaded_executable, "LoadedExecutable_GetExecutable");
  PJRT_Executable* e = new PJRT_Executable;
  e->st = args->loaded_executable->st;
  args->executable = e;
  return nullptr;
}

PJRT_Error* LoadedExecutable_AddressableDevices(PJRT_LoadedExecutable_AddressableDevices_Args* args) {
  CHECK_ARGS(args, PJRT_LoadedExecutable_AddressableDevices_Args);
  NEED_EXE(args->executable, "LoadedExecutable_AddressableDevices");
  args->addressable_devices = args->executable->st->client->devices;
  args->num_addressable_devices = 1;
  return nullptr;
}

PJRT_Error* LoadedExecutable_Delete(PJRT_LoadedExecutable_Delete_Args* args) {
  CHECK_ARGS(args, PJRT_LoadedExecutable_Delete_Args);
  NEED_EXE(args->executable, "LoadedExecutable_Delete");
  args->executable->deleted = true;
  return nullptr;
}

PJRT_Error* LoadedExecutable_IsDeleted(PJRT_LoadedExecutable_IsDeleted_Args* args) {
  CHECK_ARGS(args, PJRT_LoadedExecutable_IsDeleted_Args);
  NEED_EXE(args->executable, "LoadedExecutable_IsDeleted");
  args->is_deleted = args->executable->deleted;
  return nullptr;
}

PJRT_Error* LoadedExecutable_Fingerprint(PJRT_LoadedExecutable_Fingerprint_Args* args) {
  CHECK_ARGS(args, PJRT_LoadedExecutable_Fingerprint_Args);
  NEED_EXE(args->executable, "LoadedExecutable_Fingerprint");
  const char* fp = mkrt_executable_fingerprint(args->executable->st->exe);
  args->executable_fingerprint = fp;
  args->executable_fingerprint_size = strlen(fp);
  return nullptr;
}

void delete_assignment(PJRT_DeviceAssignmentSerialized* d) { delete reinterpret_cast<SerializedBlob*>(d); }

PJRT_Error* LoadedExecutable_GetDeviceAssignment(PJRT_LoadedExecutable_GetDeviceAssignment_Args* args) {
  CHECK_ARGS(args, PJRT_LoadedExecutable_GetDeviceAssignment_Args);
  SerializedBlob* blob = new SerializedBlob;
  blob->bytes.assign(kDeviceAssignment, sizeof(kDeviceAssignment));
  args->serialized_bytes = blob->bytes.data();
  args->serialized_bytes_size = blob->bytes.size();
  args->serialized_device_assignment = reinterpret_cast<PJRT_DeviceAssignmentSerialized*>(blob);
  args->serialized_device_assignment_deleter = delete_assignment;
  return nullptr;
}

// Inputs are borrowed; every output is a new buffer owning its memory and
// device_complete_events[0] fires when the whole execution has run
// (api/pjrt_executable.cc:245-301).  One device: argument_lists[0] only.
PJRT_Error* LoadedExecutable_Execute(PJRT_LoadedExecutable_Execute_Args* args) {
  CHECK_ARGS(args, PJRT_LoadedExecutable_Execute_Args);
  NEED_EXE(args->executable, "Execute");
  if (args->executable->deleted)
    return make_error(PJRT_Error_Code_FAILED_PRECONDITION, "Execute: the executable has been deleted");
  if (args->num_devices != 1)
    return make_error(PJRT_Error_Code_INVALID_ARGUMENT,
                      "Execute: one device; asked for " + std::to_string(args->num_devices));
  if (!args->output_lists || !args->output_lists[0] || (args->num_args && (!args->argument_lists ||
                                                                           !args->argument_lists[0])))
    return make_error(PJRT_Error_Code_INVALID_ARGUMENT, "Execute: null argument or output list");
  ExeState& s = *args->executable->st;
  std::vector<mkrt_buffer*> in(args->num_args, nullptr);
  for (size_t i = 0; i < args->num_args; ++i) {
    PJRT_Buffer* b = args->argument_lists[0][i];
    if (!b) return make_error(PJRT_Error_Code_INVALID_ARGUMENT, "Execute: argument " + std::to_string(i) + " is null");
    in[i] = b->b;
  }
  std::vector<mkrt_buffer*> out(s.out_types.size(), nullptr);
  mkrt_event* done = nullptr;
  if (PJRT_Error* e = take(mkrt_execute(s.exe, in.data(), (int)in.size(), out.data(),
                                        args->device_complete_events ? &done : nullptr)))
    return e;
  for (size_t r = 0; r < out.size(); ++r) args->output_lists[0][r] = wrap_buffer(s.client, out[r]);
  if (args->device_complete_events) args->device_complete_events[0] = wrap_event(done);
  return nullptr;
}

// ---------------------------------------------------------------- buffers

#define NEED_BUF(x, what) \
  if (!(x) || !(x)->b) return make_error(PJRT_Error_Code_INVALID_ARGUMENT, what ": null buffer")

PJRT_Error* Buffer_Destroy(PJRT_Buffer_Destroy_Args* args) {
  CHECK_ARGS(args, PJRT_Buffer_Destroy_Args);
  if (args->buffer) {
    mkrt_buffer_destroy(args->buffer->b);
    delete args->buffer;
  }
  return nullptr;
}

PJRT_Error* Buffer_ElementType(PJRT_Buffer_ElementType_Args* args) {
  CHECK_ARGS(args, PJRT_Buffer_ElementType_Args);
  NEED_BUF(args->buffer, "Buffer_ElementType");
  args->type = static_cast<PJRT_Buffer_Type>(mkrt_buffer_type(args->buffer->b));
  return nullptr;
}

PJRT_Error* Buffer_Dimensions(PJRT_Buffer_Dimensions_Args* args) {
  CHECK_ARGS(args, PJRT_Buffer_Dimensions_Args);
  NEED_BUF(args->buffer, "Buffer_Dimensions");
  args->dims = mkrt_buffer_dims(args->buffer->b);
  args->num_dims = (size_t)mkrt_buffer_ndims(args->buffer->b);
  return nullptr;
}

PJRT_Error* Buffer_UnpaddedDimensions(PJRT_Buffer_UnpaddedDimensions_Args* args) {
  CHECK_ARGS(args, PJRT_Buffer_UnpaddedDimensions_Args);
  NEED_BUF(args->buffer, "Buffer_UnpaddedDimensions");
  args->unpadded_dims = mkrt_buffer_dims(args->buffer->b);
  args->num_dims = (size_t)mkrt_buffer_ndims(args->buffer->b);
  return nullptr;
}

PJRT_Error* Buffer_DynamicDimensionIndices(PJRT_Buffer_DynamicDimensionIndices_Args* args) {
  CHECK_ARGS(args, PJRT_Buffer_DynamicDimensionIndices_Args);
  args->dynamic_dim_indices = nullptr;
  args->num_dynamic_dims = 0;
  return nullptr;
}

PJRT_Error* Buffer_GetMemoryLayout(PJRT_Buffer_GetMemoryLayout_Args* args) {
  CHECK_ARGS(args, PJRT_Buffer_GetMemoryLayout_Args);
  NEED_BUF(args->buffer, "Buffer_GetMemoryLayout");
  memset(&args->layout, 0, sizeof(args->layout));
  args->layout.struct_size = PJRT_Buffer_MemoryLayout_STRUCT_SIZE;
  args->layout.type = PJRT_Buffer_MemoryLayout_Type_Strides;
  args->layout.strides.struct_size = PJRT_Buffer_MemoryLayout_Strides_STRUCT_SIZE;
  args->layout.strides.byte_strides = args->buffer->strides.data();
  args->layout.strides.num_byte_strides = args->buffer->strides.size();
  return nullptr;
}

PJRT_Error* Buffer_OnDeviceSizeInBytes(PJRT_Buffer_OnDeviceSizeInBytes_Args* args) {
  CHECK_ARGS(args, PJRT_Buffer_OnDeviceSizeInBytes_Args);
  NEED_BUF(args->buffer, "Buffer_OnDeviceSizeInBytes");
  args->on_device_size_in_bytes = (size_t)mkrt_buffer_bytes(args->buffer->b);
  return nullptr;
}

PJRT_Error* Buffer_Device(PJRT_Buffer_Device_Args* args) {
  CHECK_ARGS(args, PJRT_Buffer_Device_Args);
  NEED_BUF(args->buffer, "Buffer_Device");
  args->device = &args->buffer->client->device;
  return nullptr;
}

PJRT_Error* Buffer_Memory(PJRT_Buffer_Memory_Args* args) {
  CHECK_ARGS(args, PJRT_Buffer_Memory_Args);
  NEED_BUF(args->buffer, "Buffer_Memory");
  args->memory = &args->buffer->client->memory;
  return nullptr;
}

PJRT_Error* Buffer_Delete(PJRT_Buffer_Delete_Args* args) {
  CHECK_ARGS(args, PJRT_Buffer_Delete_Args);
  NEED_BUF(args->buffer, "Buffer_Delete");
  mkrt_buffer_delete(args->buffer->b);
  return nullptr;
}

PJRT_Error* Buffer_IsDeleted(PJRT_Buffer_IsDeleted_Args* args) {
  CHECK_ARGS(args, PJRT_Buffer_IsDeleted_Args);
  NEED_BUF(args->buffer, "Buffer_IsDeleted");
  args->is_deleted = mkrt_buffer_is_deleted(args->buffer->b) != 0;
  return nullptr;
}

PJRT_Error* Buffer_CopyToDevice(PJRT_Buffer_CopyToDevice_Args* args) {
  CHECK_ARGS(args, PJRT_Buffer_CopyToDevice_Args);
  NEED_BUF(args->buffer, "Buffer_CopyToDevice");
  args->dst_buffer = nullptr;
  if (args->dst_device && args->dst_device != &args->buffer->client->device)
    return make_error(PJRT_Error_Code_INVALID_ARGUMENT, "CopyToDevice: device of another client");
  mkrt_buffer* b = nullptr;
  if (PJRT_Error* e = take(mkrt_buffer_copy(args->buffer->b, &b))) return e;
  args->dst_buffer = wrap_buffer(args->buffer->client, b);
  return nullptr;
}

PJRT_Error* Buffer_CopyToMemory(PJRT_Buffer_CopyToMemory_Args* args) {
  CHECK_ARGS(args, PJRT_Buffer_CopyToMemory_Args);
  NEED_BUF(args->buffer, "Buffer_CopyToMemory");
  args->dst_buffer = nullptr;
  if (args->dst_memory && args->dst_memory != &args->buffer->client->memory)
    return make_error(PJRT_Error_Code_INVALID_ARGUMENT, "CopyToMemory: memory of another client");
  mkrt_buffer* b = nullptr;
  if (PJRT_Error* e = take(mkrt_buffer_copy(args->buffer->b, &b))) return e;
  args->dst_buffer = wrap_buffer(args->buffer->client, b);
  return nullptr;
}

// The copy runs when called, after the producer (a ready event is
// returned); a failed copy or a producer error is reported on the event, as
// the reference does (api/pjrt_buffer.cc:217-234).  dst == NULL asks for the
// size in dst_size.
PJRT_Error* Buffer_ToHostBuffer(PJRT_Buffer_ToHostBuffer_Args* args) {
  CHECK_ARGS(args, PJRT_Buffer_ToHostBuffer_Args);
  NEED_BUF(args->src, "Buffer_ToHostBuffer");
  args->event = nullptr;
  mkrt_buffer* b = args->src->b;
  const int64_t bytes = mkrt_buffer_bytes(b);
  if (!row_major_layout(args->host_layout, mkrt_buffer_dims(b), (size_t)mkrt_buffer_ndims(b),
                        elem_bytes(mkrt_buffer_type(b))))
    return make_error(PJRT_Error_Code_UNIMPLEMENTED, "ToHostBuffer: only row-major host layouts");
  if (!args->dst) {
    args->dst_size = (size_t)bytes;
    return nullptr;
  }
  mkrt_event* done = nullptr;
  mkrt_error* e = mkrt_buffer_to_host(b, args->dst, (int64_t)args->dst_size, &done);
  if (e && mkrt_error_code(e) == MKRT_INVALID_ARGUMENT) return take(e);  // caller error: returned, not deferred
  args->event = e ? done_event(e) : wrap_event(done);
  return nullptr;
}

PJRT_Error* Buffer_CopyRawToHost(PJRT_Buffer_CopyRawToHost_Args* args) {
  CHECK_ARGS(args, PJRT_Buffer_CopyRawToHost_Args);
  NEED_BUF(args->buffer, "Buffer_CopyRawToHost");
  args->event = nullptr;
  if (!args->dst) return make_error(PJRT_Error_Code_INVALID_ARGUMENT, "CopyRawToHost: null destination");
  mkrt_event* done = nullptr;
  mkrt_error* e = mkrt_buffer_copy_raw_to_host(args->buffer->b, args->dst, args->offset, args->transfer_size, &done);
  if (e && mkrt_error_code(e) == MKRT_INVALID_ARGUMENT) return take(e);
  args->event = e ? done_event(e) : wrap_event(done);
  return nullptr;
}

struct RawFuture {
  mkrt_buffer* buffer;
  int64_t offset, size;
  std::shared_ptr<EventHolder> ev;
};

// Called by the consumer once it has a destination (or an error): copies and
// completes the event handed out by Buffer_CopyRawToHostFuture.
void raw_future_ready(PJRT_Buffer_CopyRawToHostFuture_Callback_Args* cb) {
  if (!cb || !cb->callback_data) return;
  RawFuture* f = static_cast<RawFuture*>(cb->callback_data);
  if (cb->error_code != PJRT_Error_Code_OK) {
    const std::string msg(cb->error_message ? cb->error_message : "", cb->error_message ? cb->error_message_size : 0);
    mkrt_event_set(f->ev->ev, cb->error_code, msg.c_str());
  } else if (!cb->dst) {
    mkrt_event_set(f->ev->ev, MKRT_INVALID_ARGUMENT, "CopyRawToHostFuture: null destination");
  } else {
    mkrt_event* done = nullptr;
    mkrt_error* e = mkrt_buffer_copy_raw_to_host(f->buffer, cb->dst, f->offset, f->size, &done);
    if (e) {
      mkrt_event_set(f->ev->ev, mkrt_error_code(e), mkrt_error_message(e));
      mkrt_error_destroy(e);
    } else {
      mkrt_event_destroy(done);
      mkrt_event_set(f->ev->ev, MKRT_OK, "");
    }
  }
  delete f;
}

// The destination arrives later through future_ready_callback
// (api/pjrt_buffer.cc:171-215); the returned event completes then.  The
// buffer must outlive the callback, as in the reference.
PJRT_Error* Buffer_CopyRawToHostFuture(PJRT_Buffer_CopyRawToHostFuture_Args* args) {
  CHECK_ARGS(args, PJRT_Buffer_CopyRawToHostFuture_Args);
  NEED_BUF(args->buffer, "CopyRawToHostFuture");
  args->event = nullptr;
  mkrt_event* ev = nullptr;
  if (PJRT_Error* e = take(mkrt_event_create(&ev))) return e;
  PJRT_Event* pe = wrap_event(ev);
  args->event = pe;
  args->callback_data = new RawFuture{args->buffer->b, args->offset, args->transfer_size, pe->h};
  args->future_ready_callback = raw_future_ready;
  return nullptr;
}

PJRT_Error* Buffer_IsOnCpu(PJRT_Buffer_IsOnCpu_Args* args) {
  CHECK_ARGS(args, PJRT_Buffer_IsOnCpu_Args);
  args->is_on_cpu = false;
  return nullptr;
}

PJRT_Error* Buffer_ReadyEvent(PJRT_Buffer_ReadyEvent_Args* args) {
  CHECK_ARGS(args, PJRT_Buffer_ReadyEvent_Args);
  NEED_BUF(args->buffer, "Buffer_ReadyEvent");
  mkrt_event* e = nullptr;
  if (PJRT_Error* err = take(mkrt_buffer_ready_event(args->buffer->b, &e))) return err;
  args->event = wrap_event(e);
  return nullptr;
}

PJRT_Error* Buffer_UnsafePointer(PJRT_Buffer_UnsafePointer_Args* args) {
  CHECK_ARGS(args, PJRT_Buffer_UnsafePointer_Args);
  NEED_BUF(args->buffer, "Buffer_UnsafePointer");
  args->buffer_pointer = (uintptr_t)mkrt_buffer_device_pointer(args->buffer->b);
  return nullptr;
}

PJRT_Error* Buffer_IncreaseExternalReferenceCount(PJRT_Buffer_IncreaseExternalReferenceCount_Args* args) {
  CHECK_ARGS(args, PJRT_Buffer_IncreaseExternalReferenceCount_Args);
  NEED_BUF(args->buffer, "IncreaseExternalReferenceCount");
  ++args->buffer->external_refs;
  return nullptr;
}

PJRT_Error* Buffer_DecreaseExternalReferenceCount(PJRT_Buffer_DecreaseExternalReferenceCount_Args* args) {
  CHECK_ARGS(args, PJRT_Buffer_DecreaseExternalReferenceCount_Args);
  NEED_BUF(args->buffer, "DecreaseExternalReferenceCount");
  if (args->buffer->external_refs <= 0)
    return make_error(PJRT_Error_Code_FAILED_PRECONDITION, "DecreaseExternalReferenceCount: count is already 0");
  --args->buffer->external_refs;
  return nullptr;
}

PJRT_Error* Buffer_OpaqueDeviceMemoryDataPointer(PJRT_Buffer_OpaqueDeviceMemoryDataPointer_Args* args) {
  CHECK_ARGS(args, PJRT_Buffer_OpaqueDeviceMemoryDataPointer_Args);
  NEED_BUF(args->buffer, "OpaqueDeviceMemoryDataPointer");
  args->device_memory_ptr = mkrt_buffer_device_pointer(args->buffer->b);
  return nullptr;
}

// Host-to-device streams are not offered (the reference's are stubs too,
// api/pjrt_buffer.cc:267-288).
PJRT_Error* CopyToDeviceStream_Destroy(PJRT_CopyToDeviceStream_Destroy_Args* args) {
  CHECK_ARGS(args, PJRT_CopyToDeviceStream_Destroy_Args);
  return nullptr;
}
PJRT_Error* CopyToDeviceStream_AddChunk(PJRT_CopyToDeviceStream_AddChunk_Args* args) {
  CHECK_ARGS(args, PJRT_CopyToDeviceStream_AddChunk_Args);
  return make_error(PJRT_Error_Code_UNIMPLEMENTED, "CopyToDeviceStream is not implemented");
}
PJRT_Error* CopyToDeviceStream_TotalBytes(PJRT_CopyToDeviceStream_TotalBytes_Args* args) {
  CHECK_ARGS(args, PJRT_CopyToDeviceStream_TotalBytes_Args);
  args->total_bytes = 0;
  return nullptr;
}
PJRT_Error* CopyToDeviceStream_GranuleSize(PJRT_CopyToDeviceStream_GranuleSize_Args* args) {
  CHECK_ARGS(args, PJRT_CopyToDeviceStream_GranuleSize_Args);
  args->granule_size_in_bytes = 0;
  return nullptr;
}
PJRT_Error* CopyToDeviceStream_CurrentBytes(PJRT_CopyToDeviceStream_CurrentBytes_Args* args) {
  CHECK_ARGS(args, PJRT_CopyToDeviceStream_CurrentBytes_Args);
  args->current_bytes = 0;
  return nullptr;
}

// --------------------------------------------------------------- topology

PJRT_Error* TopologyDescription_Create(PJRT_TopologyDescription_Create_Args* args) {
  CHECK_ARGS(args, PJRT_TopologyDescription_Create_Args);
  args->topology = new PJRT_TopologyDescription;  // one MI355X, no client
  return nullptr;
}

PJRT_Error* TopologyDescription_Destroy(PJRT_TopologyDescription_Destroy_Args* args) {
  CHECK_ARGS(args, PJRT_TopologyDescription_Destroy_Args);
  // A client's topology belongs to the client.
  if (args->topology && !args->topology->client) delete args->topology;
  return nullptr;
}

PJRT_Error* TopologyDescription_PlatformName(PJRT_TopologyDescription_PlatformName_Args* args) {
  CHECK_ARGS(args, PJRT_TopologyDescription_PlatformName_Args);
  args->platform_name = kPlatformName;
  args->platform_name_size = sizeof(kPlatformName) - 1;
  return nullptr;
}

PJRT_Error* TopologyDescription_PlatformVersion(PJRT_TopologyDescription_PlatformVersion_Args* args) {
  CHECK_ARGS(args, PJRT_TopologyDescription_PlatformVersion_Args);
  args->platform_version = kPlatformVersion;
  args->platform_version_size = sizeof(kPlatformVersion) - 1;
  return nullptr;
}

PJRT_Error* TopologyDescription_GetDeviceDescriptions(PJRT_TopologyDescription_GetDeviceDescriptions_Args* args) {
  CHECK_ARGS(args, PJRT_TopologyDescription_GetDeviceDescriptions_Args);
  if (!args->topology) return make_error(PJRT_Error_Code_INVALID_ARGUMENT, "GetDeviceDescriptions: null topology");
  args->descriptions = args->topology->descs;
  args->num_descriptions = 1;
  return nullptr;
}

PJRT_Error* TopologyDescription_Serialize(PJRT_TopologyDescription_Serialize_Args* args) {
  CHECK_ARGS(args, PJRT_TopologyDescription_Serialize_Args);
  return make_error(PJRT_Error_Code_UNIMPLEMENTED, "TopologyDescription_Serialize is not implemented");
}

PJRT_Error* TopologyDescription_Attributes(PJRT_TopologyDescription_Attributes_Args* args) {
  CHECK_ARGS(args, PJRT_TopologyDescription_Attributes_Args);
  args->attributes = nullptr;
  args->num_attributes = 0;
  return nullptr;
}

// FNV-1a 64 over length-prefixed platform name, version and device list:
// stable across processes (no addresses), as the reference's fingerprint is
// (api/pjrt_topology.cc:69-104).
PJRT_Error* TopologyDescription_Fingerprint(PJRT_TopologyDescription_Fingerprint_Args* args) {
  CHECK_ARGS(args, PJRT_TopologyDescription_Fingerprint_Args);
  if (!args->topology) return make_error(PJRT_Error_Code_INVALID_ARGUMENT, "Fingerprint: null topology");
  uint64_t h = 1469598103934665603ull;
  auto byte = [&](uint8_t b) { h = (h ^ b) * 1099511628211ull; };
  auto num = [&](uint64_t v) {
    for (int i = 0; i < 8; ++i, v >>= 8) byte((uint8_t)v);
  };
  auto str = [&](const char* s, size_t n) {
    num(n);
    for (size_t i = 0; i < n; ++i) byte((uint8_t)s[i]);
  };
  str(kPlatformName, sizeof(kPlatformName) - 1);
  str(kPlatformVersion, sizeof(kPlatformVersion) - 1);
  num(1);
  num((uint64_t)args->topology->desc.id);
  str(kDeviceKind, sizeof(kDeviceKind) - 1);
  args->fingerprint = h;
  return nullptr;
}

PJRT_Error* Compile(PJRT_Compile_Args* args) {
  CHECK_ARGS(args, PJRT_Compile_Args);
  return make_error(PJRT_Error_Code_UNIMPLEMENTED,
                    "PJRT_Compile (compile without a client) is not implemented; use PJRT_Client_Compile");
}

PJRT_Api make_api() {
  PJRT_Api a;
  memset(&a, 0, sizeof(a));
  a.struct_size = PJRT_Api_STRUCT_SIZE;
  a.extension_start = nullptr;
  a.pjrt_api_version.struct_size = PJRT_Api_Version_STRUCT_SIZE;
  a.pjrt_api_version.extension_start = nullptr;
  a.pjrt_api_version.major_version = PJRT_API_MAJOR;
  a.pjrt_api_version.minor_version = PJRT_API_MINOR;
#define SET(name) a.PJRT_##name = name
  SET(Error_Destroy);
  SET(Error_Message);
  SET(Error_GetCode);
  SET(Plugin_Initialize);
  SET(Plugin_Attributes);
  SET(Event_Destroy);
  SET(Event_IsReady);
  SET(Event_Error);
  SET(Event_Await);
  SET(Event_OnReady);
  SET(Client_Create);
  SET(Client_Destroy);
  SET(Client_PlatformName);
  SET(Client_ProcessIndex);
  SET(Client_PlatformVersion);
  SET(Client_Devices);
  SET(Client_AddressableDevices);
  SET(Client_LookupDevice);
  SET(Client_LookupAddressableDevice);
  SET(Client_AddressableMemories);
  SET(Client_Compile);
  SET(Client_DefaultDeviceAssignment);
  SET(Client_BufferFromHostBuffer);
  SET(DeviceDescription_Id);
  SET(DeviceDescription_ProcessIndex);
  SET(DeviceDescription_Attributes);
  SET(DeviceDescription_Kind);
  SET(DeviceDescription_DebugString);
  SET(DeviceDescription_ToString);
  SET(Device_GetDescription);
  SET(Device_IsAddressable);
  SET(Device_LocalHardwareId);
  SET(Device_AddressableMemories);
  SET(Device_DefaultMemory);
  SET(Device_MemoryStats);
  SET(Memory_Id);
  SET(Memory_Kind);
  SET(Memory_DebugString);
  SET(Memory_ToString);
  SET(Memory_AddressableByDevices);
  SET(Executable_Destroy);
  SET(Executable_Name);
  SET(Executable_NumReplicas);
  SET(Executable_NumPartitions);
  SET(Executable_NumOutputs);
  SET(Executable_SizeOfGeneratedCodeInBytes);
  SET(Executable_GetCostAnalysis);
  SET(Executable_OutputMemoryKinds);
  SET(Executable_OptimizedProgram);
  SET(Executable_Serialize);
  SET(LoadedExecutable_Destroy);
  SET(LoadedExecutable_GetExecutable);
  SET(LoadedExecutable_AddressableDevices);
  SET(LoadedExecutable_Delete);
  SET(LoadedExecutable_IsDeleted);
  SET(LoadedExecutable_Execute);
  SET(Executable_DeserializeAndLoad);
  SET(LoadedExecutable_Fingerprint);
  SET(Buffer_Destroy);
  SET(Buffer_ElementType);
  SET(Buffer_Dimensions);
  SET(Buffer_UnpaddedDimensions);
  SET(Buffer_DynamicDimensionIndices);
  SET(Buffer_GetMemoryLayout);
  SET(Buffer_OnDeviceSizeInBytes);
  SET(Buffer_Device);
  SET(Buffer_Memory);
  SET(Buffer_Delete);
  SET(Buffer_IsDeleted);
  SET(Buffer_CopyToDevice);
  SET(Buffer_ToHostBuffer);
  SET(Buffer_IsOnCpu);
  SET(Buffer_ReadyEvent);
  SET(Buffer_UnsafePointer);
  SET(Buffer_IncreaseExternalReferenceCount);
  SET(Buffer_DecreaseExternalReferenceCount);
  SET(Buffer_OpaqueDeviceMemoryDataPointer);
  SET(CopyToDeviceStream_Destroy);
  SET(CopyToDeviceStream_AddChunk);
  SET(CopyToDeviceStream_TotalBytes);
  SET(CopyToDeviceStream_GranuleSize);
  SET(CopyToDeviceStream_CurrentBytes);
  SET(TopologyDescription_Create);
  SET(TopologyDescription_Destroy);
  SET(TopologyDescription_PlatformName);
  SET(TopologyDescription_PlatformVersion);
  SET(TopologyDescription_GetDeviceDescriptions);
  SET(TopologyDescription_Serialize);
  SET(TopologyDescription_Attributes);
  SET(Compile);
  SET(Executable_OutputElementTypes);
  SET(Executable_OutputDimensions);
  SET(Buffer_CopyToMemory);
  SET(Client_CreateViewOfDeviceBuffer);
  SET(Executable_Fingerprint);
  SET(Client_TopologyDescription);
  SET(Memory_Kind_Id);
  SET(Buffer_CopyRawToHost);
  SET(Client_CreateUninitializedBuffer);
  SET(LoadedExecutable_GetDeviceAssignment);
  SET(Client_CreateErrorBuffer);
  SET(Buffer_CopyRawToHostFuture);
  SET(Event_Create);
  SET(Event_Set);
  SET(Error_ForEachPayload);
  SET(TopologyDescription_Fingerprint);
  SET(Executable_ParameterMemoryKinds);
#undef SET
  return a;
}

}  // namespace

extern "C" __attribute__((visibility("default"))) const PJRT_Api* GetPjrtApi(void) {
  static const PJRT_Api api = make_api();
  return &api;
}
