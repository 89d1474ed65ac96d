/*
 * Test harness for libmk_pjrt.so, in C, built with -fsanitize=address,undefined.
 *
 * It loads the plugin with dlopen, as jaxlib does, and drives it only
 * through the exported GetPjrtApi table (the reference's own checks of its
 * table: tests/test_pjrt_required_callbacks.py:118-160 and
 * tests/test_pjrt_handle_abi.py:15-25 under /root/reference).  Modes:
 *
 *   api LIB [expect_client]        table shape, errors, events, topology,
 *                                  argument-struct checks; Client_Create
 *                                  must succeed ("gpu") or fail with
 *                                  UNAVAILABLE ("nogpu")
 *   parse KLIB FILE...             mkrt_compile_check on each StableHLO file
 *                                  and on every truncation and a set of
 *                                  byte flips of it (the parser and planner
 *                                  under the sanitizers); never crashes
 *   inspect KLIB FILE...           mkrt_serialized_inspect on each
 *                                  serialized executable and on every
 *                                  truncation and byte flip of its header
 *   run LIB PROGRAM OUT IN...      Client_Create, Compile, BufferFromHostBuffer
 *                                  per input, Execute, Event_Await,
 *                                  ToHostBuffer; writes output 0 to OUT.
 *                                  An input file is "TYPE:d0xd1x...:path"
 *                                  with TYPE the PJRT_Buffer_Type number.
 *                                  Also checks Serialize / DeserializeAndLoad,
 *                                  output metadata, the device assignment,
 *                                  CopyRawToHost, buffer deletion.
 *   time LIB PROGRAM WARMUP ITERS IN...
 *                                  the plugin path as a C caller drives it:
 *                                  Compile once, then per call Execute,
 *                                  Event_Await and Buffer_Destroy of the
 *                                  outputs, inputs resident; prints one
 *                                  JSON line of per-call wall-clock times
 *   floor KLIB HIPLIB WARMUP ITERS the host floor under that path: the int4
 *                                  g64 M=16 K=4096 N=14336 product called
 *                                  straight through the kernel library's
 *                                  C-ABI on a stream of its own, an event
 *                                  recorded behind it and polled until
 *                                  ready, per call; same JSON line
 *
 * Exit status 0 on success; a failing check prints "FAIL: ..." and exits 1.
 */
#define _POSIX_C_SOURCE 200809L
#include <dlfcn.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "pjrt_c_api_mi355x.h"

static const PJRT_Api* api;
static int checks;

static void check(int ok, const char* what) {
  ++checks;
  if (!ok) {
    fprintf(stderr, "FAIL: %s\n", what);
    exit(1);
  }
}

#define ARGS(T, name) \
  T name;             \
  memset(&name, 0, sizeof(name)); \
  name.struct_size = T##_STRUCT_SIZE

static PJRT_Error_Code code_of(PJRT_Error* e) {
  ARGS(PJRT_Error_GetCode_Args, a);
  a.error = e;
  check(api->PJRT_Error_GetCode(&a) == NULL, "Error_GetCode succeeds");
  return a.code;
}

static void message_of(PJRT_Error* e, char* out, size_t n) {
  ARGS(PJRT_Error_Message_Args, a);
  a.error = e;
  api->PJRT_Error_Message(&a);
  snprintf(out, n, "%.*s", (int)a.message_size, a.message ? a.message : "");
}

static void destroy_error(PJRT_Error* e) {
  ARGS(PJRT_Error_Destroy_Args, a);
  a.error = e;
  api->PJRT_Error_Destroy(&a);
}

/* Expect an error of `code`; consume it. */
static void expect_error(PJRT_Error* e, PJRT_Error_Code code, const char* what) {
  char buf[512];
  if (!e) {
    fprintf(stderr, "FAIL: %s: expected error code %d, got success\n", what, (int)code);
    exit(1);
  }
  message_of(e, buf, sizeof buf);
  if (code_of(e) != code) {
    fprintf(stderr, "FAIL: %s: expected code %d, got %d (%s)\n", what, (int)code, (int)code_of(e), buf);
    exit(1);
  }
  check(buf[0] != 0, "error carries a message");
  destroy_error(e);
  ++checks;
}

static void ok(PJRT_Error* e, const char* what) {
  if (e) {
    char buf[1024];
    message_of(e, buf, sizeof buf);
    fprintf(stderr, "FAIL: %s: [%d] %s\n", what, (int)code_of(e), buf);
    exit(1);
  }
  ++checks;
}

static void* load(const char* path) {
  void* h = dlopen(path, RTLD_NOW | RTLD_LOCAL);
  if (!h) {
    fprintf(stderr, "FAIL: dlopen %s: %s\n", path, dlerror());
    exit(1);
  }
  return h;
}

/* ------------------------------------------------------------------ api */

static int ready_calls;
static PJRT_Error_Code ready_code;
static char ready_msg[256];
static void on_ready(PJRT_Error* e, void* user) {
  ++ready_calls;
  check(user == (void*)&ready_calls, "OnReady passes user_arg");
  ready_code = e ? code_of(e) : PJRT_Error_Code_OK;
  ready_msg[0] = 0;
  if (e) {
    message_of(e, ready_msg, sizeof ready_msg);
    destroy_error(e);
  }
}

static int payloads;
static void visit(const char* k, size_t kn, const char* v, size_t vn, void* u) {
  (void)k; (void)kn; (void)v; (void)vn; (void)u;
  ++payloads;
}

static PJRT_Event* new_event(void) {
  ARGS(PJRT_Event_Create_Args, a);
  ok(api->PJRT_Event_Create(&a), "Event_Create");
  check(a.event != NULL, "Event_Create returns an event");
  return a.event;
}

static void destroy_event(PJRT_Event* ev) {
  ARGS(PJRT_Event_Destroy_Args, a);
  a.event = ev;
  ok(api->PJRT_Event_Destroy(&a), "Event_Destroy");
}

static void test_table(void) {
  check(api->struct_size == PJRT_Api_STRUCT_SIZE, "PJRT_Api struct_size");
  check(api->pjrt_api_version.major_version == PJRT_API_MAJOR && api->pjrt_api_version.minor_version == PJRT_API_MINOR,
        "API version 0.114");
  check(api->pjrt_api_version.struct_size == PJRT_Api_Version_STRUCT_SIZE, "version struct_size");
  /* Every entry the reference's table sets (api/pjrt_api.cc:172-321) is set;
   * the ones it leaves NULL stay NULL. */
  const void* const* fn = (const void* const*)&api->PJRT_Error_Destroy;
  const size_t n = (PJRT_Api_STRUCT_SIZE - offsetof(PJRT_Api, PJRT_Error_Destroy)) / sizeof(void*);
  size_t set = 0;
  for (size_t i = 0; i < n; ++i) set += fn[i] != NULL;
  check(n == 131, "131 table entries through ParameterMemoryKinds");
  check(set == 107, "107 entries set (the reference's non-null set)");
  check(api->PJRT_ExecuteContext_Create == NULL && api->PJRT_Client_DmaMap == NULL &&
            api->PJRT_AsyncHostToDeviceTransferManager_Destroy == NULL && api->PJRT_Executable_GetCompiledMemoryStats == NULL,
        "optional entries stay NULL");
  check(api->PJRT_Error_ForEachPayload && api->PJRT_TopologyDescription_Fingerprint &&
            api->PJRT_Executable_ParameterMemoryKinds && api->PJRT_Event_Create && api->PJRT_Event_Set,
        "version-required entries (0.99 / 0.101 / 0.102) are set");
}

static void test_errors(void) {
  /* A null argument struct and a short one are INVALID_ARGUMENT. */
  expect_error(api->PJRT_Event_IsReady(NULL), PJRT_Error_Code_INVALID_ARGUMENT, "null args");
  PJRT_Event_IsReady_Args s;
  memset(&s, 0, sizeof s);
  s.struct_size = PJRT_Event_IsReady_Args_STRUCT_SIZE - 1;
  expect_error(api->PJRT_Event_IsReady(&s), PJRT_Error_Code_INVALID_ARGUMENT, "short struct_size");
  /* The error's own function table matches the API calls. */
  PJRT_Error* e = api->PJRT_Event_IsReady(NULL);
  check(e && e->vtable && e->vtable->struct_size == PJRT_Error_FunctionTable_STRUCT_SIZE,
        "error function table present");
  const char* m = NULL;
  size_t mn = 0;
  e->vtable->message(e, &m, &mn);
  char via_api[512];
  message_of(e, via_api, sizeof via_api);
  check(mn == strlen(via_api) && strncmp(m, via_api, mn) == 0, "vtable message == Error_Message");
  check(e->vtable->get_code(e) == PJRT_Error_Code_INVALID_ARGUMENT, "vtable code");
  ARGS(PJRT_Error_ForEachPayload_Args, fp);
  fp.error = e;
  fp.visitor = visit;
  ok(api->PJRT_Error_ForEachPayload(&fp), "Error_ForEachPayload");
  check(payloads == 0, "no payloads");
  destroy_error(e);
  /* Destroying / reading a NULL error is harmless. */
  ARGS(PJRT_Error_Destroy_Args, d);
  api->PJRT_Error_Destroy(&d);
  ARGS(PJRT_Error_GetCode_Args, g);
  ok(api->PJRT_Error_GetCode(&g), "GetCode(NULL)");
  check(g.code == PJRT_Error_Code_OK, "GetCode(NULL) is OK");
}

static void test_events(void) {
  PJRT_Event* ev = new_event();
  ARGS(PJRT_Event_IsReady_Args, r);
  r.event = ev;
  ok(api->PJRT_Event_IsReady(&r), "Event_IsReady");
  check(!r.is_ready, "new event is pending");
  ARGS(PJRT_Event_Error_Args, er);
  er.event = ev;
  expect_error(api->PJRT_Event_Error(&er), PJRT_Error_Code_FAILED_PRECONDITION, "Event_Error before ready");
  ARGS(PJRT_Event_OnReady_Args, on);
  on.event = ev;
  on.callback = on_ready;
  on.user_arg = &ready_calls;
  ok(api->PJRT_Event_OnReady(&on), "Event_OnReady");
  check(ready_calls == 0, "callback waits for the event");
  ARGS(PJRT_Event_Set_Args, set);
  set.event = ev;
  set.error_code = PJRT_Error_Code_DATA_LOSS - 2;  /* INTERNAL = 13 */
  set.error_message = "device fell over";
  set.error_message_size = strlen("device fell over");
  ok(api->PJRT_Event_Set(&set), "Event_Set");
  check(ready_calls == 1 && ready_code == PJRT_Error_Code_INTERNAL && strcmp(ready_msg, "device fell over") == 0,
        "callback ran once with the error");
  ok(api->PJRT_Event_IsReady(&r), "IsReady after set");
  check(r.is_ready, "set event is ready");
  ARGS(PJRT_Event_Await_Args, aw);
  aw.event = ev;
  expect_error(api->PJRT_Event_Await(&aw), PJRT_Error_Code_INTERNAL, "Await returns the event's error");
  expect_error(api->PJRT_Event_Error(&er), PJRT_Error_Code_INTERNAL, "Event_Error after ready");
  /* A callback added to a ready event runs inline. */
  ok(api->PJRT_Event_OnReady(&on), "OnReady on a ready event");
  check(ready_calls == 2, "inline callback");
  destroy_event(ev);
  /* A successful event. */
  ev = new_event();
  set.event = ev;
  set.error_code = PJRT_Error_Code_OK;
  set.error_message = NULL;
  set.error_message_size = 0;
  ok(api->PJRT_Event_Set(&set), "Event_Set OK");
  aw.event = ev;
  ok(api->PJRT_Event_Await(&aw), "Await OK");
  er.event = ev;
  ok(api->PJRT_Event_Error(&er), "Event_Error OK");
  destroy_event(ev);
}

static void test_topology(void) {
  ARGS(PJRT_TopologyDescription_Create_Args, c);
  ok(api->PJRT_TopologyDescription_Create(&c), "TopologyDescription_Create");
  check(c.topology != NULL, "topology");
  ARGS(PJRT_TopologyDescription_PlatformName_Args, pn);
  pn.topology = c.topology;
  ok(api->PJRT_TopologyDescription_PlatformName(&pn), "PlatformName");
  check(pn.platform_name_size == 6 && memcmp(pn.platform_name, "mi355x", 6) == 0, "platform name mi355x");
  ARGS(PJRT_TopologyDescription_GetDeviceDescriptions_Args, dd);
  dd.topology = c.topology;
  ok(api->PJRT_TopologyDescription_GetDeviceDescriptions(&dd), "GetDeviceDescriptions");
  check(dd.num_descriptions == 1 && dd.descriptions && dd.descriptions[0], "one device description");
  ARGS(PJRT_DeviceDescription_Kind_Args, k);
  k.device_description = dd.descriptions[0];
  ok(api->PJRT_DeviceDescription_Kind(&k), "DeviceDescription_Kind");
  check(k.device_kind_size > 0, "device kind");
  ARGS(PJRT_TopologyDescription_Fingerprint_Args, f);
  f.topology = c.topology;
  ok(api->PJRT_TopologyDescription_Fingerprint(&f), "Fingerprint");
  uint64_t first = f.fingerprint;
  ok(api->PJRT_TopologyDescription_Fingerprint(&f), "Fingerprint again");
  check(f.fingerprint == first && first != 0, "fingerprint repeatable");
  f.topology = NULL;
  expect_error(api->PJRT_TopologyDescription_Fingerprint(&f), PJRT_Error_Code_INVALID_ARGUMENT, "null topology");
  ARGS(PJRT_TopologyDescription_Serialize_Args, ser);
  ser.topology = c.topology;
  expect_error(api->PJRT_TopologyDescription_Serialize(&ser), PJRT_Error_Code_UNIMPLEMENTED, "Serialize topology");
  ARGS(PJRT_Compile_Args, comp);
  comp.topology = c.topology;
  expect_error(api->PJRT_Compile(&comp), PJRT_Error_Code_UNIMPLEMENTED, "PJRT_Compile");
  ARGS(PJRT_TopologyDescription_Destroy_Args, d);
  d.topology = c.topology;
  ok(api->PJRT_TopologyDescription_Destroy(&d), "TopologyDescription_Destroy");
  ARGS(PJRT_Plugin_Initialize_Args, pi);
  ok(api->PJRT_Plugin_Initialize(&pi), "Plugin_Initialize");
  ARGS(PJRT_Plugin_Attributes_Args, pa);
  ok(api->PJRT_Plugin_Attributes(&pa), "Plugin_Attributes");
}

static PJRT_Client* create_client(int expect_ok) {
  ARGS(PJRT_Client_Create_Args, c);
  PJRT_Error* e = api->PJRT_Client_Create(&c);
  if (!expect_ok) {
    expect_error(e, PJRT_Error_Code_UNAVAILABLE, "Client_Create without a GPU");
    check(c.client == NULL, "no client on failure");
    return NULL;
  }
  ok(e, "Client_Create");
  check(c.client != NULL, "client");
  return c.client;
}

static void destroy_client(PJRT_Client* c) {
  ARGS(PJRT_Client_Destroy_Args, d);
  d.client = c;
  ok(api->PJRT_Client_Destroy(&d), "Client_Destroy");
}

static void test_client(PJRT_Client* c) {
  ARGS(PJRT_Client_PlatformName_Args, pn);
  pn.client = c;
  ok(api->PJRT_Client_PlatformName(&pn), "Client_PlatformName");
  check(pn.platform_name_size == 6 && memcmp(pn.platform_name, "mi355x", 6) == 0, "client platform name");
  ARGS(PJRT_Client_Devices_Args, dv);
  dv.client = c;
  ok(api->PJRT_Client_Devices(&dv), "Client_Devices");
  check(dv.num_devices == 1, "one device");
  ARGS(PJRT_Client_LookupDevice_Args, lk);
  lk.client = c;
  lk.id = 0;
  ok(api->PJRT_Client_LookupDevice(&lk), "LookupDevice 0");
  check(lk.device == dv.devices[0], "device 0");
  lk.id = 3;
  expect_error(api->PJRT_Client_LookupDevice(&lk), PJRT_Error_Code_INVALID_ARGUMENT, "LookupDevice 3");
  ARGS(PJRT_Device_DefaultMemory_Args, dm);
  dm.device = dv.devices[0];
  ok(api->PJRT_Device_DefaultMemory(&dm), "Device_DefaultMemory");
  ARGS(PJRT_Memory_Kind_Args, mk);
  mk.memory = dm.memory;
  ok(api->PJRT_Memory_Kind(&mk), "Memory_Kind");
  check(mk.kind_size == 6 && memcmp(mk.kind, "device", 6) == 0, "memory kind device");
  /* The memory's user-data table (API >= 0.105). */
  check(dm.memory->vtable && dm.memory->vtable->get_user_data, "memory function table");
  static int key, value;
  dm.memory->vtable->set_user_data(dm.memory, &key, &value, NULL);
  check(dm.memory->vtable->get_user_data(dm.memory, &key) == &value, "memory user data round trip");
  dm.memory->vtable->set_user_data(dm.memory, &key, NULL, NULL);
  check(dm.memory->vtable->get_user_data(dm.memory, &key) == NULL, "memory user data removed");
  ARGS(PJRT_Device_MemoryStats_Args, ms);
  ms.device = dv.devices[0];
  ok(api->PJRT_Device_MemoryStats(&ms), "Device_MemoryStats");
  check(ms.bytes_limit_is_set && ms.bytes_limit > ((int64_t)100 << 30), "HBM limit > 100 GiB");
  int assign[1] = {-1};
  ARGS(PJRT_Client_DefaultDeviceAssignment_Args, da);
  da.client = c;
  da.num_replicas = 1;
  da.num_partitions = 1;
  da.default_assignment_size = 1;
  da.default_assignment = assign;
  ok(api->PJRT_Client_DefaultDeviceAssignment(&da), "DefaultDeviceAssignment");
  check(assign[0] == 0, "assignment to device 0");
  da.num_replicas = 2;
  expect_error(api->PJRT_Client_DefaultDeviceAssignment(&da), PJRT_Error_Code_INVALID_ARGUMENT, "two replicas");
  /* Unsupported program text fails at compile with UNIMPLEMENTED naming the op. */
  static char prog[] =
      "module @m {\n  func.func public @main(%arg0: tensor<4xf32>) -> tensor<4xf32> {\n"
      "    %0 = stablehlo.cosine %arg0 : tensor<4xf32>\n    return %0 : tensor<4xf32>\n  }\n}\n";
  ARGS(PJRT_Program, p);
  p.code = prog;
  p.code_size = strlen(prog);
  p.format = "mlir";
  p.format_size = 4;
  ARGS(PJRT_Client_Compile_Args, cc);
  cc.client = c;
  cc.program = &p;
  expect_error(api->PJRT_Client_Compile(&cc), PJRT_Error_Code_UNIMPLEMENTED, "unsupported op at compile");
  p.format = "tflite";
  p.format_size = 6;
  expect_error(api->PJRT_Client_Compile(&cc), PJRT_Error_Code_INVALID_ARGUMENT, "unknown format");
}

static int mode_api(const char* lib, const char* expect) {
  void* h = load(lib);
  const PJRT_Api* (*get)(void) = (const PJRT_Api* (*)(void))dlsym(h, "GetPjrtApi");
  check(get != NULL, "GetPjrtApi exported");
  api = get();
  check(api != NULL && get() == api, "one static table");
  test_table();
  test_errors();
  test_events();
  test_topology();
  PJRT_Client* c = create_client(strcmp(expect, "gpu") == 0);
  if (c) {
    test_client(c);
    destroy_client(c);
  }
  printf("api ok: %d checks\n", checks);
  return 0;
}

/* ---------------------------------------------------------- parse/inspect */

typedef struct mkrt_error mkrt_error;
static mkrt_error* (*compile_check)(const char*, int64_t, const char*, char*, int64_t, int*);
static mkrt_error* (*inspect)(const void*, int64_t, int64_t*, int*);
static void (*err_destroy)(mkrt_error*);
static int (*err_code)(const mkrt_error*);

static char* read_file(const char* path, long* n) {
  FILE* f = fopen(path, "rb");
  if (!f) {
    fprintf(stderr, "FAIL: open %s\n", path);
    exit(1);
  }
  fseek(f, 0, SEEK_END);
  *n = ftell(f);
  fseek(f, 0, SEEK_SET);
  char* b = (char*)malloc((size_t)*n + 1);
  if (fread(b, 1, (size_t)*n, f) != (size_t)*n) {
    fprintf(stderr, "FAIL: read %s\n", path);
    exit(1);
  }
  b[*n] = 0;
  fclose(f);
  return b;
}

static void load_runtime(const char* klib) {
  void* h = load(klib);
  compile_check = dlsym(h, "mkrt_compile_check");
  inspect = dlsym(h, "mkrt_serialized_inspect");
  err_destroy = dlsym(h, "mkrt_error_destroy");
  err_code = dlsym(h, "mkrt_error_code");
  check(compile_check && inspect && err_destroy && err_code, "runtime entry points");
}

/* Run fn on a heap copy of exactly n bytes (so a read past the end is caught). */
static int run_copy(const char* data, long n, int is_text) {
  char* b = (char*)malloc(n > 0 ? (size_t)n : 1);
  memcpy(b, data, (size_t)n);
  int code;
  if (is_text) {
    char plan[4096];
    int steps = 0;
    mkrt_error* e = compile_check(b, n, "mlir", plan, sizeof plan, &steps);
    code = e ? err_code(e) : 0;
    if (e) err_destroy(e);
  } else {
    int64_t pb = 0;
    int no = 0;
    mkrt_error* e = inspect(b, n, &pb, &no);
    code = e ? err_code(e) : 0;
    if (e) err_destroy(e);
  }
  free(b);
  return code;
}

static int mode_fuzz(int argc, char** argv, int is_text) {
  load_runtime(argv[2]);
  long cases = 0;
  for (int i = 3; i < argc; ++i) {
    long n = 0;
    char* d = read_file(argv[i], &n);
    int base = run_copy(d, n, is_text);
    if (is_text) check(base == 0, "the unmodified program compiles");
    else check(base == 0, "the unmodified blob inspects");
    const long step = n > 4000 ? n / 2000 : 1;
    for (long cut = 0; cut < n; cut += step, ++cases) {
      int c = run_copy(d, cut, is_text);
      check(c == 0 || c == 3 || c == 12, "truncation gives OK, INVALID_ARGUMENT or UNIMPLEMENTED");
    }
    /* Byte flips over the first 4 KB: every byte of a blob or of MLIR
       bytecode, every 7th of a text program. */
    const long lim = n < 4096 ? n : 4096;
    const int every = is_text && !(n >= 4 && memcmp(d, "ML\xefR", 4) == 0) ? 7 : 1;
    for (long k = 0; k < lim; k += every, ++cases) {
      char* m = (char*)malloc((size_t)n);
      memcpy(m, d, (size_t)n);
      m[k] ^= (char)(0x5A + (k & 0x7F));
      int c = run_copy(m, n, is_text);
      check(c == 0 || c == 3 || c == 12, "byte flip gives OK, INVALID_ARGUMENT or UNIMPLEMENTED");
      free(m);
    }
    free(d);
  }
  printf("%s ok: %d files, %ld mutated cases\n", is_text ? "parse" : "inspect", argc - 3, cases);
  return 0;
}

/* ------------------------------------------------------------------- run */

static int64_t parse_dims(const char* s, int64_t* dims) {
  int64_t n = 0;
  while (*s) {
    dims[n++] = strtoll(s, (char**)&s, 10);
    if (*s == 'x') ++s;
  }
  return n;
}


static PJRT_Buffer* upload(PJRT_Client* c, const char* spec) {
  char type_s[16], dims_s[128], path[1024];
  const char* a = strchr(spec, ':');
  const char* b = a ? strchr(a + 1, ':') : NULL;
  check(a && b, "input spec TYPE:DIMS:PATH");
  snprintf(type_s, sizeof type_s, "%.*s", (int)(a - spec), spec);
  snprintf(dims_s, sizeof dims_s, "%.*s", (int)(b - a - 1), a + 1);
  snprintf(path, sizeof path, "%s", b + 1);
  int64_t dims[16];
  const int64_t nd = parse_dims(dims_s, dims);
  long n = 0;
  char* data = read_file(path, &n);
  ARGS(PJRT_Client_BufferFromHostBuffer_Args, u);
  u.client = c;
  u.data = data;
  u.type = (PJRT_Buffer_Type)atoi(type_s);
  u.dims = dims;
  u.num_dims = (size_t)nd;
  u.host_buffer_semantics = PJRT_HostBufferSemantics_kImmutableOnlyDuringCall;
  ok(api->PJRT_Client_BufferFromHostBuffer(&u), "BufferFromHostBuffer");
  check(u.buffer && u.done_with_host_buffer, "buffer and done event");
  ARGS(PJRT_Event_Await_Args, aw);
  aw.event = u.done_with_host_buffer;
  ok(api->PJRT_Event_Await(&aw), "done_with_host_buffer");
  destroy_event(u.done_with_host_buffer);
  free(data);  /* the host array is no longer needed */
  return u.buffer;
}

static void destroy_buffer(PJRT_Buffer* b) {
  ARGS(PJRT_Buffer_Destroy_Args, d);
  d.buffer = b;
  ok(api->PJRT_Buffer_Destroy(&d), "Buffer_Destroy");
}

static char* to_host(PJRT_Buffer* b, size_t* n) {
  ARGS(PJRT_Buffer_ToHostBuffer_Args, t);
  t.src = b;
  ok(api->PJRT_Buffer_ToHostBuffer(&t), "ToHostBuffer size query");
  *n = t.dst_size;
  char* host = (char*)malloc(*n ? *n : 1);
  t.dst = host;
  ok(api->PJRT_Buffer_ToHostBuffer(&t), "ToHostBuffer");
  ARGS(PJRT_Event_Await_Args, aw);
  aw.event = t.event;
  ok(api->PJRT_Event_Await(&aw), "ToHostBuffer event");
  destroy_event(t.event);
  return host;
}

static PJRT_LoadedExecutable* compile_program(PJRT_Client* c, char* text, long n) {
  ARGS(PJRT_Program, p);
  p.code = text;
  p.code_size = (size_t)n;
  p.format = "mlir";
  p.format_size = 4;
  ARGS(PJRT_Client_Compile_Args, cc);
  cc.client = c;
  cc.program = &p;
  ok(api->PJRT_Client_Compile(&cc), "Client_Compile");
  return cc.executable;
}

static void execute(PJRT_LoadedExecutable* le, PJRT_Buffer** in, size_t nin, PJRT_Buffer** out) {
  PJRT_Buffer* const* lists[1] = {in};
  PJRT_Buffer** outs[1] = {out};
  PJRT_Event* done[1] = {NULL};
  ARGS(PJRT_LoadedExecutable_Execute_Args, ex);
  ex.executable = le;
  ex.argument_lists = lists;
  ex.num_devices = 1;
  ex.num_args = nin;
  ex.output_lists = outs;
  ex.device_complete_events = done;
  ok(api->PJRT_LoadedExecutable_Execute(&ex), "Execute");
  check(done[0] != NULL, "device_complete_events[0]");
  ARGS(PJRT_Event_Await_Args, aw);
  aw.event = done[0];
  ok(api->PJRT_Event_Await(&aw), "Execute completion");
  destroy_event(done[0]);
}

static int mode_run(int argc, char** argv) {
  void* h = load(argv[2]);
  const PJRT_Api* (*get)(void) = (const PJRT_Api* (*)(void))dlsym(h, "GetPjrtApi");
  check(get != NULL, "GetPjrtApi");
  api = get();
  PJRT_Client* c = create_client(1);
  long plen = 0;
  char* prog = read_file(argv[3], &plen);
  PJRT_LoadedExecutable* le = compile_program(c, prog, plen);
  const size_t nin = (size_t)(argc - 5);
  PJRT_Buffer** in = (PJRT_Buffer**)calloc(nin + 1, sizeof(PJRT_Buffer*));
  for (size_t i = 0; i < nin; ++i) in[i] = upload(c, argv[5 + i]);

  /* Output signature from the executable. */
  ARGS(PJRT_LoadedExecutable_GetExecutable_Args, ge);
  ge.loaded_executable = le;
  ok(api->PJRT_LoadedExecutable_GetExecutable(&ge), "GetExecutable");
  ARGS(PJRT_Executable_NumOutputs_Args, no);
  no.executable = ge.executable;
  ok(api->PJRT_Executable_NumOutputs(&no), "NumOutputs");
  check(no.num_outputs >= 1 && no.num_outputs <= 16, "output count");
  ARGS(PJRT_Executable_OutputElementTypes_Args, ot);
  ot.executable = ge.executable;
  ok(api->PJRT_Executable_OutputElementTypes(&ot), "OutputElementTypes");
  ARGS(PJRT_Executable_OutputDimensions_Args, od);
  od.executable = ge.executable;
  ok(api->PJRT_Executable_OutputDimensions(&od), "OutputDimensions");
  check(od.num_outputs == no.num_outputs && ot.num_output_types == no.num_outputs, "output metadata agrees");
  ARGS(PJRT_Executable_Name_Args, nm);
  nm.executable = ge.executable;
  ok(api->PJRT_Executable_Name(&nm), "Executable_Name");
  ARGS(PJRT_Executable_Fingerprint_Args, fpa);
  fpa.executable = ge.executable;
  ok(api->PJRT_Executable_Fingerprint(&fpa), "Executable_Fingerprint");
  check(fpa.executable_fingerprint_size == 16, "16-digit fingerprint");
  /* A second GetExecutable handle is independent of the first. */
  ARGS(PJRT_LoadedExecutable_GetExecutable_Args, ge2);
  ge2.loaded_executable = le;
  ok(api->PJRT_LoadedExecutable_GetExecutable(&ge2), "GetExecutable twice");
  ARGS(PJRT_Executable_Destroy_Args, xd);
  xd.executable = ge2.executable;
  ok(api->PJRT_Executable_Destroy(&xd), "Executable_Destroy (second handle)");
  ARGS(PJRT_Executable_OptimizedProgram_Args, op);
  ARGS(PJRT_Program, opp);
  op.executable = ge.executable;
  op.program = &opp;
  ok(api->PJRT_Executable_OptimizedProgram(&op), "OptimizedProgram size query");
  if (plen >= 4 && memcmp(prog, "ML\xefR", 4) == 0) {
    /* Compiled from bytecode: the optimized program is its MLIR text. */
    check(opp.code_size > 0, "program text of a bytecode program");
    char* text = (char*)malloc(opp.code_size);
    opp.code = text;
    ok(api->PJRT_Executable_OptimizedProgram(&op), "OptimizedProgram text");
    check(opp.code_size >= 6 && memcmp(text, "module", 6) == 0, "decoded program text starts with module");
    free(text);
  } else {
    check(opp.code_size == (size_t)plen, "program size");
  }
  ARGS(PJRT_LoadedExecutable_GetDeviceAssignment_Args, gd);
  gd.executable = le;
  ok(api->PJRT_LoadedExecutable_GetDeviceAssignment(&gd), "GetDeviceAssignment");
  static const unsigned char want[] = {0x08, 0x01, 0x10, 0x01, 0x1A, 0x03, 0x0A, 0x01, 0x00};
  check(gd.serialized_bytes_size == sizeof want && memcmp(gd.serialized_bytes, want, sizeof want) == 0,
        "DeviceAssignmentProto bytes");
  gd.serialized_device_assignment_deleter(gd.serialized_device_assignment);

  PJRT_Buffer** out = (PJRT_Buffer**)calloc(no.num_outputs, sizeof(PJRT_Buffer*));
  execute(le, in, nin, out);
  ARGS(PJRT_Buffer_Dimensions_Args, bd);
  bd.buffer = out[0];
  ok(api->PJRT_Buffer_Dimensions(&bd), "Buffer_Dimensions");
  check(bd.num_dims == od.dim_sizes[0], "output rank");
  for (size_t i = 0; i < bd.num_dims; ++i) check(bd.dims[i] == od.dims[i], "output dims");
  ARGS(PJRT_Buffer_ElementType_Args, bt);
  bt.buffer = out[0];
  ok(api->PJRT_Buffer_ElementType(&bt), "Buffer_ElementType");
  check(bt.type == ot.output_types[0], "output type");
  size_t nbytes = 0;
  char* host = to_host(out[0], &nbytes);
  FILE* f = fopen(argv[4], "wb");
  check(f && fwrite(host, 1, nbytes, f) == nbytes, "write output");
  fclose(f);
  /* CopyRawToHost of the second half agrees with ToHostBuffer. */
  char* half = (char*)malloc(nbytes / 2 + 1);
  ARGS(PJRT_Buffer_CopyRawToHost_Args, raw);
  raw.buffer = out[0];
  raw.dst = half;
  raw.offset = (int64_t)(nbytes - nbytes / 2);
  raw.transfer_size = (int64_t)(nbytes / 2);
  ok(api->PJRT_Buffer_CopyRawToHost(&raw), "CopyRawToHost");
  ARGS(PJRT_Event_Await_Args, aw);
  aw.event = raw.event;
  ok(api->PJRT_Event_Await(&aw), "CopyRawToHost event");
  destroy_event(raw.event);
  check(memcmp(half, host + (nbytes - nbytes / 2), nbytes / 2) == 0, "raw copy matches");
  raw.offset = (int64_t)nbytes;
  raw.transfer_size = 1;
  expect_error(api->PJRT_Buffer_CopyRawToHost(&raw), PJRT_Error_Code_INVALID_ARGUMENT, "raw copy past the end");

  /* Serialize -> DeserializeAndLoad -> Execute gives the same bytes. */
  ARGS(PJRT_Executable_Serialize_Args, se);
  se.executable = ge.executable;
  ok(api->PJRT_Executable_Serialize(&se), "Executable_Serialize");
  ARGS(PJRT_Executable_DeserializeAndLoad_Args, dl);
  dl.client = c;
  dl.serialized_executable = se.serialized_bytes;
  dl.serialized_executable_size = se.serialized_bytes_size;
  ok(api->PJRT_Executable_DeserializeAndLoad(&dl), "DeserializeAndLoad");
  se.serialized_executable_deleter(se.serialized_executable);
  PJRT_Buffer** out2 = (PJRT_Buffer**)calloc(no.num_outputs, sizeof(PJRT_Buffer*));
  execute(dl.loaded_executable, in, nin, out2);
  size_t n2 = 0;
  char* host2 = to_host(out2[0], &n2);
  check(n2 == nbytes && memcmp(host, host2, nbytes) == 0, "deserialized executable gives the same bytes");
  dl.serialized_executable_size = 0;
  expect_error(api->PJRT_Executable_DeserializeAndLoad(&dl), PJRT_Error_Code_INVALID_ARGUMENT, "empty blob");

  /* A deleted input is refused; the buffer handle stays valid. */
  ARGS(PJRT_Buffer_Delete_Args, del);
  del.buffer = in[0];
  ok(api->PJRT_Buffer_Delete(&del), "Buffer_Delete");
  ARGS(PJRT_Buffer_IsDeleted_Args, isd);
  isd.buffer = in[0];
  ok(api->PJRT_Buffer_IsDeleted(&isd), "Buffer_IsDeleted");
  check(isd.is_deleted, "deleted");
  {
    PJRT_Buffer* const* lists[1] = {in};
    PJRT_Buffer** outs[1] = {out2};
    ARGS(PJRT_LoadedExecutable_Execute_Args, ex);
    ex.executable = le;
    ex.argument_lists = lists;
    ex.num_devices = 1;
    ex.num_args = nin;
    ex.output_lists = outs;
    expect_error(api->PJRT_LoadedExecutable_Execute(&ex), PJRT_Error_Code_INVALID_ARGUMENT, "deleted input");
  }
  for (size_t r = 0; r < no.num_outputs; ++r) {
    destroy_buffer(out[r]);
    destroy_buffer(out2[r]);
  }
  for (size_t i = 0; i < nin; ++i) destroy_buffer(in[i]);
  xd.executable = ge.executable;
  ok(api->PJRT_Executable_Destroy(&xd), "Executable_Destroy");
  ARGS(PJRT_LoadedExecutable_Destroy_Args, ld);
  ld.executable = le;
  ok(api->PJRT_LoadedExecutable_Destroy(&ld), "LoadedExecutable_Destroy");
  ld.executable = dl.loaded_executable;
  ok(api->PJRT_LoadedExecutable_Destroy(&ld), "LoadedExecutable_Destroy (deserialized)");
  destroy_client(c);
  free(host);
  free(host2);
  free(half);
  free(in);
  free(out);
  free(out2);
  free(prog);
  printf("run ok: %d checks, %zu output bytes\n", checks, nbytes);
  return 0;
}

static double now_us(void) {
  struct timespec t;
  clock_gettime(CLOCK_MONOTONIC, &t);
  return (double)t.tv_sec * 1e6 + (double)t.tv_nsec * 1e-3;
}

static int cmp_double(const void* a, const void* b) {
  const double x = *(const double*)a, y = *(const double*)b;
  return (x > y) - (x < y);
}

static void report(const char* what, double* t, int n) {
  qsort(t, (size_t)n, sizeof(double), cmp_double);
  printf("{\"what\": \"%s\", \"median_us\": %.2f, \"min_us\": %.2f, \"p90_us\": %.2f, \"iters\": %d}\n", what,
         t[n / 2], t[0], t[(int)(0.9 * (n - 1))], n);
}

static int mode_time(int argc, char** argv) {
  void* h = load(argv[2]);
  const PJRT_Api* (*get)(void) = (const PJRT_Api* (*)(void))dlsym(h, "GetPjrtApi");
  check(get != NULL, "GetPjrtApi");
  api = get();
  PJRT_Client* c = create_client(1);
  long plen = 0;
  char* prog = read_file(argv[3], &plen);
  PJRT_LoadedExecutable* le = compile_program(c, prog, plen);
  const int warmup = atoi(argv[4]), iters = atoi(argv[5]);
  check(warmup >= 0 && iters > 0, "WARMUP >= 0, ITERS > 0");
  const size_t nin = (size_t)(argc - 6);
  PJRT_Buffer** in = (PJRT_Buffer**)calloc(nin + 1, sizeof(PJRT_Buffer*));
  for (size_t i = 0; i < nin; ++i) in[i] = upload(c, argv[6 + i]);
  ARGS(PJRT_LoadedExecutable_GetExecutable_Args, ge);
  ge.loaded_executable = le;
  ok(api->PJRT_LoadedExecutable_GetExecutable(&ge), "GetExecutable");
  ARGS(PJRT_Executable_NumOutputs_Args, no);
  no.executable = ge.executable;
  ok(api->PJRT_Executable_NumOutputs(&no), "NumOutputs");
  PJRT_Buffer** out = (PJRT_Buffer**)calloc(no.num_outputs + 1, sizeof(PJRT_Buffer*));
  double* t = (double*)malloc(sizeof(double) * (size_t)iters);
  for (int i = 0; i < warmup + iters; ++i) {
    const double t0 = now_us();
    execute(le, in, nin, out);
    for (size_t r = 0; r < no.num_outputs; ++r) destroy_buffer(out[r]);
    if (i >= warmup) t[i - warmup] = now_us() - t0;
  }
  report("PJRT table from C: Execute + Event_Await + Buffer_Destroy", t, iters);
  for (size_t i = 0; i < nin; ++i) destroy_buffer(in[i]);
  ARGS(PJRT_Executable_Destroy_Args, xd);
  xd.executable = ge.executable;
  ok(api->PJRT_Executable_Destroy(&xd), "Executable_Destroy");
  ARGS(PJRT_LoadedExecutable_Destroy_Args, ld);
  ld.executable = le;
  ok(api->PJRT_LoadedExecutable_Destroy(&ld), "LoadedExecutable_Destroy");
  destroy_client(c);
  free(t);
  free(in);
  free(out);
  free(prog);
  return 0;
}

/* HIP runtime entry points used by the floor mode, resolved with dlsym (the
 * harness is plain C with no HIP headers); hipError_t is an int, 0 success,
 * 600 hipErrorNotReady. */
typedef int (*hip_malloc_fn)(void**, size_t);
typedef int (*hip_memset_fn)(void*, int, size_t);
typedef int (*hip_free_fn)(void*);
typedef int (*hip_handle_fn)(void**);
typedef int (*hip_event_create_fn)(void**, unsigned);
typedef int (*hip_record_fn)(void*, void*);
typedef int (*hip_query_fn)(void*);
typedef int (*hip_destroy_fn)(void*);
typedef int (*hip_sync_fn)(void);
typedef int64_t (*mk_ws_fn)(int, int64_t, int64_t, int64_t);
typedef int (*mk_int4_fn)(const void*, const void*, const void*, const void*, void*, int64_t, int64_t, int64_t, void*,
                          int64_t, void*);

static void* sym(void* h, const char* name) {
  void* f = dlsym(h, name);
  if (!f) {
    fprintf(stderr, "FAIL: symbol %s: %s\n", name, dlerror());
    exit(1);
  }
  return f;
}

static int mode_floor(char** argv) {
  void* hk = load(argv[2]);
  void* hh = load(argv[3]);
  const int warmup = atoi(argv[4]), iters = atoi(argv[5]);
  check(warmup >= 0 && iters > 0, "WARMUP >= 0, ITERS > 0");
  hip_malloc_fn hmalloc = (hip_malloc_fn)sym(hh, "hipMalloc");
  hip_memset_fn hmemset = (hip_memset_fn)sym(hh, "hipMemset");
  hip_free_fn hfree = (hip_free_fn)sym(hh, "hipFree");
  hip_handle_fn hstream = (hip_handle_fn)sym(hh, "hipStreamCreate");
  hip_event_create_fn hevent = (hip_event_create_fn)sym(hh, "hipEventCreateWithFlags");
  hip_record_fn hrecord = (hip_record_fn)sym(hh, "hipEventRecord");
  hip_query_fn hquery = (hip_query_fn)sym(hh, "hipEventQuery");
  hip_destroy_fn hsdestroy = (hip_destroy_fn)sym(hh, "hipStreamDestroy");
  hip_destroy_fn hedestroy = (hip_destroy_fn)sym(hh, "hipEventDestroy");
  hip_sync_fn hsync = (hip_sync_fn)sym(hh, "hipDeviceSynchronize");
  mk_ws_fn ws_bytes = (mk_ws_fn)sym(hk, "mk_qmatmul_workspace_bytes");
  mk_int4_fn int4 = (mk_int4_fn)sym(hk, "mk_int4g64_matmul_bf16");
  const int64_t M = 16, K = 4096, N = 14336;
  /* x bf16 [M,K], w [K/2,N], scale bf16 [K/64,N], zero [K/64,N], y bf16 [M,N];
   * zero-filled (the kernel's time does not depend on the values). */
  const size_t bytes[5] = {(size_t)(M * K * 2), (size_t)(K / 2 * N), (size_t)(K / 64 * N * 2), (size_t)(K / 64 * N),
                           (size_t)(M * N * 2)};
  void* d[5];
  for (int i = 0; i < 5; ++i) {
    check(hmalloc(&d[i], bytes[i]) == 0, "hipMalloc");
    check(hmemset(d[i], 0, bytes[i]) == 0, "hipMemset");
  }
  const int64_t wsb = ws_bytes(0, M, K, N);
  void* ws = NULL;
  if (wsb > 0) {
    check(hmalloc(&ws, (size_t)wsb) == 0, "hipMalloc workspace");
    check(hmemset(ws, 0, (size_t)wsb) == 0, "hipMemset workspace");
  }
  void *stream = NULL, *ev = NULL;
  check(hstream(&stream) == 0, "hipStreamCreate");
  check(hevent(&ev, 2u /* hipEventDisableTiming */) == 0, "hipEventCreateWithFlags");
  check(hsync() == 0, "hipDeviceSynchronize");
  double* t = (double*)malloc(sizeof(double) * (size_t)iters);
  for (int i = 0; i < warmup + iters; ++i) {
    const double t0 = now_us();
    check(int4(d[0], d[1], d[2], d[3], d[4], M, K, N, ws, wsb, stream) == 0, "mk_int4g64_matmul_bf16");
    check(hrecord(ev, stream) == 0, "hipEventRecord");
    int q;
    while ((q = hquery(ev)) == 600) {
    }
    check(q == 0, "hipEventQuery");
    if (i >= warmup) t[i - warmup] = now_us() - t0;
  }
  report("kernel C-ABI launch + hipEventRecord + hipEventQuery poll", t, iters);
  check(hedestroy(ev) == 0 && hsdestroy(stream) == 0, "destroy stream and event");
  for (int i = 0; i < 5; ++i) hfree(d[i]);
  if (ws) hfree(ws);
  free(t);
  return 0;
}

int main(int argc, char** argv) {
  if (argc >= 4 && strcmp(argv[1], "api") == 0) return mode_api(argv[2], argv[3]);
  if (argc >= 4 && strcmp(argv[1], "parse") == 0) return mode_fuzz(argc, argv, 1);
  if (argc >= 4 && strcmp(argv[1], "inspect") == 0) return mode_fuzz(argc, argv, 0);
  if (argc >= 5 && strcmp(argv[1], "run") == 0) return mode_run(argc, argv);
  if (argc >= 6 && strcmp(argv[1], "time") == 0) return mode_time(argc, argv);
  if (argc == 6 && strcmp(argv[1], "floor") == 0) return mode_floor(argv);
  fprintf(stderr, "usage: pjrt_harness api LIB gpu|nogpu | parse KLIB FILE... | inspect KLIB FILE... | "
                  "run LIB PROGRAM OUT TYPE:DIMS:PATH... | time LIB PROGRAM WARMUP ITERS TYPE:DIMS:PATH... | "
                  "floor KLIB HIPLIB WARMUP ITERS\n");
  return 2;
}
