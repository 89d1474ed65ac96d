// Runtime behind include/mk_runtime.h: one HIP device, one stream, a caching
// device allocator, completion events fired by a completion thread, and
// executables that run a kernel plan (planner.h).
//
// Ordering model.  Every device operation of a client (host<->device copies,
// kernel steps, copies between buffers) is issued on the client's single
// stream, so stream order alone makes buffer reuse safe: memory returned to
// the allocator can be handed out again at once, since any later user is
// queued behind every earlier reader.  Host-visible completion is tracked
// with events: each execute records a HIP event, and the completion thread
// waits for those in order and marks the matching mkrt_event ready,
// running its callbacks there (the reference's CompletionEvent fired from
// Metal's completion handler, core/completion_event.h:32-229).
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <condition_variable>
#include <deque>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "../ew_jit.h"
#include "mk_kernels.h"
#include "mk_runtime.h"
#include "mlir_bytecode.h"
#include "planner.h"
#include "shlo.h"

struct mkrt_error {
  int code;
  std::string message;
};

namespace {

mkrt_error* make_error(int code, const char* fmt, ...) {
  char buf[2048];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  return new mkrt_error{code, buf};
}

mkrt_error* copy_error(const mkrt_error* e) { return e ? new mkrt_error{e->code, e->message} : nullptr; }

// Shared state of one completion: ready flag, optional error, callbacks.
struct EventState {
  std::mutex mu;
  std::condition_variable cv;
  bool ready = false;
  int code = MKRT_OK;
  std::string message;
  std::vector<std::pair<mkrt_event_callback, void*>> callbacks;
  std::atomic<bool> done{false};  // `ready`, readable without the mutex

  void set(int c, const std::string& m) {
    std::vector<std::pair<mkrt_event_callback, void*>> cbs;
    {
      std::lock_guard<std::mutex> g(mu);
      if (ready) return;
      ready = true;
      code = c;
      message = m;
      cbs.swap(callbacks);
      done.store(true, std::memory_order_release);
    }
    cv.notify_all();
    for (auto& cb : cbs) cb.first(c == MKRT_OK ? nullptr : new mkrt_error{c, m}, cb.second);
  }
};

std::shared_ptr<EventState> ready_state(int code = MKRT_OK, const std::string& msg = std::string()) {
  auto s = std::make_shared<EventState>();
  s->ready = true;
  s->done.store(true, std::memory_order_relaxed);
  s->code = code;
  s->message = msg;
  return s;
}

// Completions are first polled for up to this long (MK_COMPLETION_SPIN_US,
// default 200 us; 0 disables) before the waiting thread blocks: a blocking
// wait's wake-up costs more than a short kernel takes.
int64_t spin_us() {
  static const int64_t v = [] {
    const char* e = getenv("MK_COMPLETION_SPIN_US");
    return e && *e ? std::max<int64_t>(0, atoll(e)) : 200;
  }();
  return v;
}

// Polls `ready()` until it holds or spin_us() has passed; true if it held.
template <typename F>
bool spin_until(F ready) {
  const int64_t us = spin_us();
  if (us <= 0) return ready();
  const auto end = std::chrono::steady_clock::now() + std::chrono::microseconds(us);
  for (int i = 0;; ++i) {
    if (ready()) return true;
    if ((i & 63) == 63 && std::chrono::steady_clock::now() >= end) return ready();
  }
}

int64_t default_timeout_ms() {
  const char* v = getenv("MK_COMPLETION_TIMEOUT_MS");
  if (v && *v) {
    const long long t = atoll(v);
    if (t > 0) return t;
  }
  return 30000;
}

// Caching allocator: freed blocks are kept per rounded size and handed out
// again in stream order.  Sizes round to 512 B below 1 MiB and to 2 MiB above.
class Allocator {
 public:
  ~Allocator() { release_cached(); }

  static size_t round(size_t n) {
    if (n == 0) return 0;
    if (n < (1u << 20)) return (n + 511) & ~(size_t)511;
    return (n + (2u << 20) - 1) & ~(((size_t)2 << 20) - 1);
  }

  hipError_t alloc(size_t bytes, void** out) {
    *out = nullptr;
    const size_t r = round(bytes);
    if (r == 0) return hipSuccess;
    {
      std::lock_guard<std::mutex> g(mu_);
      auto it = free_.find(r);
      if (it != free_.end()) {
        *out = it->second;
        free_.erase(it);
        cached_ -= r;
        in_use_ += r;
        sizes_[*out] = r;
        return hipSuccess;
      }
    }
    hipError_t e = hipMalloc(out, r);
    if (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation) {
      (void)hipGetLastError();
      release_cached();
      e = hipMalloc(out, r);
    }
    if (e != hipSuccess) {
      *out = nullptr;
      return e;
    }
    std::lock_guard<std::mutex> g(mu_);
    sizes_[*out] = r;
    in_use_ += r;
    return hipSuccess;
  }

  void free(void* p) {
    if (!p) return;
    std::lock_guard<std::mutex> g(mu_);
    auto it = sizes_.find(p);
    if (it == sizes_.end()) return;
    const size_t r = it->second;
    sizes_.erase(it);
    in_use_ -= r;
    cached_ += r;
    free_.emplace(r, p);
  }

  void release_cached() {
    std::multimap<size_t, void*> blocks;
    {
      std::lock_guard<std::mutex> g(mu_);
      blocks.swap(free_);
      cached_ = 0;
    }
    for (auto& b : blocks) (void)hipFree(b.second);
  }

  int64_t in_use() {
    std::lock_guard<std::mutex> g(mu_);
    return (int64_t)in_use_;
  }

 private:
  std::mutex mu_;
  std::multimap<size_t, void*> free_;
  std::map<void*, size_t> sizes_;
  size_t in_use_ = 0, cached_ = 0;
};

}  // namespace

struct mkrt_client {
  int device = 0;
  hipStream_t stream = nullptr;
  Allocator alloc;
  std::mutex stream_mu;  // serialises multi-call sequences on the stream

  // Completion thread.
  std::mutex q_mu;
  std::condition_variable q_cv;
  std::deque<std::pair<hipEvent_t, std::shared_ptr<EventState>>> queue;
  bool stopping = false;
  std::thread worker;
  std::mutex ev_pool_mu;
  std::vector<hipEvent_t> ev_pool;

  hipEvent_t get_event() {
    {
      std::lock_guard<std::mutex> g(ev_pool_mu);
      if (!ev_pool.empty()) {
        hipEvent_t e = ev_pool.back();
        ev_pool.pop_back();
        return e;
      }
    }
    hipEvent_t e = nullptr;
    if (hipEventCreateWithFlags(&e, hipEventDisableTiming | hipEventBlockingSync) != hipSuccess) return nullptr;
    return e;
  }

  void completion_loop() {
    (void)hipSetDevice(device);
    while (true) {
      std::pair<hipEvent_t, std::shared_ptr<EventState>> item;
      {
        std::unique_lock<std::mutex> l(q_mu);
        q_cv.wait(l, [&] { return stopping || !queue.empty(); });
        if (queue.empty()) return;
        item = queue.front();
        queue.pop_front();
      }
      hipError_t e = hipErrorNotReady;
      spin_until([&] { return (e = hipEventQuery(item.first)) != hipErrorNotReady; });
      if (e == hipErrorNotReady) e = hipEventSynchronize(item.first);
      {
        std::lock_guard<std::mutex> g(ev_pool_mu);
        ev_pool.push_back(item.first);
      }
      if (e == hipSuccess) item.second->set(MKRT_OK, std::string());
      else item.second->set(MKRT_INTERNAL, std::string("device execution failed: ") + hipGetErrorString(e));
    }
  }

  // Marks `st` ready once everything issued so far on the stream has run.
  hipError_t track(const std::shared_ptr<EventState>& st) {
    hipEvent_t e = get_event();
    if (!e) return hipErrorOutOfMemory;
    hipError_t r = hipEventRecord(e, stream);
    if (r != hipSuccess) {
      std::lock_guard<std::mutex> g(ev_pool_mu);
      ev_pool.push_back(e);
      return r;
    }
    {
      std::lock_guard<std::mutex> g(q_mu);
      queue.emplace_back(e, st);
    }
    q_cv.notify_one();
    return hipSuccess;
  }
};

struct mkrt_buffer {
  mkrt_client* client = nullptr;
  int type = 0;
  std::vector<int64_t> dims;
  int64_t bytes = 0;
  void* data = nullptr;
  std::shared_ptr<EventState> ready;  // producer
  // A view of memory the caller owns (CreateViewOfDeviceBuffer): released
  // through the callback instead of the allocator.
  bool view = false;
  mkrt_release_callback on_release = nullptr;
  void* release_user = nullptr;
  bool deleted = false;  // device memory released, handle still valid
};

struct mkrt_event {
  std::shared_ptr<EventState> st;
};

struct mkrt_executable {
  mkrt_client* client = nullptr;
  std::string program;      // the program bytes it was compiled from (text or bytecode)
  std::string program_text; // its MLIR text (the bytecode's decoded text)
  std::string fingerprint;  // 16 hex digits of FNV-1a 64 over program
  mkrt::Function fn;
  mkrt::Plan plan;
  std::string plan_text;
  std::mutex plan_mu;
  std::atomic<bool> prepared{false};
  std::vector<void*> const_mem;  // per slot, SLOT_CONST only
  void* workspace = nullptr;
};

namespace {

int64_t dims_numel(const int64_t* dims, int ndims) {
  int64_t n = 1;
  for (int i = 0; i < ndims; ++i) n *= dims[i];
  return n;
}

mkrt_error* hip_error(const char* what, hipError_t e) {
  return make_error(MKRT_INTERNAL, "%s: %s", what, hipGetErrorString(e));
}

mkrt_error* await_state(const std::shared_ptr<EventState>& st, int64_t timeout_ms) {
  if (timeout_ms < 0) timeout_ms = default_timeout_ms();
  spin_until([&] { return st->done.load(std::memory_order_acquire); });
  std::unique_lock<std::mutex> l(st->mu);
  if (!st->cv.wait_for(l, std::chrono::milliseconds(timeout_ms), [&] { return st->ready; }))
    return make_error(MKRT_DEADLINE_EXCEEDED, "completion not signalled within %lld ms (MK_COMPLETION_TIMEOUT_MS)",
                      (long long)timeout_ms);
  if (st->code != MKRT_OK) return new mkrt_error{st->code, st->message};
  return nullptr;
}

mkrt_buffer* new_buffer(mkrt_client* c, int type, const std::vector<int64_t>& dims, void* data, int64_t bytes,
                        std::shared_ptr<EventState> ready) {
  mkrt_buffer* b = new mkrt_buffer;
  b->client = c;
  b->type = type;
  b->dims = dims;
  b->bytes = bytes;
  b->data = data;
  b->ready = std::move(ready);
  return b;
}

// First-execute preparation: constants uploaded, workspace allocated,
// elementwise programs compiled (core/mps_executable.mm:9152 builds the
// plan lazily under plan_mutex_, mps_executable.h:96-100).
// GEMM routes measured at the first plan build, as the reference autotunes
// its GEMM variants (AutotuneGemm, src/pjrt_plugin/core/mps_executable.mm:
// 3433-3725): MK_GEMM_AUTOTUNE=0 keeps the built-in choice.  The route table
// persists across processes as gemm_routes.txt in the library's cache
// directory (MK_CACHE_DIR; none with MK_DISABLE_CACHE_PERSIST=1), as the
// reference's cache does (:3270-3420).  Every route gives the same bits, so
// this only changes speed.
bool gemm_autotune_enabled() {
  const char* v = getenv("MK_GEMM_AUTOTUNE");
  return !(v && v[0] == '0' && v[1] == '\0');
}

std::string gemm_route_cache_path() {
  const std::string dir = mkc::cache_directory();
  return dir.empty() ? dir : dir + "/gemm_routes.txt";
}

std::mutex g_route_cache_mu;
bool g_route_cache_loaded = false;

// Fills st.route of every [K, N] bf16 GEMM step: the table's entry, or a
// measurement on scratch operands of the step's sizes (bf16 0x3c3c, about
// 0.0115, everywhere).  A failed measurement leaves the built-in choice.
// Called with the client's stream lock held.
void tune_gemm_steps(mkrt_executable* x) {
  if (!gemm_autotune_enabled()) return;
  mkrt_client* c = x->client;
  const std::string path = gemm_route_cache_path();
  {
    std::lock_guard<std::mutex> g(g_route_cache_mu);
    if (!g_route_cache_loaded && !path.empty()) {
      FILE* f = fopen(path.c_str(), "r");
      if (f) {
        fclose(f);
        mk_gemm_autotune_load(path.c_str());  // a malformed file is ignored
      }
    }
    g_route_cache_loaded = true;
  }
  bool added = false;
  for (mkrt::Step& st : x->plan.steps) {
    if (st.kind != mkrt::ST_GEMM_BF16 || st.b_t) continue;
    int r = mk_gemm_tuned_route(st.batch, st.M, st.N, st.K, MK_EPI_NONE, st.out_f32);
    if (r == MK_GEMM_ROUTE_DEFAULT) {
      const size_t ab = (size_t)(st.batch * st.M * st.K * 2), bb = (size_t)(st.batch * st.K * st.N * 2);
      const size_t cb = (size_t)(st.batch * st.M * st.N * (st.out_f32 ? 4 : 2));
      void *A = nullptr, *B = nullptr, *C = nullptr;
      if (c->alloc.alloc(ab, &A) == hipSuccess && c->alloc.alloc(bb, &B) == hipSuccess &&
          c->alloc.alloc(cb, &C) == hipSuccess && hipMemsetAsync(A, 0x3c, ab, c->stream) == hipSuccess &&
          hipMemsetAsync(B, 0x3c, bb, c->stream) == hipSuccess) {
        int route = 0;
        float us = 0.f;
        if (mk_gemm_bf16_autotune(A, B, C, nullptr, MK_EPI_NONE, st.batch, st.M, st.N, st.K, st.out_f32, c->stream,
                                  &route, &us) == MK_OK) {
          r = route;
          added = true;
        }
      }
      (void)hipStreamSynchronize(c->stream);
      for (void* q : {A, B, C})
        if (q) c->alloc.free(q);
    }
    st.route = r;
  }
  if (added && !path.empty()) {
    std::lock_guard<std::mutex> g(g_route_cache_mu);
    mk_gemm_autotune_save(path.c_str());  // best effort: an unwritable cache only costs a re-measurement
  }
}

mkrt_error* prepare(mkrt_executable* x) {
  if (x->prepared.load(std::memory_order_acquire)) return nullptr;
  std::lock_guard<std::mutex> g(x->plan_mu);
  if (x->prepared.load(std::memory_order_relaxed)) return nullptr;
  mkrt_client* c = x->client;
  x->const_mem.assign(x->plan.slots.size(), nullptr);
  for (size_t i = 0; i < x->plan.slots.size(); ++i) {
    const mkrt::Slot& s = x->plan.slots[i];
    if (s.kind != mkrt::SLOT_CONST || s.bytes == 0) continue;
    void* p = nullptr;
    hipError_t e = c->alloc.alloc((size_t)s.bytes, &p);
    if (e != hipSuccess) return hip_error("constant allocation", e);
    x->const_mem[i] = p;
    std::lock_guard<std::mutex> sg(c->stream_mu);
    e = hipMemcpyAsync(p, s.data.data(), (size_t)s.bytes, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) return hip_error("constant upload", e);
  }
  if (x->plan.workspace_bytes > 0) {
    // The dequant-matmul workspace starts zero-filled (its arrival counters).
    hipError_t e = c->alloc.alloc((size_t)x->plan.workspace_bytes, &x->workspace);
    if (e != hipSuccess) return hip_error("workspace allocation", e);
    std::lock_guard<std::mutex> sg(c->stream_mu);
    e = hipMemsetAsync(x->workspace, 0, (size_t)x->plan.workspace_bytes, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) return hip_error("workspace clear", e);
  }
  for (const mkrt::Step& st : x->plan.steps) {
    if (st.kind != mkrt::ST_EW) continue;
    if (mk_elementwise_prepare(st.dt, st.prog.data(), (int)st.prog.size(), (int)st.in.size(), st.prog_out) != MK_OK)
      return make_error(MKRT_INTERNAL, "elementwise program: %s", mk_last_error());
  }
  {
    std::lock_guard<std::mutex> sg(c->stream_mu);
    tune_gemm_steps(x);
  }
  x->prepared.store(true, std::memory_order_release);
  return nullptr;
}

int run_step(const mkrt::Step& st, const std::vector<void*>& mem, void* ws, int64_t ws_bytes, hipStream_t s) {
  auto in = [&](int i) { return (const void*)mem[st.in[i]]; };
  void* out = mem[st.out];
  switch (st.kind) {
    case mkrt::ST_GEMM_BF16:
      if (st.b_t) return mk_gemm_bf16_nt(in(0), in(1), out, nullptr, MK_EPI_NONE, st.batch, st.M, st.N, st.K, s);
      if (st.route != MK_GEMM_ROUTE_DEFAULT)
        return mk_gemm_bf16_route(in(0), in(1), out, nullptr, MK_EPI_NONE, st.batch, st.M, st.N, st.K, st.out_f32,
                                  st.route, s);
      return mk_gemm_bf16(in(0), in(1), out, st.batch, st.M, st.N, st.K, st.out_f32, s);
    case mkrt::ST_GEMM_F32:
      return mk_gemm_f32(in(0), in(1), out, st.batch, st.M, st.N, st.K, s);
    case mkrt::ST_QMM_INT4:
      if (st.epi != MK_EPI_NONE)
        return mk_int4g64_matmul_epilogue_bf16(in(0), in(1), in(2), in(3), out, in(4), st.epi, st.M, st.K, st.N, ws,
                                               ws_bytes, s);
      return mk_int4g64_matmul_bf16(in(0), in(1), in(2), in(3), out, st.M, st.K, st.N, ws, ws_bytes, s);
    case mkrt::ST_QMM_INT8:
      if (st.epi != MK_EPI_NONE)
        return mk_int8pc_matmul_epilogue_bf16(in(0), in(1), in(2), out, in(3), st.epi, st.M, st.K, st.N, ws, ws_bytes,
                                              s);
      return mk_int8pc_matmul_bf16(in(0), in(1), in(2), out, st.M, st.K, st.N, ws, ws_bytes, s);
    case mkrt::ST_QMM_PAIR_INT4:
      return mk_int4g64_matmul_swiglu_pair_bf16(in(0), in(1), in(2), in(3), in(4), in(5), in(6), out, st.M, st.K,
                                                st.N, ws, ws_bytes, s);
    case mkrt::ST_QMM_PAIR_INT8:
      return mk_int8pc_matmul_swiglu_pair_bf16(in(0), in(1), in(2), in(3), in(4), out, st.M, st.K, st.N, ws, ws_bytes,
                                               s);
    case mkrt::ST_SOFTMAX:
      return mk_softmax_lastdim(st.dt, in(0), out, st.rows, st.cols, s);
    case mkrt::ST_RMSNORM:
      return mk_rmsnorm_lastdim(st.dt, in(0), in(1), out, st.rows, st.cols, st.eps, s);
    case mkrt::ST_ARGMAX:
      return mk_argmax_lastdim(st.dt, in(0), out, st.rows, st.cols, s);
    case mkrt::ST_REDUCE:
      return mk_reduce_lastdim(st.dt, st.reduce_op, in(0), out, st.rows, st.cols, s);
    case mkrt::ST_EW: {
      std::vector<const void*> ins;
      for (size_t i = 0; i < st.in.size(); ++i) ins.push_back(in((int)i));
      return mk_elementwise(st.dt, st.prog.data(), (int)st.prog.size(), ins.data(), st.in_numel.data(),
                            (int)ins.size(), st.prog_out, out, st.n, s);
    }
    case mkrt::ST_COPY:
      if (st.bytes == 0) return MK_OK;
      return hipMemcpyAsync(out, in(0), (size_t)st.bytes, hipMemcpyDeviceToDevice, s) == hipSuccess ? MK_OK
                                                                                                     : MK_ELAUNCH;
    case mkrt::ST_DOT_GENERIC:
      return mk_dot_general(st.type_a, st.type_a, st.type_out, in(0), in(1), out, st.batch, st.M, st.N, st.K, st.sa,
                            st.sb, s);
    case mkrt::ST_ZERO:
      if (st.bytes == 0) return MK_OK;
      return hipMemsetAsync(out, 0, (size_t)st.bytes, s) == hipSuccess ? MK_OK : MK_ELAUNCH;
    case mkrt::ST_LAYOUT:
      return mk_strided_copy(in(0), out, st.elem_bytes, (int)st.shape.size(), st.shape.data(), st.src_st.data(),
                             st.src_off, st.dst_st.data(), st.dst_off, s);
    case mkrt::ST_IOTA:
      return mk_iota(out, st.type_out, (int)st.shape.size(), st.shape.data(), st.iota_dim, s);
    case mkrt::ST_ROPE:
      return mk_rope_qkv_split_bf16(in(0), static_cast<const float*>(in(1)), static_cast<const float*>(in(2)), out,
                                    mem[st.outs[0]], mem[st.outs[1]], st.B, st.S, st.H, st.D, 1, s);
    case mkrt::ST_ATTN:
      return mk_attention_causal_bf16(in(0), in(1), in(2), out, st.B, st.H, st.S, st.D, st.scale, s);
  }
  return MK_EUNSUPPORTED;
}

}  // namespace

extern "C" {

void mkrt_error_destroy(mkrt_error* err) { delete err; }
const char* mkrt_error_message(const mkrt_error* err) { return err ? err->message.c_str() : ""; }
int mkrt_error_code(const mkrt_error* err) { return err ? err->code : MKRT_OK; }

mkrt_error* mkrt_client_create(mkrt_client** out) {
  if (!out) return make_error(MKRT_INVALID_ARGUMENT, "mkrt_client_create: null out");
  *out = nullptr;
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n < 1) {
    (void)hipGetLastError();
    return make_error(MKRT_UNAVAILABLE, "no HIP device available (%s)", hipGetErrorString(e));
  }
  e = hipSetDevice(0);
  if (e != hipSuccess) return hip_error("hipSetDevice", e);
  mkrt_client* c = new mkrt_client;
  e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    delete c;
    return hip_error("hipStreamCreate", e);
  }
  c->worker = std::thread([c] { c->completion_loop(); });
  *out = c;
  return nullptr;
}

void mkrt_client_destroy(mkrt_client* c) {
  if (!c) return;
  (void)hipStreamSynchronize(c->stream);
  {
    std::lock_guard<std::mutex> g(c->q_mu);
    c->stopping = true;
  }
  c->q_cv.notify_all();
  if (c->worker.joinable()) c->worker.join();
  for (hipEvent_t e : c->ev_pool) (void)hipEventDestroy(e);
  (void)hipStreamDestroy(c->stream);
  delete c;
}

const char* mkrt_client_platform_name(const mkrt_client*) { return "mi355x"; }

mkrt_error* mkrt_client_memory_stats(mkrt_client* c, int64_t* bytes_in_use, int64_t* bytes_limit) {
  if (!c || !bytes_in_use || !bytes_limit) return make_error(MKRT_INVALID_ARGUMENT, "mkrt_client_memory_stats: null argument");
  size_t fr = 0, total = 0;
  hipError_t e = hipMemGetInfo(&fr, &total);
  if (e != hipSuccess) return hip_error("hipMemGetInfo", e);
  *bytes_in_use = c->alloc.in_use();
  *bytes_limit = (int64_t)total;
  return nullptr;
}

mkrt_error* mkrt_buffer_from_host(mkrt_client* c, const void* data, int type, const int64_t* dims, int ndims,
                                  mkrt_buffer** out, mkrt_event** done_with_host) {
  if (!c || !out || (ndims > 0 && !dims) || ndims < 0)
    return make_error(MKRT_INVALID_ARGUMENT, "mkrt_buffer_from_host: null argument");
  *out = nullptr;
  const int eb = mkrt::dtype_bytes(type);
  if (eb == 0) return make_error(MKRT_INVALID_ARGUMENT, "mkrt_buffer_from_host: unsupported element type %d", type);
  for (int i = 0; i < ndims; ++i)
    if (dims[i] < 0) return make_error(MKRT_INVALID_ARGUMENT, "mkrt_buffer_from_host: negative dimension");
  const int64_t bytes = dims_numel(dims, ndims) * eb;
  if (bytes > 0 && !data) return make_error(MKRT_INVALID_ARGUMENT, "mkrt_buffer_from_host: null data");
  void* p = nullptr;
  hipError_t e = c->alloc.alloc((size_t)bytes, &p);
  if (e != hipSuccess) return make_error(MKRT_RESOURCE_EXHAUSTED, "device allocation of %lld bytes: %s",
                                         (long long)bytes, hipGetErrorString(e));
  if (bytes > 0) {
    std::lock_guard<std::mutex> g(c->stream_mu);
    e = hipMemcpyAsync(p, data, (size_t)bytes, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) {
      c->alloc.free(p);
      return hip_error("host-to-device copy", e);
    }
  }
  *out = new_buffer(c, type, std::vector<int64_t>(dims, dims + ndims), p, bytes, ready_state());
  if (done_with_host) *done_with_host = new mkrt_event{ready_state()};
  return nullptr;
}

mkrt_error* mkrt_buffer_to_host(mkrt_buffer* b, void* dst, int64_t dst_bytes, mkrt_event** done) {
  if (!b) return make_error(MKRT_INVALID_ARGUMENT, "mkrt_buffer_to_host: null buffer");
  if (done) *done = nullptr;
  if (b->deleted) return make_error(MKRT_FAILED_PRECONDITION, "mkrt_buffer_to_host: the buffer has been deleted");
  if (dst_bytes < b->bytes || (b->bytes > 0 && !dst))
    return make_error(MKRT_INVALID_ARGUMENT, "mkrt_buffer_to_host: destination holds %lld bytes, buffer has %lld",
                      (long long)dst_bytes, (long long)b->bytes);
  if (mkrt_error* err = await_state(b->ready, -1)) return err;
  if (b->bytes > 0) {
    std::lock_guard<std::mutex> g(b->client->stream_mu);
    hipError_t e = hipMemcpyAsync(dst, b->data, (size_t)b->bytes, hipMemcpyDeviceToHost, b->client->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(b->client->stream);
    if (e != hipSuccess) return hip_error("device-to-host copy", e);
  }
  if (done) *done = new mkrt_event{ready_state()};
  return nullptr;
}

int mkrt_buffer_type(const mkrt_buffer* b) { return b ? b->type : 0; }
int mkrt_buffer_ndims(const mkrt_buffer* b) { return b ? (int)b->dims.size() : 0; }
const int64_t* mkrt_buffer_dims(const mkrt_buffer* b) { return b ? b->dims.data() : nullptr; }
int64_t mkrt_buffer_bytes(const mkrt_buffer* b) { return b ? b->bytes : 0; }

mkrt_error* mkrt_buffer_ready_event(mkrt_buffer* b, mkrt_event** out) {
  if (!b || !out) return make_error(MKRT_INVALID_ARGUMENT, "mkrt_buffer_ready_event: null argument");
  *out = new mkrt_event{b->ready};
  return nullptr;
}

mkrt_error* mkrt_buffer_create_error(mkrt_client* c, int code, const char* message, int type, const int64_t* dims,
                                     int ndims, mkrt_buffer** out) {
  if (!c || !out || (ndims > 0 && !dims) || ndims < 0)
    return make_error(MKRT_INVALID_ARGUMENT, "mkrt_buffer_create_error: null argument");
  if (code == MKRT_OK) return make_error(MKRT_INVALID_ARGUMENT, "mkrt_buffer_create_error: code must not be OK");
  const int eb = mkrt::dtype_bytes(type);
  *out = new_buffer(c, type, std::vector<int64_t>(dims, dims + ndims), nullptr,
                    eb ? dims_numel(dims, ndims) * eb : 0, ready_state(code, message ? message : ""));
  return nullptr;
}

// Returns the buffer's device memory: waits for the producer
// (core/mps_buffer.mm:656-662); later users of the memory are ordered behind
// every earlier reader on the stream.  A view's memory goes back to its owner
// through the release callback, after the stream has drained, since the
// owner may reuse it at once.
static void release_memory(mkrt_buffer* b) {
  if (b->deleted) return;
  b->deleted = true;
  if (!b->data && !b->view) return;
  {
    std::unique_lock<std::mutex> l(b->ready->mu);
    b->ready->cv.wait(l, [&] { return b->ready->ready; });
  }
  if (b->view) {
    {
      std::lock_guard<std::mutex> g(b->client->stream_mu);
      (void)hipStreamSynchronize(b->client->stream);
    }
    if (b->on_release) b->on_release(b->data, b->release_user);
  } else {
    b->client->alloc.free(b->data);
  }
  b->data = nullptr;
}

void mkrt_buffer_destroy(mkrt_buffer* b) {
  if (!b) return;
  release_memory(b);
  delete b;
}

void mkrt_buffer_delete(mkrt_buffer* b) {
  if (b) release_memory(b);
}

int mkrt_buffer_is_deleted(const mkrt_buffer* b) { return !b || b->deleted ? 1 : 0; }

void* mkrt_buffer_device_pointer(const mkrt_buffer* b) { return b && !b->deleted ? b->data : nullptr; }

// Element count and bytes of a shape, rejecting negative dimensions and
// types the runtime does not hold.
static mkrt_error* shape_bytes(const char* fn, int type, const int64_t* dims, int ndims, int64_t* bytes) {
  if ((ndims > 0 && !dims) || ndims < 0) return make_error(MKRT_INVALID_ARGUMENT, "%s: null dims", fn);
  const int eb = mkrt::dtype_bytes(type);
  if (eb == 0) return make_error(MKRT_INVALID_ARGUMENT, "%s: unsupported element type %d", fn, type);
  int64_t n = 1;
  for (int i = 0; i < ndims; ++i) {
    if (dims[i] < 0) return make_error(MKRT_INVALID_ARGUMENT, "%s: negative dimension", fn);
    if (dims[i] > 0 && n > ((int64_t)1 << 46) / dims[i]) return make_error(MKRT_INVALID_ARGUMENT, "%s: shape too large", fn);
    n *= dims[i];
  }
  *bytes = n * eb;
  return nullptr;
}

mkrt_error* mkrt_buffer_from_host_strided(mkrt_client* c, const void* data, int type, const int64_t* dims, int ndims,
                                          const int64_t* byte_strides, int num_strides, mkrt_buffer** out,
                                          mkrt_event** done_with_host) {
  if (!c || !out) return make_error(MKRT_INVALID_ARGUMENT, "BufferFromHostBuffer: null argument");
  *out = nullptr;
  if (done_with_host) *done_with_host = nullptr;
  if (!byte_strides || num_strides == 0)
    return mkrt_buffer_from_host(c, data, type, dims, ndims, out, done_with_host);
  int64_t bytes = 0;
  if (mkrt_error* e = shape_bytes("BufferFromHostBuffer", type, dims, ndims, &bytes)) return e;
  if (num_strides != ndims)
    return make_error(MKRT_INVALID_ARGUMENT, "BufferFromHostBuffer: %d byte strides for %d dimensions", num_strides,
                      ndims);
  const int64_t eb = mkrt::dtype_bytes(type);
  // Dense row-major already: one copy.
  bool dense = true;
  int64_t expect = eb;
  for (int i = ndims - 1; i >= 0; --i) {
    if (dims[i] > 1 && byte_strides[i] != expect) dense = false;
    expect *= dims[i];
  }
  if (dense || bytes == 0) return mkrt_buffer_from_host(c, data, type, dims, ndims, out, done_with_host);
  if (!data) return make_error(MKRT_INVALID_ARGUMENT, "BufferFromHostBuffer: null data");
  // Gather the strided host array into a dense row-major staging copy
  // (mps_client.mm:133-176 copies element by element the same way).
  std::vector<unsigned char> dense_copy((size_t)bytes);
  std::vector<int64_t> idx(ndims, 0);
  const unsigned char* src = static_cast<const unsigned char*>(data);
  const int64_t n = bytes / eb;
  for (int64_t k = 0; k < n; ++k) {
    int64_t off = 0;
    for (int i = 0; i < ndims; ++i) off += idx[i] * byte_strides[i];
    memcpy(dense_copy.data() + k * eb, src + off, (size_t)eb);
    for (int i = ndims - 1; i >= 0; --i) {
      if (++idx[i] < dims[i]) break;
      idx[i] = 0;
    }
  }
  return mkrt_buffer_from_host(c, dense_copy.data(), type, dims, ndims, out, done_with_host);
}

mkrt_error* mkrt_buffer_copy_raw_to_host(mkrt_buffer* b, void* dst, int64_t offset, int64_t size, mkrt_event** done) {
  if (done) *done = nullptr;
  if (!b || (!dst && size > 0)) return make_error(MKRT_INVALID_ARGUMENT, "CopyRawToHost: null argument");
  if (b->deleted) return make_error(MKRT_FAILED_PRECONDITION, "CopyRawToHost: the buffer has been deleted");
  if (offset < 0 || size < 0 || offset > b->bytes || size > b->bytes - offset)
    return make_error(MKRT_INVALID_ARGUMENT, "CopyRawToHost: range [%lld, %lld) outside the buffer's %lld bytes",
                      (long long)offset, (long long)(offset + size), (long long)b->bytes);
  if (mkrt_error* err = await_state(b->ready, -1)) return err;
  if (size > 0) {
    std::lock_guard<std::mutex> g(b->client->stream_mu);
    hipError_t e = hipMemcpyAsync(dst, static_cast<unsigned char*>(b->data) + offset, (size_t)size,
                                  hipMemcpyDeviceToHost, b->client->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(b->client->stream);
    if (e != hipSuccess) return hip_error("device-to-host copy", e);
  }
  if (done) *done = new mkrt_event{ready_state()};
  return nullptr;
}

mkrt_error* mkrt_buffer_create_view(mkrt_client* c, void* device_ptr, int type, const int64_t* dims, int ndims,
                                    mkrt_release_callback on_release, void* user, mkrt_buffer** out) {
  if (!c || !out) return make_error(MKRT_INVALID_ARGUMENT, "CreateViewOfDeviceBuffer: null argument");
  *out = nullptr;
  if (!device_ptr) return make_error(MKRT_INVALID_ARGUMENT, "CreateViewOfDeviceBuffer: null device_buffer_ptr");
  int64_t bytes = 0;
  if (mkrt_error* e = shape_bytes("CreateViewOfDeviceBuffer", type, dims, ndims, &bytes)) return e;
  mkrt_buffer* b = new_buffer(c, type, std::vector<int64_t>(dims, dims + ndims), device_ptr, bytes, ready_state());
  b->view = true;
  b->on_release = on_release;
  b->release_user = user;
  *out = b;
  return nullptr;
}

mkrt_error* mkrt_buffer_create_uninitialized(mkrt_client* c, int type, const int64_t* dims, int ndims,
                                             mkrt_buffer** out) {
  if (!c || !out) return make_error(MKRT_INVALID_ARGUMENT, "CreateUninitializedBuffer: null argument");
  *out = nullptr;
  int64_t bytes = 0;
  if (mkrt_error* e = shape_bytes("CreateUninitializedBuffer", type, dims, ndims, &bytes)) return e;
  void* p = nullptr;
  hipError_t e = c->alloc.alloc((size_t)bytes, &p);
  if (e != hipSuccess)
    return make_error(MKRT_RESOURCE_EXHAUSTED, "device allocation of %lld bytes: %s", (long long)bytes,
                      hipGetErrorString(e));
  *out = new_buffer(c, type, std::vector<int64_t>(dims, dims + ndims), p, bytes, ready_state());
  return nullptr;
}

mkrt_error* mkrt_buffer_copy(mkrt_buffer* b, mkrt_buffer** out) {
  if (!b || !out) return make_error(MKRT_INVALID_ARGUMENT, "CopyToDevice: null argument");
  *out = nullptr;
  if (b->deleted) return make_error(MKRT_FAILED_PRECONDITION, "CopyToDevice: the buffer has been deleted");
  {
    std::lock_guard<std::mutex> g(b->ready->mu);
    if (b->ready->ready && b->ready->code != MKRT_OK) {
      *out = new_buffer(b->client, b->type, b->dims, nullptr, b->bytes, ready_state(b->ready->code, b->ready->message));
      return nullptr;
    }
  }
  mkrt_client* c = b->client;
  void* p = nullptr;
  hipError_t e = c->alloc.alloc((size_t)b->bytes, &p);
  if (e != hipSuccess)
    return make_error(MKRT_RESOURCE_EXHAUSTED, "device allocation of %lld bytes: %s", (long long)b->bytes,
                      hipGetErrorString(e));
  auto st = std::make_shared<EventState>();
  {
    // The copy is queued behind the producer on the client's one stream.
    std::lock_guard<std::mutex> g(c->stream_mu);
    if (b->bytes > 0) e = hipMemcpyAsync(p, b->data, (size_t)b->bytes, hipMemcpyDeviceToDevice, c->stream);
    if (e == hipSuccess) e = c->track(st);
  }
  if (e != hipSuccess) {
    c->alloc.free(p);
    return hip_error("device-to-device copy", e);
  }
  *out = new_buffer(c, b->type, b->dims, p, b->bytes, st);
  return nullptr;
}

}  // extern "C"

namespace {

// Parse + plan (no device work): the compile-time support check.
mkrt_error* compile_text(const char* code, int64_t code_bytes, const char* format, mkrt::Function* fn,
                         mkrt::Plan* plan, std::string* text_out = nullptr) {
  if (format && strcmp(format, "mlir") != 0)
    return make_error(MKRT_UNIMPLEMENTED, "program format '%s' is not supported (StableHLO MLIR text only)", format);
  std::string text(code, code_bytes >= 0 ? (size_t)code_bytes : strlen(code));
  if (mkrt::is_mlir_bytecode(text.data(), text.size())) {
    // A portable artifact (pjrt_client.cc:178-244): bytecode -> MLIR text.
    try {
      text = mkrt::mlir_bytecode_to_text(text.data(), text.size());
    } catch (const mkrt::BytecodeError& e) {
      return make_error(e.kind == mkrt::BytecodeError::UNSUPPORTED ? MKRT_UNIMPLEMENTED : MKRT_INVALID_ARGUMENT,
                        "MLIR bytecode: %s", e.what());
    } catch (const std::exception& e) {
      return make_error(MKRT_INVALID_ARGUMENT, "MLIR bytecode: %s", e.what());
    }
  }
  if (text_out) *text_out = text;
  try {
    *fn = mkrt::parse_stablehlo_text(text);
    *plan = mkrt::build_plan(*fn);
  } catch (const mkrt::PlanError& e) {
    return make_error(e.code, "%s", e.what());
  } catch (const std::exception& e) {
    return make_error(MKRT_INVALID_ARGUMENT, "StableHLO parse error: %s", e.what());
  }
  return nullptr;
}

std::string fingerprint_of(const std::string& program) {
  uint64_t h = 1469598103934665603ull;
  for (unsigned char ch : program) h = (h ^ ch) * 1099511628211ull;
  char b[20];
  snprintf(b, sizeof(b), "%016llx", (unsigned long long)h);
  return b;
}

// Serialized executable: "MKEX" | u32 version | u32 flags (0) | u64 tag
// bytes | tag | u64 program bytes | program | u32 code objects | per object:
// u64 source bytes | source | u64 code bytes | code.  Little-endian.  The
// tag is the elementwise compile tag (hiprtc version and options) the code
// objects were built under.
constexpr uint32_t kSerialVersion = 2;

void put_u32(std::string& b, uint32_t v) { b.append(reinterpret_cast<const char*>(&v), 4); }
void put_u64(std::string& b, uint64_t v) { b.append(reinterpret_cast<const char*>(&v), 8); }

mkrt_error* serialize_plan(const std::string& program, const mkrt::Plan& plan, std::string* out) {
  std::vector<std::pair<std::string, std::vector<char>>> objs;
  for (const mkrt::Step& st : plan.steps) {
    if (st.kind != mkrt::ST_EW) continue;
    std::string src;
    std::vector<char> code;
    if (mkc::ew_jit_code(st.dt, st.prog.data(), (int)st.prog.size(), (int)st.in.size(), st.prog_out, &src, &code) !=
        MK_OK)
      return make_error(MKRT_INTERNAL, "serialize: elementwise program: %s", mk_last_error());
    bool dup = false;
    for (const auto& o : objs) dup = dup || o.first == src;
    if (!dup) objs.emplace_back(std::move(src), std::move(code));
  }
  std::string& b = *out;
  b.clear();
  b.append("MKEX", 4);
  put_u32(b, kSerialVersion);
  put_u32(b, 0);
  const std::string& tag = mkc::ew_jit_tag();
  put_u64(b, tag.size());
  b += tag;
  put_u64(b, program.size());
  b += program;
  put_u32(b, (uint32_t)objs.size());
  for (const auto& o : objs) {
    put_u64(b, o.first.size());
    b += o.first;
    put_u64(b, o.second.size());
    b.append(o.second.data(), o.second.size());
  }
  return nullptr;
}

// Parsed view of a serialized executable (pointers into the caller's bytes).
struct SerialView {
  std::string tag;
  const char* program = nullptr;
  uint64_t program_bytes = 0;
  std::vector<std::pair<std::string, std::vector<char>>> objs;
};

mkrt_error* parse_serialized(const void* bytes, int64_t size, SerialView* v, bool copy_objects) {
  if (!bytes || size <= 0)
    return make_error(MKRT_INVALID_ARGUMENT, "DeserializeAndLoad: empty serialized data");
  const char* p = static_cast<const char*>(bytes);
  const char* end = p + size;
  auto take = [&](void* dst, size_t n) {
    if ((size_t)(end - p) < n) return false;
    memcpy(dst, p, n);
    p += n;
    return true;
  };
  char magic[4];
  uint32_t ver = 0, flags = 0, nobj = 0;
  if (!take(magic, 4) || memcmp(magic, "MKEX", 4) != 0)
    return make_error(MKRT_INVALID_ARGUMENT, "DeserializeAndLoad: not a serialized mi355x executable (bad magic)");
  if (!take(&ver, 4) || !take(&flags, 4))
    return make_error(MKRT_INVALID_ARGUMENT, "DeserializeAndLoad: truncated header");
  if (ver != kSerialVersion)
    return make_error(MKRT_INVALID_ARGUMENT, "DeserializeAndLoad: serialized format version %u, this build reads %u",
                      ver, kSerialVersion);
  uint64_t tag_bytes = 0;
  if (!take(&tag_bytes, 8) || (uint64_t)(end - p) < tag_bytes || tag_bytes > 4096)
    return make_error(MKRT_INVALID_ARGUMENT, "DeserializeAndLoad: truncated compile tag");
  v->tag.assign(p, tag_bytes);
  p += tag_bytes;
  if (!take(&v->program_bytes, 8) || (uint64_t)(end - p) < v->program_bytes)
    return make_error(MKRT_INVALID_ARGUMENT, "DeserializeAndLoad: truncated program");
  v->program = p;
  p += v->program_bytes;
  if (!take(&nobj, 4)) return make_error(MKRT_INVALID_ARGUMENT, "DeserializeAndLoad: truncated code-object table");
  for (uint32_t i = 0; i < nobj; ++i) {
    uint64_t sl = 0, cl = 0;
    if (!take(&sl, 8) || (uint64_t)(end - p) < sl)
      return make_error(MKRT_INVALID_ARGUMENT, "DeserializeAndLoad: truncated code object %u", i);
    const char* src = p;
    p += sl;
    if (!take(&cl, 8) || (uint64_t)(end - p) < cl || cl == 0)
      return make_error(MKRT_INVALID_ARGUMENT, "DeserializeAndLoad: truncated code object %u", i);
    const char* code = p;
    p += cl;
    if (copy_objects) v->objs.emplace_back(std::string(src, sl), std::vector<char>(code, code + cl));
    else v->objs.emplace_back(std::string(), std::vector<char>());
  }
  if (p != end) return make_error(MKRT_INVALID_ARGUMENT, "DeserializeAndLoad: %lld trailing bytes",
                                  (long long)(end - p));
  return nullptr;
}

}  // namespace

struct mkrt_serialized {
  std::string bytes;
};

extern "C" {

mkrt_error* mkrt_compile(mkrt_client* c, const char* code, int64_t code_bytes, const char* format,
                         mkrt_executable** out) {
  if (!c || !code || !out) return make_error(MKRT_INVALID_ARGUMENT, "mkrt_compile: null argument");
  *out = nullptr;
  mkrt_executable* x = new mkrt_executable;
  x->client = c;
  if (mkrt_error* err = compile_text(code, code_bytes, format, &x->fn, &x->plan, &x->program_text)) {
    delete x;
    return err;
  }
  x->program.assign(code, code_bytes >= 0 ? (size_t)code_bytes : strlen(code));
  x->fingerprint = fingerprint_of(x->program);
  x->plan_text = x->plan.describe();
  *out = x;
  return nullptr;
}

mkrt_error* mkrt_compile_check(const char* code, int64_t code_bytes, const char* format, char* plan_text,
                               int64_t plan_text_bytes, int* num_steps) {
  if (!code) return make_error(MKRT_INVALID_ARGUMENT, "mkrt_compile_check: null code");
  mkrt::Function fn;
  mkrt::Plan plan;
  if (mkrt_error* err = compile_text(code, code_bytes, format, &fn, &plan)) return err;
  if (num_steps) *num_steps = (int)plan.steps.size();
  if (plan_text && plan_text_bytes > 0) {
    const std::string t = plan.describe();
    const size_t n = std::min((size_t)plan_text_bytes - 1, t.size());
    memcpy(plan_text, t.data(), n);
    plan_text[n] = 0;
  }
  return nullptr;
}

mkrt_error* mkrt_bytecode_to_text(const char* data, int64_t size, char* text, int64_t text_bytes,
                                  int64_t* text_size) {
  if (!data || size < 0) return make_error(MKRT_INVALID_ARGUMENT, "mkrt_bytecode_to_text: null or negative input");
  std::string t;
  try {
    t = mkrt::mlir_bytecode_to_text(data, (size_t)size);
  } catch (const mkrt::BytecodeError& e) {
    return make_error(e.kind == mkrt::BytecodeError::UNSUPPORTED ? MKRT_UNIMPLEMENTED : MKRT_INVALID_ARGUMENT,
                      "MLIR bytecode: %s", e.what());
  } catch (const std::exception& e) {
    return make_error(MKRT_INVALID_ARGUMENT, "MLIR bytecode: %s", e.what());
  }
  if (text_size) *text_size = (int64_t)t.size();
  if (text && text_bytes > 0) {
    const size_t n = std::min((size_t)text_bytes - 1, t.size());
    memcpy(text, t.data(), n);
    text[n] = 0;
  }
  return nullptr;
}

int mkrt_executable_num_inputs(const mkrt_executable* x) { return x ? (int)x->plan.in_slot.size() : 0; }

int mkrt_executable_output_type(const mkrt_executable* x, int i) {
  return x && i >= 0 && i < (int)x->plan.out_type.size() ? x->plan.out_type[i].dtype : 0;
}
int mkrt_executable_output_ndims(const mkrt_executable* x, int i) {
  return x && i >= 0 && i < (int)x->plan.out_type.size() ? (int)x->plan.out_type[i].dims.size() : 0;
}
const int64_t* mkrt_executable_output_dims(const mkrt_executable* x, int i) {
  return x && i >= 0 && i < (int)x->plan.out_type.size() ? x->plan.out_type[i].dims.data() : nullptr;
}
const char* mkrt_executable_program(const mkrt_executable* x, int64_t* size) {
  if (size) *size = x ? (int64_t)x->program_text.size() : 0;
  return x ? x->program_text.data() : "";
}
int mkrt_executable_num_outputs(const mkrt_executable* x) { return x ? (int)x->plan.out_slot.size() : 0; }
int mkrt_executable_num_steps(const mkrt_executable* x) { return x ? (int)x->plan.steps.size() : 0; }
const char* mkrt_executable_plan(const mkrt_executable* x) { return x ? x->plan_text.c_str() : ""; }

mkrt_error* mkrt_execute(mkrt_executable* x, mkrt_buffer* const* inputs, int num_inputs, mkrt_buffer** outputs,
                         mkrt_event** done) {
  if (!x) return make_error(MKRT_INVALID_ARGUMENT, "No executable to execute");
  if (done) *done = nullptr;
  const mkrt::Plan& p = x->plan;
  if (num_inputs != (int)p.in_slot.size() || (num_inputs > 0 && !inputs) || (!outputs && !p.out_slot.empty()))
    return make_error(MKRT_INVALID_ARGUMENT, "mkrt_execute: expected %d inputs, got %d", (int)p.in_slot.size(),
                      num_inputs);
  for (int i = 0; i < num_inputs; ++i) {
    const mkrt_buffer* b = inputs[i];
    if (!b) return make_error(MKRT_INVALID_ARGUMENT, "mkrt_execute: input %d is null", i);
    if (b->client != x->client) return make_error(MKRT_INVALID_ARGUMENT, "mkrt_execute: input %d from another client", i);
    if (b->deleted) return make_error(MKRT_INVALID_ARGUMENT, "mkrt_execute: input %d has been deleted", i);
    if (b->type != p.in_type[i].dtype || b->dims != p.in_type[i].dims)
      return make_error(MKRT_INVALID_ARGUMENT, "mkrt_execute: input %d is %s, the program takes %s", i,
                        mkrt::TensorType{b->type, b->dims}.str().c_str(), p.in_type[i].str().c_str());
    std::lock_guard<std::mutex> g(b->ready->mu);
    if (b->ready->ready && b->ready->code != MKRT_OK)
      return make_error(b->ready->code, "mkrt_execute: input %d carries an error: %s", i, b->ready->message.c_str());
  }
  if (mkrt_error* err = prepare(x)) return err;
  mkrt_client* c = x->client;

  // Device memory for every slot.
  std::vector<void*> mem(p.slots.size(), nullptr);
  std::vector<char> is_out(p.slots.size(), 0);
  for (int s : p.out_slot) is_out[s] = 1;
  std::vector<void*> temps;
  mkrt_error* err = nullptr;
  for (size_t i = 0; i < p.slots.size() && !err; ++i) {
    const mkrt::Slot& s = p.slots[i];
    if (s.kind == mkrt::SLOT_ARG) {
      mem[i] = inputs[s.arg_index]->data;
    } else if (s.kind == mkrt::SLOT_CONST) {
      mem[i] = x->const_mem[i];
    } else if (s.kind == mkrt::SLOT_VIEW) {
      // A contiguous slice of an earlier argument or constant slot.
      mem[i] = static_cast<char*>(mem[s.base]) + s.offset;
    } else {
      hipError_t e = c->alloc.alloc((size_t)s.bytes, &mem[i]);
      if (e != hipSuccess)
        err = make_error(MKRT_RESOURCE_EXHAUSTED, "device allocation of %lld bytes: %s", (long long)s.bytes,
                         hipGetErrorString(e));
      else
        temps.push_back(mem[i]);
    }
  }
  auto st = std::make_shared<EventState>();
  if (!err) {
    std::lock_guard<std::mutex> g(c->stream_mu);
    for (size_t k = 0; k < p.steps.size() && !err; ++k) {
      const int rc = run_step(p.steps[k], mem, x->workspace, p.workspace_bytes, c->stream);
      if (rc != MK_OK)
        err = make_error(MKRT_INTERNAL, "step %zu (%s) failed: %s", k, p.steps[k].desc.c_str(),
                         rc == MK_ELAUNCH && mk_last_error()[0] == 0 ? "launch error" : mk_last_error());
    }
    if (!err) {
      hipError_t e = c->track(st);
      if (e != hipSuccess) err = hip_error("completion event", e);
    }
  }
  if (err) {
    // Memory is returned in stream order; anything already queued finishes
    // before a later user of the same blocks.
    for (void* t : temps) c->alloc.free(t);
    return err;
  }
  for (size_t i = 0; i < p.slots.size(); ++i)
    if (p.slots[i].kind == mkrt::SLOT_TEMP && !is_out[i]) c->alloc.free(mem[i]);
  for (size_t r = 0; r < p.out_slot.size(); ++r) {
    const mkrt::TensorType& t = p.out_type[r];
    outputs[r] = new_buffer(c, t.dtype, t.dims, mem[p.out_slot[r]], t.bytes(), st);
  }
  if (done) *done = new mkrt_event{st};
  return nullptr;
}

mkrt_error* mkrt_executable_serialize(const mkrt_executable* x, mkrt_serialized** out) {
  if (!x || !out) return make_error(MKRT_INVALID_ARGUMENT, "Serialize: null executable");
  *out = nullptr;
  mkrt_serialized* s = new mkrt_serialized;
  if (mkrt_error* e = serialize_plan(x->program, x->plan, &s->bytes)) {
    delete s;
    return e;
  }
  *out = s;
  return nullptr;
}

mkrt_error* mkrt_serialize_program(const char* code, int64_t code_bytes, const char* format, mkrt_serialized** out) {
  if (!code || !out) return make_error(MKRT_INVALID_ARGUMENT, "mkrt_serialize_program: null argument");
  *out = nullptr;
  mkrt::Function fn;
  mkrt::Plan plan;
  if (mkrt_error* e = compile_text(code, code_bytes, format, &fn, &plan)) return e;
  mkrt_serialized* s = new mkrt_serialized;
  const std::string program(code, code_bytes >= 0 ? (size_t)code_bytes : strlen(code));
  if (mkrt_error* e = serialize_plan(program, plan, &s->bytes)) {
    delete s;
    return e;
  }
  *out = s;
  return nullptr;
}

const void* mkrt_serialized_data(const mkrt_serialized* s) { return s ? s->bytes.data() : nullptr; }
int64_t mkrt_serialized_size(const mkrt_serialized* s) { return s ? (int64_t)s->bytes.size() : 0; }
void mkrt_serialized_destroy(mkrt_serialized* s) { delete s; }

mkrt_error* mkrt_serialized_inspect(const void* bytes, int64_t size, int64_t* program_bytes, int* num_code_objects) {
  SerialView v;
  if (mkrt_error* e = parse_serialized(bytes, size, &v, false)) return e;
  if (program_bytes) *program_bytes = (int64_t)v.program_bytes;
  if (num_code_objects) *num_code_objects = (int)v.objs.size();
  return nullptr;
}

mkrt_error* mkrt_deserialize(mkrt_client* c, const void* bytes, int64_t size, mkrt_executable** out) {
  if (!c || !out) return make_error(MKRT_INVALID_ARGUMENT, "DeserializeAndLoad: null argument");
  *out = nullptr;
  SerialView v;
  if (mkrt_error* e = parse_serialized(bytes, size, &v, true)) return e;
  // Code objects built by another toolchain or with other options are not
  // reused: the program's elementwise steps are then compiled again.
  if (v.tag == mkc::ew_jit_tag())
    for (const auto& o : v.objs) mkc::ew_jit_seed(o.first, o.second);
  mkrt_error* e = mkrt_compile(c, v.program, (int64_t)v.program_bytes, "mlir", out);
  if (e) {
    mkrt_error* w = make_error(e->code, "DeserializeAndLoad: %s", e->message.c_str());
    mkrt_error_destroy(e);
    return w;
  }
  return nullptr;
}

const char* mkrt_executable_fingerprint(const mkrt_executable* x) { return x ? x->fingerprint.c_str() : ""; }

void mkrt_jit_cache_stats(int64_t* compiles, int64_t* disk_hits, int64_t* memory_hits) {
  int64_t c = 0, d = 0, m = 0;
  mkc::ew_jit_stats(&c, &d, &m);
  if (compiles) *compiles = c;
  if (disk_hits) *disk_hits = d;
  if (memory_hits) *memory_hits = m;
}

void mkrt_executable_destroy(mkrt_executable* x) {
  if (!x) return;
  mkrt_client* c = x->client;
  for (void* p : x->const_mem) c->alloc.free(p);
  c->alloc.free(x->workspace);
  delete x;
}

mkrt_error* mkrt_event_create(mkrt_event** out) {
  if (!out) return make_error(MKRT_INVALID_ARGUMENT, "mkrt_event_create: null out");
  *out = new mkrt_event{std::make_shared<EventState>()};
  return nullptr;
}

mkrt_error* mkrt_event_set(mkrt_event* ev, int code, const char* message) {
  if (!ev) return make_error(MKRT_INVALID_ARGUMENT, "mkrt_event_set: null event");
  ev->st->set(code, message ? message : "");
  return nullptr;
}

int mkrt_event_is_ready(const mkrt_event* ev) {
  if (!ev) return 0;
  std::lock_guard<std::mutex> g(ev->st->mu);
  return ev->st->ready ? 1 : 0;
}

mkrt_error* mkrt_event_error(const mkrt_event* ev) {
  if (!ev) return make_error(MKRT_INVALID_ARGUMENT, "mkrt_event_error: null event");
  std::lock_guard<std::mutex> g(ev->st->mu);
  if (!ev->st->ready) return make_error(MKRT_FAILED_PRECONDITION, "event is not ready");
  if (ev->st->code != MKRT_OK) return new mkrt_error{ev->st->code, ev->st->message};
  return nullptr;
}

mkrt_error* mkrt_event_await(mkrt_event* ev, int64_t timeout_ms) {
  if (!ev) return make_error(MKRT_INVALID_ARGUMENT, "mkrt_event_await: null event");
  return await_state(ev->st, timeout_ms);
}

mkrt_error* mkrt_event_on_ready(mkrt_event* ev, mkrt_event_callback cb, void* user) {
  if (!ev || !cb) return make_error(MKRT_INVALID_ARGUMENT, "mkrt_event_on_ready: null argument");
  int code;
  std::string msg;
  {
    std::lock_guard<std::mutex> g(ev->st->mu);
    if (!ev->st->ready) {
      ev->st->callbacks.emplace_back(cb, user);
      return nullptr;
    }
    code = ev->st->code;
    msg = ev->st->message;
  }
  cb(code == MKRT_OK ? nullptr : new mkrt_error{code, msg}, user);
  return nullptr;
}

void mkrt_event_destroy(mkrt_event* ev) { delete ev; }

}  // extern "C"
