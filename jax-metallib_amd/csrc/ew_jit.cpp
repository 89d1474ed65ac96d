// Fused elementwise emitter: turns an mk_ew_instr program into straight-line
// HIP source, compiles it for gfx950 with hiprtc on first use and caches the
// loaded kernel per (device, dtype, program).
//
// Compiled code objects are cached at two more levels, keyed by the exact
// source text, the compile options and the hiprtc version:
//   * in memory for the process (shared by every device), and seedable from
//     a serialized executable (mkrt_deserialize), so a deserialized program
//     launches without compiling;
//   * on disk, one file per code object under MK_CACHE_DIR (default
//     $HOME/.cache/mi355x-mk), written atomically (temporary file + rename)
//     and verified against the full key on read.  MK_DISABLE_CACHE_PERSIST=1
//     turns the disk level off.  This is the counterpart of the reference's
//     persisted autotune cache (core/mps_executable.mm:3270-3420,
//     JAX_METALLIB_AUTOTUNE_CACHE_DIR / _DISABLE_AUTOTUNE_CACHE_PERSIST):
//     here the first-call cost is the hiprtc compile, not autotuning.
//
// This is the MI355X counterpart of the reference's generated fusion kernels
// (GenerateFusedKernelSource, core/mps_executable.mm:4445-4586, with a
// pipeline cache keyed by the chain, :4588-4629).  The generated kernel
// keeps every intermediate in registers, reads each live input once and
// writes the output once, with 8 elements per thread per iteration (16- or
// 32-byte vector accesses when aligned).  Rounding points are the same as
// the precompiled interpreter kernel (eltwise.hip): bf16 programs round every
// float op result to bf16 (round-to-nearest-even), compare/select results
// are exact; no a*b+c is contracted into an FMA.  It is compiled with the
// packed-FP32 target feature disabled, like every other kernel here.
#include <hip/hip_runtime.h>
#include <hip/hiprtc.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <stdlib.h>
#include <sys/stat.h>
#include <unistd.h>

#include <atomic>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/mk_kernels.h"
#include "capi_internal.h"
#include "ew_jit.h"
#include "kernels/ew_math.h"

namespace mkc {
namespace {

struct JitKernel {
  hipModule_t mod = nullptr;
  hipFunction_t fn = nullptr;
};

std::mutex g_mu;
std::unordered_map<std::string, JitKernel> g_cache;                 // loaded kernels per device
std::unordered_map<std::string, std::vector<char>> g_code;          // code objects by source
std::atomic<int64_t> g_compiles{0}, g_disk_hits{0}, g_mem_hits{0};

// No FMA contraction: every StableHLO op rounds its own result, exactly as
// the interpreter kernel and the op-by-op oracle evaluate it.
const char* const kOpts[] = {"--offload-arch=gfx950", "-O3", "-ffp-contract=off", "-Xclang", "-target-feature",
                             "-Xclang", "-packed-fp32-ops"};
constexpr int kNumOpts = 7;

// Everything the code object depends on besides the source.
const std::string& compile_tag() {
  static const std::string tag = [] {
    int maj = 0, mn = 0;
    hiprtcVersion(&maj, &mn);
    std::string t = "hiprtc " + std::to_string(maj) + "." + std::to_string(mn) + "|";
    for (int i = 0; i < kNumOpts; ++i) (t += kOpts[i]) += ' ';
    return t;
  }();
  return tag;
}

uint64_t fnv1a64(const std::string& a, const std::string& b) {
  uint64_t h = 1469598103934665603ull;
  for (const std::string* s : {&a, &b})
    for (unsigned char c : *s) h = (h ^ c) * 1099511628211ull;
  return h;
}

// Disk cache directory ("" when disabled or unusable).
std::string cache_dir() {
  const char* off = getenv("MK_DISABLE_CACHE_PERSIST");
  if (off && off[0] && strcmp(off, "0") != 0) return "";
  std::string dir;
  const char* env = getenv("MK_CACHE_DIR");
  if (env && env[0]) {
    dir = env;
  } else {
    const char* home = getenv("HOME");
    if (!home || !home[0]) return "";
    dir = std::string(home) + "/.cache";
    mkdir(dir.c_str(), 0755);
    dir += "/mi355x-mk";
  }
  mkdir(dir.c_str(), 0755);
  struct stat st;
  if (stat(dir.c_str(), &st) != 0 || !S_ISDIR(st.st_mode)) return "";
  return dir;
}

// File layout: "MKCO", u32 version 1, u64 key bytes, key (tag + source),
// u64 code bytes, code.
constexpr uint32_t kCodeFileVersion = 1;

std::string cache_path(const std::string& dir, const std::string& src) {
  char name[64];
  snprintf(name, sizeof(name), "/ew-%016llx.hsaco", (unsigned long long)fnv1a64(compile_tag(), src));
  return dir + name;
}

bool read_cached(const std::string& path, const std::string& src, std::vector<char>* code) {
  FILE* f = fopen(path.c_str(), "rb");
  if (!f) return false;
  bool ok = false;
  char magic[4];
  uint32_t ver = 0;
  uint64_t klen = 0, clen = 0;
  const std::string key = compile_tag() + src;
  if (fread(magic, 1, 4, f) == 4 && memcmp(magic, "MKCO", 4) == 0 && fread(&ver, 4, 1, f) == 1 &&
      ver == kCodeFileVersion && fread(&klen, 8, 1, f) == 1 && klen == key.size()) {
    std::string k(klen, '\0');
    if (fread(&k[0], 1, klen, f) == klen && k == key && fread(&clen, 8, 1, f) == 1 && clen > 0 &&
        clen < (1ull << 30)) {
      code->resize(clen);
      ok = fread(code->data(), 1, clen, f) == clen;
    }
  }
  fclose(f);
  return ok;
}

void write_cached(const std::string& path, const std::string& src, const std::vector<char>& code) {
  const std::string key = compile_tag() + src;
  const std::string tmp = path + ".tmp." + std::to_string((long long)getpid());
  FILE* f = fopen(tmp.c_str(), "wb");
  if (!f) return;
  const uint64_t klen = key.size(), clen = code.size();
  bool ok = fwrite("MKCO", 1, 4, f) == 4 && fwrite(&kCodeFileVersion, 4, 1, f) == 1 && fwrite(&klen, 8, 1, f) == 1 &&
            fwrite(key.data(), 1, klen, f) == klen && fwrite(&clen, 8, 1, f) == 1 &&
            fwrite(code.data(), 1, clen, f) == clen;
  ok = (fclose(f) == 0) && ok;
  if (!ok || rename(tmp.c_str(), path.c_str()) != 0) unlink(tmp.c_str());
}

std::string key_of(int device, int dtype, const mk_ew_instr* prog, int n_instr, int n_inputs, int out_slot) {
  std::string k;
  k.reserve(64 + n_instr * sizeof(mk_ew_instr));
  char head[64];
  snprintf(head, sizeof(head), "d%d|t%d|i%d|o%d|", device, dtype, n_inputs, out_slot);
  k += head;
  k.append(reinterpret_cast<const char*>(prog), n_instr * sizeof(mk_ew_instr));
  return k;
}

std::string fmt_const(float v) {
  uint32_t u;
  memcpy(&u, &v, 4);
  char b[48];
  snprintf(b, sizeof(b), "__uint_as_float(0x%08xu)", u);
  return b;
}

// Source of one program.  Inputs are read as X0..X3[e] (already widened to
// f32); the result of instruction i is v<i>; slots map to the latest value.
std::string generate(int dtype, const mk_ew_instr* prog, int n_instr, int n_inputs, int out_slot) {
  const bool bf = dtype == MK_DT_BF16;
  std::string s;
  s += "typedef unsigned short u16;\n"
       "typedef unsigned int u32;\n"
       "typedef float f4 __attribute__((ext_vector_type(4)));\n"
       "typedef u32 u4 __attribute__((ext_vector_type(4)));\n"
       "__device__ __forceinline__ float bf2f(u32 b) { return __uint_as_float(b << 16); }\n"
       "__device__ __forceinline__ float R(float f) { return (float)(__bf16)f; }\n"
       "typedef float f2 __attribute__((ext_vector_type(2)));\n"
       "typedef __bf16 b2 __attribute__((ext_vector_type(2)));\n"
       "__device__ __forceinline__ u32 P2(float a, float b) {\n"
       "  return __builtin_bit_cast(u32, __builtin_convertvector((f2){a, b}, b2)); }\n"
       "__device__ __forceinline__ void R2(float& a, float& b) {\n"
       "  const u32 w = P2(a, b); a = __uint_as_float(w << 16); b = __uint_as_float(w & 0xffff0000u); }\n"
       MK_EW_MATH_SRC "\n";
  // Element loaders (bf16 and f32 inputs): vector or scalar path, a
  // 1-element broadcast, or a periodic input (element i from i mod numel).
  s += "__device__ __forceinline__ void ldh(const void* p, long long numel, long long idx, bool vec, long long n, float* o) {\n"
       "  const u16* q = (const u16*)p;\n"
       "  if (numel == 1) { float v = bf2f(q[0]); for (int e = 0; e < 8; ++e) o[e] = v; return; }\n"
       "  if (numel != n) { idx %= numel; if (!vec) { for (int e = 0; e < 8; ++e) { long long j = idx + e;\n"
       "      while (j >= numel) j -= numel; o[e] = bf2f(q[j]); } return; } }\n"
       "  if (vec) { u4 w = *(const u4*)(q + idx);\n"
       "    o[0] = bf2f(w.x & 0xffffu); o[1] = bf2f(w.x >> 16); o[2] = bf2f(w.y & 0xffffu); o[3] = bf2f(w.y >> 16);\n"
       "    o[4] = bf2f(w.z & 0xffffu); o[5] = bf2f(w.z >> 16); o[6] = bf2f(w.w & 0xffffu); o[7] = bf2f(w.w >> 16); return; }\n"
       "  for (int e = 0; e < 8; ++e) o[e] = (idx + e < n) ? bf2f(q[idx + e]) : 0.f;\n"
       "}\n"
       "__device__ __forceinline__ void ldf(const void* p, long long numel, long long idx, bool vec, long long n, float* o) {\n"
       "  const float* q = (const float*)p;\n"
       "  if (numel == 1) { float v = q[0]; for (int e = 0; e < 8; ++e) o[e] = v; return; }\n"
       "  if (numel != n) { idx %= numel; if (!vec) { for (int e = 0; e < 8; ++e) { long long j = idx + e;\n"
       "      while (j >= numel) j -= numel; o[e] = q[j]; } return; } }\n"
       "  if (vec) { f4 a = *(const f4*)(q + idx); f4 b = *(const f4*)(q + idx + 4);\n"
       "    o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w; o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w; return; }\n"
       "  for (int e = 0; e < 8; ++e) o[e] = (idx + e < n) ? q[idx + e] : 0.f;\n"
       "}\n";
  if (bf) {
    s += "__device__ __forceinline__ void st(void* p, long long idx, bool vec, long long n, const float* v) {\n"
         "  u16* q = (u16*)p;\n"
         "  if (vec) { u4 w; w.x = P2(v[0], v[1]); w.y = P2(v[2], v[3]); w.z = P2(v[4], v[5]); w.w = P2(v[6], v[7]);\n"
         "    *(u4*)(q + idx) = w; return; }\n"
         "  for (int e = 0; e < 8; ++e) if (idx + e < n) q[idx + e] = (u16)P2(v[e], 0.f);\n"
         "}\n";
  } else {
    s += "__device__ __forceinline__ void st(void* p, long long idx, bool vec, long long n, const float* v) {\n"
         "  float* q = (float*)p;\n"
         "  if (vec) { *(f4*)(q + idx) = f4{v[0], v[1], v[2], v[3]}; *(f4*)(q + idx + 4) = f4{v[4], v[5], v[6], v[7]}; return; }\n"
         "  for (int e = 0; e < 8; ++e) if (idx + e < n) q[idx + e] = v[e];\n"
         "}\n";
  }
  s += "extern \"C\" __global__ void __launch_bounds__(256) mk_ew_jit(const void* i0, const void* i1, const void* i2, "
       "const void* i3, long long n0, long long n1, long long n2, long long n3, void* out, long long n, int vec_ok) {\n"
       "  const long long chunks = (n + 7) / 8;\n"
       "  for (long long c = (long long)blockIdx.x * 256 + threadIdx.x; c < chunks; c += (long long)gridDim.x * 256) {\n"
       "    const long long idx = c * 8;\n"
       "    const bool vec = vec_ok && idx + 8 <= n;\n";
  bool used[4] = {false, false, false, false};
  bool half[4] = {bf, bf, bf, bf};  // input read as bf16 (else f32)
  for (int i = 0; i < n_instr; ++i)
    if (prog[i].op == MK_EW_LOAD) {
      used[prog[i].a] = true;
      if (prog[i].b != 0) half[prog[i].a] = prog[i].b == MK_EW_IN_BF16;
    }
  for (int k = 0; k < n_inputs; ++k) {
    if (!used[k]) continue;
    char b[128];
    snprintf(b, sizeof(b), "    float X%d[8]; %s(i%d, n%d, idx, vec, n, X%d);\n", k, half[k] ? "ldh" : "ldf", k, k, k);
    s += b;
  }
  // bf16 programs evaluate two elements per iteration so that each op's
  // rounding is one packed conversion for both (R2); f32 programs go one by one.
  const int lanes = bf ? 2 : 1;
  s += bf ? "    float res[8];\n#pragma unroll\n    for (int e = 0; e < 8; e += 2) {\n"
          : "    float res[8];\n#pragma unroll\n    for (int e = 0; e < 8; ++e) {\n";
  std::string slot[16];
  // Whether a slot's value is a bf16 value (8 significant bits): bf16 loads,
  // bf16-representable constants, every rounded result, compare results,
  // selects of two such values.  log1p of such a value takes the short form.
  bool exact[16] = {};
  for (int i = 0; i < n_instr; ++i) {
    const mk_ew_instr& in = prog[i];
    const std::string v = "v" + std::to_string(i);
    const int opc = in.op & ~MK_EW_KEEP_F32;
    bool rnd = bf && !(in.op & MK_EW_KEEP_F32);  // rounded bf16 result (short exp / logistic forms)
    const bool fast = rnd;
    std::string decl;
    for (int l = 0; l < lanes; ++l) {
      const std::string sfx = bf ? "_" + std::to_string(l) : std::string();
      // Operand fields an op does not use may hold anything (-1 included).
      auto src = [&](int k) { return k >= 0 && k < 16 && !slot[k].empty() ? slot[k] + sfx : std::string(); };
      const std::string A = src(in.a), B = src(in.b), C = src(in.c);
      std::string ex;
      switch (opc) {
        case MK_EW_LOAD: ex = "X" + std::to_string(in.a) + (l ? "[e + 1]" : "[e]"); rnd = false; break;
        case MK_EW_CONST: ex = fmt_const(in.imm); rnd = false; break;
        case MK_EW_ADD: ex = A + " + " + B; break;
        case MK_EW_SUB: ex = A + " - " + B; break;
        case MK_EW_MUL: ex = A + " * " + B; break;
        case MK_EW_DIV: ex = A + " / " + B; break;
        case MK_EW_MAX: ex = "mk_max(" + A + ", " + B + ")"; break;
        case MK_EW_MIN: ex = "mk_min(" + A + ", " + B + ")"; break;
        case MK_EW_POW: ex = "powf(" + A + ", " + B + ")"; break;
        case MK_EW_NEG: ex = "-" + A; break;
        case MK_EW_ABS: ex = "fabsf(" + A + ")"; break;
        // bf16 programs round every result to 8 significant bits, so the
        // short exp form (relative error < 2^-16) suffices there.
        case MK_EW_EXP: ex = (fast ? "mk_exp_bf(" : "mk_exp(") + A + ")"; break;
        case MK_EW_LOG: ex = (fast ? "__logf(" : "logf(") + A + ")"; break;
        case MK_EW_LOG1P:
          ex = (fast && in.a >= 0 && in.a < 16 && exact[in.a] ? "mk_log1p_bf(" : "mk_log1p(") + A + ")";
          break;
        case MK_EW_EXPM1: ex = "expm1f(" + A + ")"; break;
        case MK_EW_TANH: ex = "tanhf(" + A + ")"; break;
        case MK_EW_RSQRT: ex = "1.0f / sqrtf(" + A + ")"; break;
        case MK_EW_SQRT: ex = "sqrtf(" + A + ")"; break;
        case MK_EW_LOGISTIC: ex = (fast ? "mk_logistic_bf(" : "mk_logistic(") + A + ")"; break;
        case MK_EW_FLOOR: ex = "floorf(" + A + ")"; break;
        case MK_EW_CEIL: ex = "ceilf(" + A + ")"; break;
        case MK_EW_CMP_EQ: ex = "(" + A + " == " + B + ") ? 1.f : 0.f"; rnd = false; break;
        case MK_EW_CMP_NE: ex = "(" + A + " != " + B + ") ? 1.f : 0.f"; rnd = false; break;
        case MK_EW_CMP_LT: ex = "(" + A + " < " + B + ") ? 1.f : 0.f"; rnd = false; break;
        case MK_EW_CMP_LE: ex = "(" + A + " <= " + B + ") ? 1.f : 0.f"; rnd = false; break;
        case MK_EW_CMP_GT: ex = "(" + A + " > " + B + ") ? 1.f : 0.f"; rnd = false; break;
        case MK_EW_CMP_GE: ex = "(" + A + " >= " + B + ") ? 1.f : 0.f"; rnd = false; break;
        case MK_EW_SELECT: ex = "(" + A + " != 0.f) ? " + B + " : " + C; rnd = false; break;
        case MK_EW_ROUND_BF16: ex = "R(" + A + ")"; rnd = false; break;
        default: ex = A; rnd = false; break;
      }
      decl += (l ? ", " : "      float ") + v + sfx + " = (" + ex + ")";
    }
    s += decl + ";\n";
    // max, min, neg, abs, floor and ceil of bf16 values are bf16 values:
    // their rounding would change nothing, so it is not emitted.
    bool kept_exact = false;
    {
      auto ex = [&](int k) { return k >= 0 && k < 16 && exact[k]; };
      if (rnd && (((opc == MK_EW_MAX || opc == MK_EW_MIN) && ex(in.a) && ex(in.b)) ||
                  ((opc == MK_EW_NEG || opc == MK_EW_ABS || opc == MK_EW_FLOOR || opc == MK_EW_CEIL) && ex(in.a)))) {
        rnd = false;
        kept_exact = true;
      }
    }
    if (rnd) s += "      R2(" + v + "_0, " + v + "_1);\n";
    {
      uint32_t ib;
      memcpy(&ib, &in.imm, 4);
      auto ex_of = [&](int k) { return k >= 0 && k < 16 && exact[k]; };
      bool e = rnd || kept_exact;
      if (opc == MK_EW_LOAD) e = bf && half[in.a];
      else if (opc == MK_EW_CONST) e = (ib & 0xFFFFu) == 0u;
      else if (opc >= MK_EW_CMP_EQ && opc <= MK_EW_CMP_GE) e = true;
      else if (opc == MK_EW_SELECT) e = ex_of(in.b) && ex_of(in.c);
      else if (opc == MK_EW_ROUND_BF16) e = true;
      if (in.dst >= 0 && in.dst < 16) exact[in.dst] = e;
    }
    slot[in.dst] = v;
  }
  s += bf ? "      res[e] = " + slot[out_slot] + "_0; res[e + 1] = " + slot[out_slot] + "_1;\n"
          : "      res[e] = " + slot[out_slot] + ";\n";
  s += "    }\n    st(out, idx, vec, n, res);\n  }\n}\n";
  return s;
}

bool hiprtc_compile(const std::string& src, std::vector<char>* code, std::string* err) {
  hiprtcProgram p;
  if (hiprtcCreateProgram(&p, src.c_str(), "mk_ew_jit.hip", 0, nullptr, nullptr) != HIPRTC_SUCCESS) {
    *err = "hiprtcCreateProgram failed";
    return false;
  }
  const hiprtcResult r = hiprtcCompileProgram(p, kNumOpts, kOpts);
  if (r != HIPRTC_SUCCESS) {
    size_t ls = 0;
    hiprtcGetProgramLogSize(p, &ls);
    std::string log(ls, '\0');
    if (ls) hiprtcGetProgramLog(p, &log[0]);
    *err = "hiprtc compile failed: " + log;
    hiprtcDestroyProgram(&p);
    return false;
  }
  size_t cs = 0;
  hiprtcGetCodeSize(p, &cs);
  code->resize(cs);
  hiprtcGetCode(p, code->data());
  hiprtcDestroyProgram(&p);
  g_compiles.fetch_add(1);
  return true;
}

// Code object of a source: memory, then disk, then hiprtc (only hiprtc when
// `fresh`, which replaces whatever the caches held).  g_mu held.
const std::vector<char>* code_for(const std::string& src, std::string* err, bool fresh = false) {
  auto it = g_code.find(src);
  if (it != g_code.end() && !fresh) {
    g_mem_hits.fetch_add(1);
    return &it->second;
  }
  std::vector<char> code;
  const std::string dir = cache_dir();
  const std::string path = dir.empty() ? "" : cache_path(dir, src);
  if (!fresh && !path.empty() && read_cached(path, src, &code)) {
    g_disk_hits.fetch_add(1);
  } else {
    if (!hiprtc_compile(src, &code, err)) return nullptr;
    if (!path.empty()) write_cached(path, src, code);
  }
  std::vector<char>& slot = g_code[src];
  slot = std::move(code);
  return &slot;
}

hipError_t load_module(const std::vector<char>& code, JitKernel* k, std::string* err) {
  hipError_t e = hipModuleLoadData(&k->mod, code.data());
  if (e != hipSuccess) {
    *err = std::string("hipModuleLoadData: ") + hipGetErrorString(e);
    return e;
  }
  e = hipModuleGetFunction(&k->fn, k->mod, "mk_ew_jit");
  if (e != hipSuccess) *err = std::string("hipModuleGetFunction: ") + hipGetErrorString(e);
  return e;
}

}  // namespace

std::string cache_directory() { return cache_dir(); }

std::string ew_jit_source(int dtype, const mk_ew_instr* prog, int n_instr, int n_inputs, int out_slot) {
  return generate(dtype, prog, n_instr, n_inputs, out_slot);
}

int ew_jit_get(int dtype, const mk_ew_instr* prog, int n_instr, int n_inputs, int out_slot, void** fn_out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(MK_ELAUNCH, "mk_elementwise: no device: %s", hipGetErrorString(e));
  const std::string key = key_of(dev, dtype, prog, n_instr, n_inputs, out_slot);
  std::lock_guard<std::mutex> lock(g_mu);
  auto it = g_cache.find(key);
  if (it == g_cache.end()) {
    std::string err;
    const std::string src = generate(dtype, prog, n_instr, n_inputs, out_slot);
    const std::vector<char>* code = code_for(src, &err);
    if (!code) return fail(MK_ELAUNCH, "mk_elementwise: %s", err.c_str());
    JitKernel k;
    e = load_module(*code, &k, &err);
    if (e != hipSuccess) {
      // A cached or seeded object the runtime rejects: compile it afresh.
      code = code_for(src, &err, true);
      if (!code) return fail(MK_ELAUNCH, "mk_elementwise: %s", err.c_str());
      e = load_module(*code, &k, &err);
    }
    if (e != hipSuccess) return fail(MK_ELAUNCH, "mk_elementwise: %s", err.c_str());
    it = g_cache.emplace(key, k).first;
  }
  *fn_out = (void*)it->second.fn;
  return MK_OK;
}

int ew_jit_code(int dtype, const mk_ew_instr* prog, int n_instr, int n_inputs, int out_slot, std::string* source,
                std::vector<char>* code) {
  *source = generate(dtype, prog, n_instr, n_inputs, out_slot);
  std::lock_guard<std::mutex> lock(g_mu);
  std::string err;
  const std::vector<char>* c = code_for(*source, &err);
  if (!c) return fail(MK_ELAUNCH, "mk_elementwise: %s", err.c_str());
  *code = *c;
  return MK_OK;
}

const std::string& ew_jit_tag() { return compile_tag(); }

void ew_jit_seed(const std::string& source, const std::vector<char>& code) {
  std::lock_guard<std::mutex> lock(g_mu);
  g_code.emplace(source, code);
}

void ew_jit_stats(int64_t* compiles, int64_t* disk_hits, int64_t* mem_hits) {
  *compiles = g_compiles.load();
  *disk_hits = g_disk_hits.load();
  *mem_hits = g_mem_hits.load();
}

}  // namespace mkc
