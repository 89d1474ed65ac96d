// Fused elementwise emitter: turns an mk_ew_instr program into straight-line
// HIP source, compiles it for gfx950 with hiprtc on first use and caches the
// loaded kernel per (device, dtype, program).
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
std::unordered_map<std::string, JitKernel> g_cache;

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
  // Element loader: vector or scalar path, or a 1-element broadcast.
  if (bf) {
    s += "__device__ __forceinline__ void ld(const void* p, long long numel, long long idx, bool vec, long long n, float* o) {\n"
         "  const u16* q = (const u16*)p;\n"
         "  if (numel == 1) { float v = bf2f(q[0]); for (int e = 0; e < 8; ++e) o[e] = v; return; }\n"
         "  if (vec) { u4 w = *(const u4*)(q + idx);\n"
         "    o[0] = bf2f(w.x & 0xffffu); o[1] = bf2f(w.x >> 16); o[2] = bf2f(w.y & 0xffffu); o[3] = bf2f(w.y >> 16);\n"
         "    o[4] = bf2f(w.z & 0xffffu); o[5] = bf2f(w.z >> 16); o[6] = bf2f(w.w & 0xffffu); o[7] = bf2f(w.w >> 16); return; }\n"
         "  for (int e = 0; e < 8; ++e) o[e] = (idx + e < n) ? bf2f(q[idx + e]) : 0.f;\n"
         "}\n"
         "__device__ __forceinline__ void st(void* p, long long idx, bool vec, long long n, const float* v) {\n"
         "  u16* q = (u16*)p;\n"
         "  if (vec) { u4 w; w.x = P2(v[0], v[1]); w.y = P2(v[2], v[3]); w.z = P2(v[4], v[5]); w.w = P2(v[6], v[7]);\n"
         "    *(u4*)(q + idx) = w; return; }\n"
         "  for (int e = 0; e < 8; ++e) if (idx + e < n) q[idx + e] = (u16)P2(v[e], 0.f);\n"
         "}\n";
  } else {
    s += "__device__ __forceinline__ void ld(const void* p, long long numel, long long idx, bool vec, long long n, float* o) {\n"
         "  const float* q = (const float*)p;\n"
         "  if (numel == 1) { float v = q[0]; for (int e = 0; e < 8; ++e) o[e] = v; return; }\n"
         "  if (vec) { f4 a = *(const f4*)(q + idx); f4 b = *(const f4*)(q + idx + 4);\n"
         "    o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w; o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w; return; }\n"
         "  for (int e = 0; e < 8; ++e) o[e] = (idx + e < n) ? q[idx + e] : 0.f;\n"
         "}\n"
         "__device__ __forceinline__ void st(void* p, long long idx, bool vec, long long n, const float* v) {\n"
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
  for (int i = 0; i < n_instr; ++i)
    if (prog[i].op == MK_EW_LOAD) used[prog[i].a] = true;
  for (int k = 0; k < n_inputs; ++k) {
    if (!used[k]) continue;
    char b[128];
    snprintf(b, sizeof(b), "    float X%d[8]; ld(i%d, n%d, idx, vec, n, X%d);\n", k, k, k, k);
    s += b;
  }
  // bf16 programs evaluate two elements per iteration so that each op's
  // rounding is one packed conversion for both (R2); f32 programs go one by one.
  const int lanes = bf ? 2 : 1;
  s += bf ? "    float res[8];\n#pragma unroll\n    for (int e = 0; e < 8; e += 2) {\n"
          : "    float res[8];\n#pragma unroll\n    for (int e = 0; e < 8; ++e) {\n";
  std::string slot[16];
  for (int i = 0; i < n_instr; ++i) {
    const mk_ew_instr& in = prog[i];
    const std::string v = "v" + std::to_string(i);
    bool rnd = bf;
    std::string decl;
    for (int l = 0; l < lanes; ++l) {
      const std::string sfx = bf ? "_" + std::to_string(l) : std::string();
      // Operand fields an op does not use may hold anything (-1 included).
      auto src = [&](int k) { return k >= 0 && k < 16 && !slot[k].empty() ? slot[k] + sfx : std::string(); };
      const std::string A = src(in.a), B = src(in.b), C = src(in.c);
      std::string ex;
      switch (in.op) {
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
        case MK_EW_EXP: ex = (bf ? "mk_exp_bf(" : "mk_exp(") + A + ")"; break;
        case MK_EW_LOG: ex = (bf ? "__logf(" : "logf(") + A + ")"; break;
        case MK_EW_LOG1P: ex = "mk_log1p(" + A + ")"; break;
        case MK_EW_EXPM1: ex = "expm1f(" + A + ")"; break;
        case MK_EW_TANH: ex = "tanhf(" + A + ")"; break;
        case MK_EW_RSQRT: ex = "1.0f / sqrtf(" + A + ")"; break;
        case MK_EW_SQRT: ex = "sqrtf(" + A + ")"; break;
        case MK_EW_LOGISTIC: ex = (bf ? "mk_logistic_bf(" : "mk_logistic(") + A + ")"; break;
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
    if (rnd) s += "      R2(" + v + "_0, " + v + "_1);\n";
    slot[in.dst] = v;
  }
  s += bf ? "      res[e] = " + slot[out_slot] + "_0; res[e + 1] = " + slot[out_slot] + "_1;\n"
          : "      res[e] = " + slot[out_slot] + ";\n";
  s += "    }\n    st(out, idx, vec, n, res);\n  }\n}\n";
  return s;
}

hipError_t compile_and_load(const std::string& src, JitKernel* k, std::string* err) {
  hiprtcProgram p;
  if (hiprtcCreateProgram(&p, src.c_str(), "mk_ew_jit.hip", 0, nullptr, nullptr) != HIPRTC_SUCCESS) {
    *err = "hiprtcCreateProgram failed";
    return hipErrorUnknown;
  }
  // No FMA contraction: every StableHLO op rounds its own result, exactly as
  // the interpreter kernel and the op-by-op oracle evaluate it.
  const char* opts[] = {"--offload-arch=gfx950", "-O3", "-ffp-contract=off", "-Xclang", "-target-feature",
                        "-Xclang", "-packed-fp32-ops"};
  const hiprtcResult r = hiprtcCompileProgram(p, 7, opts);
  if (r != HIPRTC_SUCCESS) {
    size_t ls = 0;
    hiprtcGetProgramLogSize(p, &ls);
    std::string log(ls, '\0');
    if (ls) hiprtcGetProgramLog(p, &log[0]);
    *err = "hiprtc compile failed: " + log;
    hiprtcDestroyProgram(&p);
    return hipErrorUnknown;
  }
  size_t cs = 0;
  hiprtcGetCodeSize(p, &cs);
  std::vector<char> code(cs);
  hiprtcGetCode(p, code.data());
  hiprtcDestroyProgram(&p);
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
    JitKernel k;
    std::string err;
    e = compile_and_load(generate(dtype, prog, n_instr, n_inputs, out_slot), &k, &err);
    if (e != hipSuccess) return fail(MK_ELAUNCH, "mk_elementwise: %s", err.c_str());
    it = g_cache.emplace(key, k).first;
  }
  *fn_out = (void*)it->second.fn;
  return MK_OK;
}

}  // namespace mkc
