// Fused elementwise chains for gfx950: one pass over memory for a whole DAG
// of elementwise ops (the workload's 6-op chain mul/add/exp/log1p/max/select
// and the like).
//
// The reference runs such chains as MPSGraph segments on flat tensors
// (core/mps_executable.mm:7393-7508) or, opt-in, as generated MSL built from
// per-op snippets (FusionSnippet :4303-4351, GenerateFusedKernelSource
// :4445-4586; f32/f16 only, no log1p/select/compare).  Here the executor
// lowers the chain to a short register program (include/mk_kernels.h,
// mk_ew_instr) that one precompiled kernel evaluates: the program lives in the
// kernel arguments, so its control flow is wave-uniform (scalar branches),
// and each thread applies every instruction to 8 elements held in registers.
// HBM traffic is one read of each live input and one write of the output.
//
// Semantics: f32 programs compute in f32.  bf16 programs round every float
// result to bf16, as XLA:CPU does for bf16 ops (reference
// ops/registry.h:273-287).  maximum/minimum propagate NaN and order -0 < +0.
// Comparisons yield 1.0 / 0.0 (never rounded); select picks b where a != 0.
#include "common.h"
#include "ew_math.h"

#include <math.h>

namespace mk {

constexpr int kEwSlots = 12;
constexpr int kEwVec = 8;
constexpr int kEwMaxInstr = 32;
constexpr int kEwMaxInputs = 4;

struct EwArgs {
  mk_ew_instr ins[kEwMaxInstr];
  const void* in[kEwMaxInputs];
  int64_t in_numel[kEwMaxInputs];  // n (elementwise) or 1 (scalar broadcast)
  void* out;
  int64_t n;
  int n_instr;
  int out_slot;
};

__device__ __forceinline__ float ew_bf16r(float v) { return bf16_to_f32(f32_to_bf16(v)); }

MK_EW_MATH_DEFS

typedef float f32x8 __attribute__((ext_vector_type(8)));

// The slot file: 12 separate 8-wide vector values s0..s11 (locals of the
// kernel, never an aggregate in memory).  Slot access is a switch on a
// wave-uniform index in which every case names its own variable, so each
// slot is an SSA value in VGPRs and the switch costs scalar branches only.
#define MK_EW_SLOT_CASES(X) X(0) X(1) X(2) X(3) X(4) X(5) X(6) X(7) X(8) X(9) X(10) X(11)
#define MK_EW_GET_CASE(k) \
  case k:                 \
    v_ = s##k;            \
    break;
#define MK_EW_PUT_CASE(k) \
  case k:                 \
    s##k = v_;            \
    break;
#define MK_EW_GET(idx, out)                    \
  do {                                         \
    f32x8 v_ = s0;                             \
    switch (idx) { MK_EW_SLOT_CASES(MK_EW_GET_CASE) default: break; } \
    out = v_;                                  \
  } while (0)
#define MK_EW_PUT(idx, val)                    \
  do {                                         \
    const f32x8 v_ = (val);                    \
    switch (idx) { MK_EW_SLOT_CASES(MK_EW_PUT_CASE) default: break; } \
  } while (0)

template <bool BF16>
__device__ __forceinline__ void ew_load(const void* p, int64_t numel, int64_t idx, bool vec, int64_t n,
                                        f32x8& o) {
  if (numel == 1) {
    const float v = BF16 ? bf16_to_f32(*static_cast<const uint16_t*>(p)) : *static_cast<const float*>(p);
#pragma unroll
    for (int e = 0; e < kEwVec; ++e) o[e] = v;
    return;
  }
  if (numel != n) {
    // Periodic input (a broadcast over leading dimensions): element i is
    // input element i mod numel.
#pragma unroll
    for (int e = 0; e < kEwVec; ++e) {
      const int64_t i = idx + e;
      const int64_t j = i % numel;
      o[e] = i < n ? (BF16 ? bf16_to_f32(static_cast<const uint16_t*>(p)[j]) : static_cast<const float*>(p)[j]) : 0.f;
    }
    return;
  }
  if (vec) {
    if (BF16) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(p) + idx);
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        o[2 * i] = bf16_to_f32(w[i] & 0xFFFFu);
        o[2 * i + 1] = bf16_to_f32(w[i] >> 16);
      }
    } else {
      const f32x4 a = *reinterpret_cast<const f32x4*>(static_cast<const float*>(p) + idx);
      const f32x4 b = *reinterpret_cast<const f32x4*>(static_cast<const float*>(p) + idx + 4);
      o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
      o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
    }
    return;
  }
#pragma unroll
  for (int e = 0; e < kEwVec; ++e) {
    const int64_t i = idx + e;
    o[e] = i < n ? (BF16 ? bf16_to_f32(static_cast<const uint16_t*>(p)[i]) : static_cast<const float*>(p)[i])
                 : 0.f;
  }
}

template <bool BF16>
__device__ __forceinline__ void ew_store(void* p, int64_t idx, bool vec, int64_t n, const f32x8& v) {
  if (vec) {
    if (BF16) {
      *reinterpret_cast<u32x4*>(static_cast<uint16_t*>(p) + idx) =
          u32x4{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
                pack_bf16x2(v[6], v[7])};
    } else {
      *reinterpret_cast<f32x4*>(static_cast<float*>(p) + idx) = f32x4{v[0], v[1], v[2], v[3]};
      *reinterpret_cast<f32x4*>(static_cast<float*>(p) + idx + 4) = f32x4{v[4], v[5], v[6], v[7]};
    }
    return;
  }
#pragma unroll
  for (int e = 0; e < kEwVec; ++e) {
    const int64_t i = idx + e;
    if (i < n) {
      if (BF16) static_cast<uint16_t*>(p)[i] = (uint16_t)f32_to_bf16(v[e]);
      else static_cast<float*>(p)[i] = v[e];
    }
  }
}

template <bool BF16, bool VEC>
__global__ __launch_bounds__(256) void eltwise_kernel(EwArgs a) {
  const int64_t chunks = (a.n + kEwVec - 1) / kEwVec;
  for (int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x; c < chunks; c += (int64_t)gridDim.x * 256) {
    const int64_t idx = c * kEwVec;
    const bool vec = VEC && idx + kEwVec <= a.n;
    f32x8 s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f, s4 = 0.f, s5 = 0.f;
    f32x8 s6 = 0.f, s7 = 0.f, s8 = 0.f, s9 = 0.f, s10 = 0.f, s11 = 0.f;
    for (int i = 0; i < a.n_instr; ++i) {
      const mk_ew_instr in = a.ins[i];
      f32x8 x, y = 0.f, z = 0.f, r;
      if (in.op == MK_EW_LOAD) {
        const bool half = in.b == MK_EW_IN_BF16 || (in.b == MK_EW_IN_DEFAULT && BF16);
        if (half) ew_load<true>(a.in[in.a], a.in_numel[in.a], idx, vec, a.n, r);
        else ew_load<false>(a.in[in.a], a.in_numel[in.a], idx, vec, a.n, r);
        MK_EW_PUT(in.dst, r);
        continue;
      }
      if (in.op == MK_EW_CONST) {
        r = in.imm;
        MK_EW_PUT(in.dst, r);
        continue;
      }
      const int opc = in.op & ~MK_EW_KEEP_F32;
      MK_EW_GET(in.a, x);
      if ((opc >= MK_EW_ADD && opc <= MK_EW_POW) || (opc >= MK_EW_CMP_EQ && opc <= MK_EW_SELECT))
        MK_EW_GET(in.b, y);
      if (opc == MK_EW_SELECT) MK_EW_GET(in.c, z);
      // bf16 results use the short exp / logistic forms and are rounded.
      bool round = BF16 && !(in.op & MK_EW_KEEP_F32);
      // One unrolled 8-element loop per case (the switch is wave-uniform).
#define MK_EW_CASE(OPC, EXPR)                            \
  case OPC:                                              \
    _Pragma("unroll") for (int e = 0; e < kEwVec; ++e) { \
      const float u = x[e], v = y[e];                    \
      (void)u;                                           \
      (void)v;                                           \
      r[e] = (EXPR);                                     \
    }                                                    \
    break;
      switch (opc) {
        MK_EW_CASE(MK_EW_ADD, u + v)
        MK_EW_CASE(MK_EW_SUB, u - v)
        MK_EW_CASE(MK_EW_MUL, u * v)
        MK_EW_CASE(MK_EW_DIV, u / v)
        MK_EW_CASE(MK_EW_MAX, mk_max(u, v))
        MK_EW_CASE(MK_EW_MIN, mk_min(u, v))
        MK_EW_CASE(MK_EW_POW, powf(u, v))
        MK_EW_CASE(MK_EW_NEG, -u)
        MK_EW_CASE(MK_EW_ABS, fabsf(u))
        MK_EW_CASE(MK_EW_EXP, round ? mk_exp_bf(u) : mk_exp(u))
        MK_EW_CASE(MK_EW_LOG, logf(u))
        // A bf16-valued operand (low 16 bits clear) takes the short form.
        MK_EW_CASE(MK_EW_LOG1P, round && (__float_as_uint(u) & 0xFFFFu) == 0u ? mk_log1p_bf(u) : mk_log1p(u))
        MK_EW_CASE(MK_EW_EXPM1, expm1f(u))
        MK_EW_CASE(MK_EW_TANH, tanhf(u))
        MK_EW_CASE(MK_EW_RSQRT, 1.0f / sqrtf(u))
        MK_EW_CASE(MK_EW_SQRT, sqrtf(u))
        MK_EW_CASE(MK_EW_LOGISTIC, round ? mk_logistic_bf(u) : mk_logistic(u))
        MK_EW_CASE(MK_EW_FLOOR, floorf(u))
        MK_EW_CASE(MK_EW_CEIL, ceilf(u))
        MK_EW_CASE(MK_EW_CMP_EQ, u == v ? 1.f : 0.f)
        MK_EW_CASE(MK_EW_CMP_NE, u != v ? 1.f : 0.f)
        MK_EW_CASE(MK_EW_CMP_LT, u < v ? 1.f : 0.f)
        MK_EW_CASE(MK_EW_CMP_LE, u <= v ? 1.f : 0.f)
        MK_EW_CASE(MK_EW_CMP_GT, u > v ? 1.f : 0.f)
        MK_EW_CASE(MK_EW_CMP_GE, u >= v ? 1.f : 0.f)
        MK_EW_CASE(MK_EW_SELECT, u != 0.f ? v : z[e])
        MK_EW_CASE(MK_EW_ROUND_BF16, ew_bf16r(u))
        default:
          r = x;
          break;
      }
#undef MK_EW_CASE
      // Predicates and selects of already-rounded values need no rounding.
      if (opc >= MK_EW_CMP_EQ && opc <= MK_EW_SELECT) round = false;
      if (round) {
#pragma unroll
        for (int e = 0; e < kEwVec; ++e) r[e] = ew_bf16r(r[e]);
      }
      MK_EW_PUT(in.dst, r);
    }
    f32x8 o;
    MK_EW_GET(a.out_slot, o);
    ew_store<BF16>(a.out, idx, vec, a.n, o);
  }
}

}  // namespace mk

// ---------------------------------------------------------------------------
// Host launcher
// ---------------------------------------------------------------------------
#include "../capi_internal.h"
#include "../ew_jit.h"

namespace {

// Host-side validation shared by mk_elementwise and mk_elementwise_prepare:
// slots in range, loads of real inputs, sources written before use.
int validate_program(const char* fn, const mk_ew_instr* prog, int n_instr, int n_inputs, int out_slot) {
  if (!prog) return mkc::fail(MK_EINVAL, "%s: null program", fn);
  if (n_instr <= 0 || n_instr > mk::kEwMaxInstr)
    return mkc::fail(MK_EINVAL, "%s: program length %d outside 1..%d", fn, n_instr, mk::kEwMaxInstr);
  if (n_inputs < 0 || n_inputs > mk::kEwMaxInputs)
    return mkc::fail(MK_EINVAL, "%s: %d inputs (max %d)", fn, n_inputs, mk::kEwMaxInputs);
  if (out_slot < 0 || out_slot >= mk::kEwSlots) return mkc::fail(MK_EINVAL, "%s: bad output slot", fn);
  bool defined[mk::kEwSlots] = {false};
  for (int i = 0; i < n_instr; ++i) {
    const mk_ew_instr& in = prog[i];
    const int opc = in.op & ~MK_EW_KEEP_F32;
    if (in.op < 0 || opc >= MK_EW_NUM_OPS) return mkc::fail(MK_EINVAL, "%s: instr %d: bad op %d", fn, i, in.op);
    // The flag marks float arithmetic only (loads, constants, predicates,
    // selects and explicit roundings are never rounded anyway).
    if ((in.op & MK_EW_KEEP_F32) && (opc < MK_EW_ADD || opc > MK_EW_CEIL))
      return mkc::fail(MK_EINVAL, "%s: instr %d: MK_EW_KEEP_F32 on op %d", fn, i, opc);
    if (in.dst < 0 || in.dst >= mk::kEwSlots) return mkc::fail(MK_EINVAL, "%s: instr %d: bad dst", fn, i);
    int nsrc = 0;
    if (opc == MK_EW_LOAD) {
      if (in.a < 0 || in.a >= n_inputs) return mkc::fail(MK_EINVAL, "%s: instr %d: bad input %d", fn, i, in.a);
      if (in.b != MK_EW_IN_DEFAULT && in.b != MK_EW_IN_F32 && in.b != MK_EW_IN_BF16)
        return mkc::fail(MK_EINVAL, "%s: instr %d: bad input type %d", fn, i, in.b);
      for (int k = 0; k < i; ++k)
        if (prog[k].op == MK_EW_LOAD && prog[k].a == in.a && prog[k].b != in.b)
          return mkc::fail(MK_EINVAL, "%s: input %d loaded with two element types", fn, in.a);
    } else if (opc != MK_EW_CONST) {
      nsrc = (opc == MK_EW_SELECT) ? 3 : ((opc >= MK_EW_ADD && opc <= MK_EW_POW) ||
                                          (opc >= MK_EW_CMP_EQ && opc <= MK_EW_CMP_GE)) ? 2 : 1;
    }
    const int src[3] = {in.a, in.b, in.c};
    for (int k = 0; k < nsrc; ++k)
      if (src[k] < 0 || src[k] >= mk::kEwSlots || !defined[src[k]])
        return mkc::fail(MK_EINVAL, "%s: instr %d reads undefined slot %d", fn, i, src[k]);
    defined[in.dst] = true;
  }
  if (!defined[out_slot]) return mkc::fail(MK_EINVAL, "%s: output slot %d never written", fn, out_slot);
  return MK_OK;
}

bool jit_enabled() {
  const char* v = getenv("MK_EW_JIT");
  return !(v && v[0] == '0');
}

}  // namespace

extern "C" int mk_elementwise_prepare(int dtype, const mk_ew_instr* prog, int n_instr, int n_inputs,
                                      int out_slot) {
  mkc::clear_error();
  const char* fn = "mk_elementwise_prepare";
  if (dtype != MK_DT_F32 && dtype != MK_DT_BF16) return mkc::fail(MK_EUNSUPPORTED, "%s: dtype %d", fn, dtype);
  int rc = validate_program(fn, prog, n_instr, n_inputs, out_slot);
  if (rc != MK_OK || !jit_enabled()) return rc;
  void* k = nullptr;
  return mkc::ew_jit_get(dtype, prog, n_instr, n_inputs, out_slot, &k);
}

extern "C" int mk_elementwise(int dtype, const mk_ew_instr* prog, int n_instr, const void* const* inputs,
                              const int64_t* input_numel, int n_inputs, int out_slot, void* out, int64_t n,
                              void* stream) {
  mkc::clear_error();
  const char* fn = "mk_elementwise";
  if (!prog || !out || (n_inputs > 0 && (!inputs || !input_numel)))
    return mkc::fail(MK_EINVAL, "%s: null pointer argument", fn);
  if (dtype != MK_DT_F32 && dtype != MK_DT_BF16) return mkc::fail(MK_EUNSUPPORTED, "%s: dtype %d", fn, dtype);
  {
    const int rc = validate_program(fn, prog, n_instr, n_inputs, out_slot);
    if (rc != MK_OK) return rc;
  }
  if (n <= 0) return mkc::fail(MK_EINVAL, "%s: element count must be positive", fn);
  mk::EwArgs a;
  bool aligned = ((uintptr_t)out % 16 == 0) && (n % mk::kEwVec == 0);
  for (int i = 0; i < n_inputs; ++i) {
    if (!inputs[i]) return mkc::fail(MK_EINVAL, "%s: input %d is null", fn, i);
    if (input_numel[i] <= 0 || n % input_numel[i] != 0)
      return mkc::fail(MK_EINVAL, "%s: input %d has %lld elements (need 1, %lld or a divisor of it)", fn, i,
                       (long long)input_numel[i], (long long)n);
    a.in[i] = inputs[i];
    a.in_numel[i] = input_numel[i];
    if (input_numel[i] != 1 && (uintptr_t)inputs[i] % 16 != 0) aligned = false;
    if (input_numel[i] != 1 && input_numel[i] != n && input_numel[i] % mk::kEwVec != 0) aligned = false;
  }
  for (int i = n_inputs; i < mk::kEwMaxInputs; ++i) {
    a.in[i] = nullptr;
    a.in_numel[i] = 1;
  }
  for (int i = 0; i < n_instr; ++i) a.ins[i] = prog[i];
  a.out = out;
  a.n = n;
  a.n_instr = n_instr;
  a.out_slot = out_slot;
  const int64_t chunks = (n + mk::kEwVec - 1) / mk::kEwVec;
  const int blocks = (int)std::min<int64_t>((chunks + 255) / 256, 256 * 16);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (jit_enabled()) {
    // Generated straight-line kernel (compiled on the first call of this
    // program on this device; see mk_elementwise_prepare).
    void* k = nullptr;
    const int rc = mkc::ew_jit_get(dtype, prog, n_instr, n_inputs, out_slot, &k);
    if (rc != MK_OK) return rc;
    int vec_ok = aligned ? 1 : 0;
    long long nn[4] = {1, 1, 1, 1};
    for (int i = 0; i < n_inputs; ++i) nn[i] = (long long)a.in_numel[i];
    long long nl = (long long)n;
    void* args[] = {&a.in[0], &a.in[1], &a.in[2], &a.in[3], &nn[0], &nn[1], &nn[2], &nn[3], &a.out, &nl, &vec_ok};
    const int jblocks = (int)std::min<int64_t>((chunks + 255) / 256, 256 * 32);
    hipError_t e = hipModuleLaunchKernel((hipFunction_t)k, jblocks, 1, 1, 256, 1, 1, 0, st, args, nullptr);
    if (e != hipSuccess) return mkc::fail(MK_ELAUNCH, "%s: launch failed: %s", fn, hipGetErrorString(e));
    return MK_OK;
  }
  if (dtype == MK_DT_BF16) {
    if (aligned) hipLaunchKernelGGL((mk::eltwise_kernel<true, true>), dim3(blocks), dim3(256), 0, st, a);
    else hipLaunchKernelGGL((mk::eltwise_kernel<true, false>), dim3(blocks), dim3(256), 0, st, a);
  } else {
    if (aligned) hipLaunchKernelGGL((mk::eltwise_kernel<false, true>), dim3(blocks), dim3(256), 0, st, a);
    else hipLaunchKernelGGL((mk::eltwise_kernel<false, false>), dim3(blocks), dim3(256), 0, st, a);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return mkc::fail(MK_ELAUNCH, "%s: launch failed: %s", fn, hipGetErrorString(e));
  return MK_OK;
}
