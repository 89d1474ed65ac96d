// Device math for the fused elementwise kernels, shared by the precompiled
// interpreter (eltwise.hip expands MK_EW_MATH_DEFS) and the generated kernels
// (ew_jit.cpp embeds MK_EW_MATH_SRC, the same text as a string, in every
// program it compiles), so that both paths evaluate identical formulas.
//
// f32 accuracy (measured against float64 over dense sweeps by the GPU tests):
//   mk_exp    Cody-Waite reduction x = n*ln2 + r with a two-part ln2, the
//             hardware 2^y on |y| <= 1/2 and an exact ldexp; ~2 ulp, exact
//             overflow to +inf above ln(FLT_MAX), gradual underflow to 0.
//   mk_log1p  log(u) + (x - (u - 1)) / u with u = 1 + x: the second term is
//             what the rounding of u dropped, so for tiny x (u == 1) the
//             result is x itself.  The hardware log2 (v_log_f32) is within
//             1 ulp of log2 over [0.5, 2), 1 + 2^-23 included, so no series
//             is needed near 0; <= 1.9 ulp over every tested input.
//   mk_logistic 1 / (1 + mk_exp(-x)) with the hardware reciprocal (1 ulp),
//             within 4 ulp; below x = -80 the result is exp(x) itself
//             (relative difference < 1e-34), which keeps the denormal results
//             the reciprocal would flush.
// bf16 programs round every op's result to 8 significant bits, so exp and
// logistic use the short forms mk_exp_bf (2^(x*log2e), relative error
// < 2^-16) and mk_logistic_bf, and log1p of a bf16 value uses mk_log1p_bf:
// for |x| >= 2^-15, u = 1 + x is exact in f32 (x has 8 significant bits, the
// lowest at or above 2^-22; above 2^24 u rounds by at most 2^-24
// relative), so log2(u) * ln2 is within ~2 f32 ulp of log1p(x); below,
// log1p(x) = x (1 - x/2 + ...) rounds to x itself in bf16.  Infinities,
// NaN, -1 and below come out of the log as log1p defines them, and -0 stays
// -0 on the short branch.
// maximum/minimum are the IEEE 754-2019 operations (v_maximum3/v_minimum3 on
// gfx950): NaN propagates and -0 < +0, the StableHLO semantics.
#pragma once

#define MK_EW_MATH_DEFS                                                                 \
  __device__ __forceinline__ float mk_exp(float x) {                                    \
    const float L2E = 1.44269502f, LN2_HI = 0.693145751953125f, LN2_LO = 1.42860677e-06f; \
    const float xc = __builtin_fminf(__builtin_fmaxf(x, -104.0f), 89.0f);               \
    const float n = __builtin_rintf(xc * L2E);                                          \
    float r = __builtin_fmaf(-n, LN2_HI, xc);                                           \
    r = __builtin_fmaf(-n, LN2_LO, r);                                                  \
    const float y = __builtin_ldexpf(__builtin_amdgcn_exp2f(r * L2E), (int)n);          \
    return x != x ? x : y;                                                              \
  }                                                                                     \
  __device__ __forceinline__ float mk_log1p(float x) {                                  \
    const float LN2 = 0.693147182f;                                                     \
    const float u = 1.0f + x;                                                           \
    const float c = (x - (u - 1.0f)) * __builtin_amdgcn_rcpf(u + 0x1p-100f); \
    const float y = __builtin_fmaf(__builtin_amdgcn_logf(u), LN2, c);                   \
    return u == __builtin_inff() ? u : (x == 0.0f ? x : y); /* log1p(-0) = -0 */     \
  }                                                                                     \
  __device__ __forceinline__ float mk_log1p_bf(float x) {                               \
    return __builtin_fabsf(x) < 0x1p-15f ? x : __builtin_amdgcn_logf(1.0f + x) * 0.693147182f; \
  }                                                                                     \
  __device__ __forceinline__ float mk_exp_bf(float x) {                                 \
    return __builtin_exp2f(x * 1.44269502f);                                            \
  }                                                                                     \
  __device__ __forceinline__ float mk_logistic(float x) {                               \
    const float r = __builtin_amdgcn_rcpf(1.0f + mk_exp(-x));                           \
    return x < -80.0f ? mk_exp(x) : r;                                                  \
  }                                                                                     \
  __device__ __forceinline__ float mk_logistic_bf(float x) {                            \
    const float r = __builtin_amdgcn_rcpf(1.0f + mk_exp_bf(-x));                        \
    return x < -80.0f ? mk_exp_bf(x) : r;                                               \
  }                                                                                     \
  __device__ __forceinline__ float mk_max(float a, float b) {                           \
    return __builtin_elementwise_maximum(a, b);                                         \
  }                                                                                     \
  __device__ __forceinline__ float mk_min(float a, float b) {                           \
    return __builtin_elementwise_minimum(a, b);                                         \
  }

#define MK_EW_STR_(...) #__VA_ARGS__
#define MK_EW_STR(...) MK_EW_STR_(__VA_ARGS__)
#define MK_EW_MATH_SRC MK_EW_STR(MK_EW_MATH_DEFS)
