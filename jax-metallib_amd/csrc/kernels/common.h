// Shared device helpers for the gfx950 kernels of the MI355X PJRT plugin.
//
// All kernels are written for CDNA4 (gfx950): 64-lane wavefronts, MFMA
// matrix cores, 160 KB LDS per CU, 8 XCDs.  Every entry point in this
// directory is launched through the extern "C" layer in ../capi.cpp, which
// validates shapes on the host before any launch.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../../include/mk_kernels.h"

namespace mk {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

// IEEE round-to-nearest-even float -> bf16 bits (quiet NaN kept).  On gfx950
// the conversion lowers to v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
  __bf16 h = (__bf16)f;
  return (uint32_t)__builtin_bit_cast(uint16_t, h);
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return f32_to_bf16(lo) | (f32_to_bf16(hi) << 16);
}

// v_perm_b32: byte i of the result is byte sel.byte[i] of the 64-bit value
// {hi, lo}; selectors 0-3 pick lo's bytes, 4-7 pick hi's bytes.
__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}

__device__ __forceinline__ f32x4 mfma16x16x32(const u32x4& a, const u32x4& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

__device__ __forceinline__ f32x16 mfma32x32x16(const u32x4& a, const u32x4& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// Loads that must observe stores made by other workgroups of the same launch
// (split-K partials): bypass the non-coherent L1 with an agent-scope load.
__device__ __forceinline__ float load_agent(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Logical workgroup id that keeps runs of consecutive ids on one XCD.  The
// dispatcher hands workgroup b to XCD b % 8; when the grid is a multiple of 8
// this maps the b-th workgroup to logical id (b % 8) * (n / 8) + b / 8, so the
// logical ids [x*n/8, (x+1)*n/8) all run on XCD x and share its L2.
__device__ __forceinline__ uint32_t xcd_logical_id(uint32_t b, uint32_t n) {
  if ((n & 7u) != 0u) return b;
  return (b & 7u) * (n >> 3) + (b >> 3);
}

}  // namespace mk
