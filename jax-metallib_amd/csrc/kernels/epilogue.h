// Elementwise epilogues fused into the bf16 stores of the GEMM and
// dequant-matmul kernels (mk_gemm_bf16_epilogue, mk_*_matmul_epilogue_bf16).
// They reproduce, rounding for rounding, the separate bf16 elementwise
// programs they replace (every op rounded to bf16, r() below):
//   MK_EPI_ADD:    y = r(r(acc) + aux)                        (residual add)
//   MK_EPI_SWIGLU: u = r(acc), g = aux,
//                  y = r(r(g * r(logistic(g))) * u)           (silu(g) * u)
//   MK_EPI_SWIGLU_PAIRS: the same with g = r(acc) of the interleaved gate
//                  column and u = r(acc) of its up column (one GEMM).
// with the bf16 programs' own logistic (ew_math.h, mk_logistic_bf).
#pragma once

#include "common.h"
#include "ew_math.h"

namespace mk {

MK_EW_MATH_DEFS

__device__ __forceinline__ float epi_r(float v) { return bf16_to_f32(f32_to_bf16(v)); }

// Four consecutive bf16 outputs at y + off from f32 accumulators and the
// four bf16 aux values w of the same positions (already loaded).
__device__ __forceinline__ void epi_store_bf16x4_v(uint16_t* y, const u32x2& w, int epi, size_t off,
                                                   const f32x4& acc) {
  float v[4] = {acc.x, acc.y, acc.z, acc.w};
  if (epi != MK_EPI_NONE) {
    const float x[4] = {bf16_to_f32(w.x & 0xffffu), bf16_to_f32(w.x >> 16), bf16_to_f32(w.y & 0xffffu),
                        bf16_to_f32(w.y >> 16)};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float u = epi_r(v[e]);
      if (epi == MK_EPI_ADD) {
        v[e] = u + x[e];
      } else {
        const float sig = epi_r(mk_logistic_bf(x[e]));
        v[e] = epi_r(x[e] * sig) * u;
      }
    }
  }
  *reinterpret_cast<u32x2*>(y + off) = u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
}

// MK_EPI_SWIGLU_PAIRS: four bf16 outputs from the gate accumulators g and
// the up accumulators u of the same four positions, rounded as the two
// plain GEMMs would have stored them and then combined as MK_EPI_SWIGLU.
__device__ __forceinline__ void epi_store_swiglu_pair(uint16_t* y, size_t off, const f32x4& g, const f32x4& u) {
  float v[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float x = epi_r(g[e]);
    const float sig = epi_r(mk_logistic_bf(x));
    v[e] = epi_r(x * sig) * epi_r(u[e]);
  }
  *reinterpret_cast<u32x2*>(y + off) = u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
}

// The same, reading aux at the same offset (aux may equal y).
__device__ __forceinline__ void epi_store_bf16x4(uint16_t* y, const uint16_t* aux, int epi, size_t off,
                                                 const f32x4& acc) {
  u32x2 w = {0u, 0u};
  if (epi != MK_EPI_NONE) w = *reinterpret_cast<const u32x2*>(aux + off);
  epi_store_bf16x4_v(y, w, epi, off, acc);
}

}  // namespace mk
