// General dot_general: the cases the tiled GEMMs do not take.
//
// The reference's HandleDotGeneral (src/pjrt_plugin/ops/binary_ops.mm:644-1100)
// keeps these semantics, which this kernel reproduces:
//   * integer operands give exact results in the result type
//     (two's-complement wraparound; :806-809 and tests/test_int_dot.py), for
//     s8 / u8 / s16 / u16 / s32 / u32 / s64 / u64 inputs and any integer
//     result type (lax.dot with preferred_element_type=int32 included);
//   * K == 1 is a plain product, so a -0 product stays -0 as XLA:CPU keeps
//     it (:904-1004); for K >= 2 the sum starts from +0 as XLA's does;
//   * K == 0 is handled by the planner (zeros, :832-845);
//   * any K and N, and operands read through strides, so a transposed
//     operand (a @ a.T) or a vector needs no copy.
// Floating inputs (f32, bf16, f16; both the same type) accumulate in f32 in
// k order and store f32, bf16 or f16 (round to nearest even).
//
// One thread per output element, grid-stride: these are the shapes the
// tiled kernels reject, not throughput paths.
#include "common.h"

namespace mk {

struct DotArgs {
  const void* a;
  const void* b;
  void* c;
  int64_t batch, M, N, K;
  int64_t sa[3], sb[3];  // element strides: a (batch, m, k), b (batch, k, n)
  int out_type;          // PJRT_Buffer_Type numbering
};

template <typename T>
__device__ __forceinline__ uint64_t ld_int(const void* p, int64_t i) {
  // Sign- or zero-extends by the element type, then wraps into 64 bits.
  return (uint64_t)(int64_t)static_cast<const T*>(p)[i];
}

__device__ __forceinline__ float half_to_f32(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
__device__ __forceinline__ uint16_t f32_to_half(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

template <typename T>
__device__ __forceinline__ float ld_float(const void* p, int64_t i);
template <>
__device__ __forceinline__ float ld_float<float>(const void* p, int64_t i) {
  return static_cast<const float*>(p)[i];
}
template <>
__device__ __forceinline__ float ld_float<uint16_t>(const void* p, int64_t i) {  // bf16
  return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
}
template <>
__device__ __forceinline__ float ld_float<_Float16>(const void* p, int64_t i) {
  return half_to_f32(static_cast<const uint16_t*>(p)[i]);
}

enum : int { kS8 = 2, kS16 = 3, kS32 = 4, kS64 = 5, kU8 = 6, kU16 = 7, kU32 = 8, kU64 = 9, kF16 = 10,
             kF32 = 11, kBF16 = 13 };

template <typename T, bool INT>
__global__ __launch_bounds__(256) void dot_general_kernel(DotArgs p) {
  const int64_t total = p.batch * p.M * p.N;
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < total; e += (int64_t)gridDim.x * 256) {
    const int64_t n = e % p.N, bm = e / p.N, m = bm % p.M, b = bm / p.M;
    const int64_t ia = b * p.sa[0] + m * p.sa[1], ib = b * p.sb[0] + n * p.sb[2];
    if constexpr (INT) {
      uint64_t acc = 0;
      for (int64_t k = 0; k < p.K; ++k) acc += ld_int<T>(p.a, ia + k * p.sa[2]) * ld_int<T>(p.b, ib + k * p.sb[1]);
      switch (p.out_type) {
        case kS8: case kU8: static_cast<uint8_t*>(p.c)[e] = (uint8_t)acc; break;
        case kS16: case kU16: static_cast<uint16_t*>(p.c)[e] = (uint16_t)acc; break;
        case kS32: case kU32: static_cast<uint32_t*>(p.c)[e] = (uint32_t)acc; break;
        default: static_cast<uint64_t*>(p.c)[e] = acc; break;
      }
    } else {
      float acc = ld_float<T>(p.a, ia) * ld_float<T>(p.b, ib);
      if (p.K != 1) {
        acc = 0.f + acc;
        for (int64_t k = 1; k < p.K; ++k)
          acc = __builtin_fmaf(ld_float<T>(p.a, ia + k * p.sa[2]), ld_float<T>(p.b, ib + k * p.sb[1]), acc);
      }
      switch (p.out_type) {
        case kF32: static_cast<float*>(p.c)[e] = acc; break;
        case kBF16: static_cast<uint16_t*>(p.c)[e] = (uint16_t)f32_to_bf16(acc); break;
        default: static_cast<uint16_t*>(p.c)[e] = f32_to_half(acc); break;
      }
    }
  }
}

}  // namespace mk

#include "../capi_internal.h"

#include <algorithm>

namespace {

bool is_int(int t) { return t >= mk::kS8 && t <= mk::kU64; }
bool is_float(int t) { return t == mk::kF16 || t == mk::kF32 || t == mk::kBF16; }

}  // namespace

extern "C" int mk_dot_general(int type_a, int type_b, int type_out, const void* a, const void* b, void* c,
                              int64_t batch, int64_t M, int64_t N, int64_t K, const int64_t* a_strides,
                              const int64_t* b_strides, void* stream) {
  mkc::clear_error();
  const char* fn = "mk_dot_general";
  if (!a || !b || !c || !a_strides || !b_strides) return mkc::fail(MK_EINVAL, "%s: null pointer argument", fn);
  if (batch <= 0 || M <= 0 || N <= 0 || K <= 0)
    return mkc::fail(MK_EINVAL, "%s: batch, M, N, K must be positive (got %lld, %lld, %lld, %lld)", fn,
                     (long long)batch, (long long)M, (long long)N, (long long)K);
  if (type_a != type_b) return mkc::fail(MK_EUNSUPPORTED, "%s: operand types differ (%d, %d)", fn, type_a, type_b);
  const bool ints = is_int(type_a) && is_int(type_out);
  const bool floats = is_float(type_a) && (type_out == type_a || type_out == mk::kF32);
  if (!ints && !floats)
    return mkc::fail(MK_EUNSUPPORTED, "%s: operand type %d with result type %d", fn, type_a, type_out);
  for (int i = 0; i < 3; ++i)
    if (a_strides[i] < 0 || b_strides[i] < 0) return mkc::fail(MK_EINVAL, "%s: negative stride", fn);
  if (batch * M > ((int64_t)1 << 40) || M * N > ((int64_t)1 << 40) || K > ((int64_t)1 << 32))
    return mkc::fail(MK_EINVAL, "%s: shape too large", fn);
  mk::DotArgs p;
  p.a = a; p.b = b; p.c = c;
  p.batch = batch; p.M = M; p.N = N; p.K = K;
  for (int i = 0; i < 3; ++i) { p.sa[i] = a_strides[i]; p.sb[i] = b_strides[i]; }
  p.out_type = type_out;
  const int64_t total = batch * M * N;
  const unsigned grid = (unsigned)std::min<int64_t>((total + 255) / 256, 65536);
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (type_a) {
    case mk::kS8: hipLaunchKernelGGL((mk::dot_general_kernel<int8_t, true>), dim3(grid), dim3(256), 0, st, p); break;
    case mk::kU8: hipLaunchKernelGGL((mk::dot_general_kernel<uint8_t, true>), dim3(grid), dim3(256), 0, st, p); break;
    case mk::kS16: hipLaunchKernelGGL((mk::dot_general_kernel<int16_t, true>), dim3(grid), dim3(256), 0, st, p); break;
    case mk::kU16: hipLaunchKernelGGL((mk::dot_general_kernel<uint16_t, true>), dim3(grid), dim3(256), 0, st, p); break;
    case mk::kS32: hipLaunchKernelGGL((mk::dot_general_kernel<int32_t, true>), dim3(grid), dim3(256), 0, st, p); break;
    case mk::kU32: hipLaunchKernelGGL((mk::dot_general_kernel<uint32_t, true>), dim3(grid), dim3(256), 0, st, p); break;
    case mk::kS64: hipLaunchKernelGGL((mk::dot_general_kernel<int64_t, true>), dim3(grid), dim3(256), 0, st, p); break;
    case mk::kU64: hipLaunchKernelGGL((mk::dot_general_kernel<uint64_t, true>), dim3(grid), dim3(256), 0, st, p); break;
    case mk::kF32: hipLaunchKernelGGL((mk::dot_general_kernel<float, false>), dim3(grid), dim3(256), 0, st, p); break;
    case mk::kBF16: hipLaunchKernelGGL((mk::dot_general_kernel<uint16_t, false>), dim3(grid), dim3(256), 0, st, p); break;
    default: hipLaunchKernelGGL((mk::dot_general_kernel<_Float16, false>), dim3(grid), dim3(256), 0, st, p); break;
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return mkc::fail(MK_ELAUNCH, "%s: launch failed: %s", fn, hipGetErrorString(e));
  return MK_OK;
}
