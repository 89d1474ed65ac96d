// Last-axis row operations for gfx950: softmax, RMSNorm, argmax, sum, max.
//
// Semantics follow the reference's native row kernels and the XLA:CPU rules
// they emulate:
//   softmax  exp(x - max) / sum(exp(x - max)) along the last axis; a row whose
//            max is NaN or +-inf comes out all NaN (inf - inf = NaN), as the
//            reference's one-pass kernels do (runtime/metal_kernels.mm:1579-1740,
//            pattern core/mps_executable.mm:1922-2089).  bf16 keeps XLA:CPU's
//            rounding points, restated from the reference's f16 emulation
//            (metal_kernels.mm:1742-1819): d = r(x - m), e = r(exp d),
//            s = r(sum_f32 e), y = r(e / s).
//   rmsnorm  x * rsqrt(mean(x^2) + eps) * g, f32 internally (the reference has
//            no RMSNorm fusion; its nearest is LayerNorm, mps_executable.mm:1457).
//   argmax   index of the first NaN, else of the first maximum, -0 == +0
//            (ops/reduction_ops.mm:1478-1536); int32 output.
//   sum      f32 accumulation, output in the input dtype.
//   max      NaN-propagating, -0 < +0 (metal_kernels.mm:830-857 order key).
//
// Layout: X [rows, cols] row-major.  One 256-thread workgroup per row; each
// thread caches its share of the row in registers (VPT 16-byte vectors), so
// the row is read from HBM exactly once and written at most once.  Wave
// reductions use cross-lane shuffles, then one LDS exchange across the 4
// waves.  Rows longer than the register cache (or not a multiple of the
// vector width) take the streaming variant that re-reads the row.  argmax,
// max and min of rows up to 16 vectors per lane of one wave (32 for bf16)
// run one wave per row instead (row_wave_kernel).
#include "common.h"

#include <math.h>

#include <algorithm>
#include <cstdlib>

namespace mk {

constexpr int kRowThreads = 256;

// ROW_MIN is max of the negated row, negated back: negation is exact, NaN
// still propagates and -0 < +0 holds.
enum RowOp { ROW_SOFTMAX = 0, ROW_RMSNORM = 1, ROW_ARGMAX = 2, ROW_SUM = 3, ROW_MAX = 4, ROW_MIN = 5 };

struct RowArgs {
  const void* x;
  const void* g;  // RMSNorm weight [cols] (same dtype as x)
  void* y;
  int64_t rows, cols;
  float eps;
};

__device__ __forceinline__ float bf16r(float v) { return bf16_to_f32(f32_to_bf16(v)); }

// XLA max: NaN wins; +0 above -0 -- gfx950's IEEE 754-2019 maximum
// (v_maximum_f32), one instruction.
__device__ __forceinline__ float xmax(float a, float b) { return __builtin_elementwise_maximum(a, b); }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = xmax(v, __shfl_xor(v, o, 64));
  return v;
}

// (value, index) argmax combine: first NaN, else larger value, ties -> smaller
// index (-0 == +0 compare equal, so the earlier one wins).
__device__ __forceinline__ void arg_combine(float& v, int& i, float v2, int i2) {
  const bool n1 = v != v, n2 = v2 != v2;
  bool take;
  if (n1 || n2) take = n2 && (!n1 || i2 < i);
  else take = v2 > v || (v2 == v && i2 < i);
  if (take) {
    v = v2;
    i = i2;
  }
}

template <typename T>
struct Vec;
template <>
struct Vec<float> {
  static constexpr int N = 4;
  __device__ static void load(const void* p, int64_t idx, float (&o)[N]) {
    const f32x4 v = *reinterpret_cast<const f32x4*>(static_cast<const float*>(p) + idx);
    o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
  }
  __device__ static void store(void* p, int64_t idx, const float (&o)[N]) {
    *reinterpret_cast<f32x4*>(static_cast<float*>(p) + idx) = f32x4{o[0], o[1], o[2], o[3]};
  }
  __device__ static float load1(const void* p, int64_t idx) { return static_cast<const float*>(p)[idx]; }
  __device__ static void store1(void* p, int64_t idx, float v) { static_cast<float*>(p)[idx] = v; }
  static constexpr bool bf16 = false;
};
template <>
struct Vec<uint16_t> {
  static constexpr int N = 8;
  __device__ static void load(const void* p, int64_t idx, float (&o)[N]) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(p) + idx);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      o[2 * i] = bf16_to_f32(w[i] & 0xFFFFu);
      o[2 * i + 1] = bf16_to_f32(w[i] >> 16);
    }
  }
  __device__ static void store(void* p, int64_t idx, const float (&o)[N]) {
    u32x4 v;
    v.x = pack_bf16x2(o[0], o[1]);
    v.y = pack_bf16x2(o[2], o[3]);
    v.z = pack_bf16x2(o[4], o[5]);
    v.w = pack_bf16x2(o[6], o[7]);
    *reinterpret_cast<u32x4*>(static_cast<uint16_t*>(p) + idx) = v;
  }
  __device__ static float load1(const void* p, int64_t idx) {
    return bf16_to_f32(static_cast<const uint16_t*>(p)[idx]);
  }
  __device__ static void store1(void* p, int64_t idx, float v) {
    static_cast<uint16_t*>(p)[idx] = (uint16_t)f32_to_bf16(v);
  }
  static constexpr bool bf16 = true;
};

// Workgroup-wide reductions through one LDS exchange (4 waves).
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wv] = v;
  __syncthreads();
  return red[0] + red[1] + red[2] + red[3];
}

__device__ __forceinline__ float block_max(float v, float* red) {
  v = wave_max(v);
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wv] = v;
  __syncthreads();
  return xmax(xmax(red[0], red[1]), xmax(red[2], red[3]));
}

__device__ __forceinline__ int block_min_int(int v, int* red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = min(v, __shfl_xor(v, o, 64));
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wv] = v;
  __syncthreads();
  return min(min(red[0], red[1]), min(red[2], red[3]));
}

__device__ __forceinline__ void block_argmax(float& v, int& i, float* redv, int* redi) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float v2 = __shfl_xor(v, o, 64);
    const int i2 = __shfl_xor(i, o, 64);
    arg_combine(v, i, v2, i2);
  }
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) {
    redv[wv] = v;
    redi[wv] = i;
  }
  __syncthreads();
  v = redv[0];
  i = redi[0];
#pragma unroll
  for (int w = 1; w < 4; ++w) arg_combine(v, i, redv[w], redi[w]);
}

// Element e of a 16-byte vector of a row, as f32.
template <typename T>
__device__ __forceinline__ float row_elem(const u32x4& w, int e);
template <>
__device__ __forceinline__ float row_elem<float>(const u32x4& w, int e) {
  return __uint_as_float(w[e]);
}
template <>
__device__ __forceinline__ float row_elem<uint16_t>(const u32x4& w, int e) {
  const uint32_t u = w[e >> 1];
  return __uint_as_float((e & 1) ? (u & 0xFFFF0000u) : (u << 16));
}

// One wave per row for the order-free reductions (argmax, max, min): the
// wave caches the row in registers (VPW 16-byte vectors per lane, vector q of
// lane l at element (64 q + l) E), reduces it with cross-lane shuffles only
// -- no LDS, no barrier -- and its 4 sibling waves take the next rows.  A
// row in flight per wave instead of per workgroup keeps more bytes in flight
// per CU, and the short rows of a reduction no longer wait on workgroup
// barriers.  argmax keeps each vector's maximum from the first pass, so the
// second pass (the first index holding the row maximum, or the first NaN)
// tests one value per vector and then the elements of the vectors that
// match.  Same results as the workgroup kernel, bit for bit: max and min are
// exact in any order, and the index search returns the same first index.
template <typename T, int OP, int VPW>
__global__ __launch_bounds__(kRowThreads) void row_wave_kernel(RowArgs a) {
  using V = Vec<T>;
  constexpr int E = V::N;
  static_assert(OP == ROW_ARGMAX || OP == ROW_MAX || OP == ROW_MIN, "order-free reductions only");
  const int lane = threadIdx.x & 63;
  const float sg = OP == ROW_MIN ? -1.f : 1.f;
  for (int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); row < a.rows; row += (int64_t)gridDim.x * 4) {
    // The row stays in registers as loaded (bf16 pairs unpacked at each
    // use).  A buffer resource spanning the row returns zeros past its end,
    // so the loads need no per-lane guard; those vectors are masked below.
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<T*>(static_cast<const T*>(a.x) + row * a.cols), 0, (int)(a.cols * (int64_t)sizeof(T)), kBufWord3);
    const int cols = (int)a.cols;  // at most 32 * 64 * 8 here
    u32x4 raw[VPW];
    bool ok[VPW];
#pragma unroll
    for (int q = 0; q < VPW; ++q) {
      ok[q] = (q * kWave + lane) * E < cols;
      raw[q] = __builtin_amdgcn_raw_buffer_load_b128(rs, lane * 16, q * kWave * 16, 0);
    }
    // Vector maxima: kept for the index search up to 16 vectors per lane,
    // recomputed there beyond (VGPRs, hence waves per SIMD, matter more).
    constexpr bool kKeep = VPW <= 16;
    auto vec_max = [&](int q) {
      float t = sg * row_elem<T>(raw[q], 0);
#pragma unroll
      for (int e = 1; e < E; ++e) t = xmax(t, sg * row_elem<T>(raw[q], e));
      return ok[q] ? t : -INFINITY;
    };
    float cm[kKeep ? VPW : 1];
    float m = -INFINITY;
#pragma unroll
    for (int q = 0; q < VPW; ++q) {
      const float t = vec_max(q);
      if constexpr (kKeep) cm[q] = t;
      m = xmax(m, t);
    }
    m = wave_max(m);
    if (OP != ROW_ARGMAX) {
      if (lane == 0) V::store1(a.y, row, sg * m);
      continue;
    }
    // First vector of this lane holding the maximum (a NaN when m is NaN).
    const bool mnan = m != m;
    int bq = VPW;
#pragma unroll
    for (int q = VPW - 1; q >= 0; --q) {
      float t;
      if constexpr (kKeep) {
        t = cm[q];
      } else {
        asm volatile("" : "+v"(raw[q]));  // recompute, not the first pass's values
        t = vec_max(q);
      }
      if (ok[q] && (mnan ? t != t : t == m)) bq = q;
    }
    int be = 0;  // first matching element of vector bq
#pragma unroll
    for (int q = 0; q < VPW; ++q) {
      if (!__any(bq == q)) continue;
      if (bq == q) {
        // Unpack the vector again rather than keep the first pass's values
        // live across the search (they would cost 2 VGPRs per bf16 pair).
        asm volatile("" : "+v"(raw[q]));
#pragma unroll
        for (int e = E - 1; e >= 0; --e) {
          const float x = row_elem<T>(raw[q], e);
          if (mnan ? x != x : x == m) be = e;
        }
      }
    }
    int bi = bq < VPW ? (bq * kWave + lane) * E + be : 0x7FFFFFFF;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) bi = min(bi, __shfl_xor(bi, o, 64));
    if (lane == 0) static_cast<int32_t*>(a.y)[row] = bi == 0x7FFFFFFF ? 0 : bi;
  }
}

// Register-cached row kernel: the row is covered by 256 threads x VPT vectors
// (VPT * 256 * Vec::N >= cols, cols % Vec::N == 0, rows 16-byte aligned).
template <typename T, int OP, int VPT, bool GE = sizeof(T) == 4>
__global__ __launch_bounds__(kRowThreads) void row_cached_kernel(RowArgs a) {
  using V = Vec<T>;
  constexpr int E = V::N;
  __shared__ float redf[4];
  __shared__ int redi[4];
  // Rows are strided over the grid (the launch caps it), so any row count
  // fits a launch; every wave of a workgroup runs the same iterations, so
  // the barriers inside the reductions stay uniform.
  for (int64_t row = blockIdx.x; row < a.rows; row += gridDim.x) {
  const int64_t base = row * a.cols;
  const int tid = threadIdx.x;
  float v[VPT][E];
  bool ok[VPT];
#pragma unroll
  for (int q = 0; q < VPT; ++q) {
    const int64_t c = (int64_t)(q * kRowThreads + tid) * E;
    ok[q] = c < a.cols;
    if (ok[q]) V::load(a.x, base + c, v[q]);
  }
  // RMSNorm, GE: the weight g is loaded with the row, so its latency is not
  // exposed after the reduction.  8192^2 f32: 100.4 -> 91.6 us.  bf16 keeps
  // the load after the reduction: loaded early it costs VGPRs and waves per
  // SIMD (47.6 against 49.0 us packed, 52.9 us unpacked).
  u32x4 graw[OP == ROW_RMSNORM ? VPT : 1];
  if constexpr (OP == ROW_RMSNORM && GE) {
#pragma unroll
    for (int q = 0; q < VPT; ++q)
      if (ok[q])
        graw[q] = *reinterpret_cast<const u32x4*>(static_cast<const T*>(a.g) + (int64_t)(q * kRowThreads + tid) * E);
  }

  if (OP == ROW_SOFTMAX) {
    float m = -INFINITY;
#pragma unroll
    for (int q = 0; q < VPT; ++q)
      if (ok[q])
#pragma unroll
        for (int e = 0; e < E; ++e) m = xmax(m, v[q][e]);
    m = block_max(m, redf);
    float s = 0.f;
#pragma unroll
    for (int q = 0; q < VPT; ++q)
      if (ok[q])
#pragma unroll
        for (int e = 0; e < E; ++e) {
          float d = v[q][e] - m;
          if (V::bf16) d = bf16r(d);
          float ex = __expf(d);
          if (V::bf16) ex = bf16r(ex);
          v[q][e] = ex;
          s += ex;
        }
    s = block_sum(s, redf);
    if (V::bf16) s = bf16r(s);
    const float r = 1.0f / s;
    // bf16: y = r(e / s) with e / s the IEEE f32 quotient (XLA:CPU divides in
    // f32).  e and s carry 8 significant bits, so e / s is never an f32
    // rounding tie: q = RN(e * RN(1 / s)) is within one ulp of it, and one
    // Markstein correction, q + RN(1 / s) * (e - q s) with the remainder
    // exact in an FMA, gives it exactly.
#pragma unroll
    for (int q = 0; q < VPT; ++q)
      if (ok[q]) {
#pragma unroll
        for (int e = 0; e < E; ++e) {
          if (V::bf16) {
            const float q0 = v[q][e] * r;
            v[q][e] = __builtin_fmaf(__builtin_fmaf(-q0, s, v[q][e]), r, q0);
          } else {
            v[q][e] = v[q][e] * r;
          }
        }
        V::store(a.y, base + (int64_t)(q * kRowThreads + tid) * E, v[q]);
      }
  } else if (OP == ROW_RMSNORM) {
    float s = 0.f;
#pragma unroll
    for (int q = 0; q < VPT; ++q)
      if (ok[q])
#pragma unroll
        for (int e = 0; e < E; ++e) s += v[q][e] * v[q][e];
    s = block_sum(s, redf);
    const float r = rsqrtf(s / (float)a.cols + a.eps);
#pragma unroll
    for (int q = 0; q < VPT; ++q)
      if (ok[q]) {
        const int64_t c = (int64_t)(q * kRowThreads + tid) * E;
        if constexpr (!GE) graw[q] = *reinterpret_cast<const u32x4*>(static_cast<const T*>(a.g) + c);
#pragma unroll
        for (int e = 0; e < E; ++e) v[q][e] = v[q][e] * r * row_elem<T>(graw[q], e);
        V::store(a.y, base + c, v[q]);
      }
  } else if (OP == ROW_ARGMAX) {
    // Two passes over the cached row: the NaN-propagating row maximum m,
    // then the first index holding it (the first NaN when m is NaN; -0 and
    // +0 compare equal, so the earlier zero wins).  Each thread's indices
    // rise with (q, e), so a reverse walk that overwrites keeps its first.
    float m = -INFINITY;
#pragma unroll
    for (int q = 0; q < VPT; ++q)
      if (ok[q])
#pragma unroll
        for (int e = 0; e < E; ++e) m = xmax(m, v[q][e]);
    m = block_max(m, redf);
    int bi = 0x7FFFFFFF;
    if (m != m) {
#pragma unroll
      for (int q = VPT - 1; q >= 0; --q)
        if (ok[q])
#pragma unroll
          for (int e = E - 1; e >= 0; --e) bi = v[q][e] != v[q][e] ? (q * kRowThreads + tid) * E + e : bi;
    } else {
#pragma unroll
      for (int q = VPT - 1; q >= 0; --q)
        if (ok[q])
#pragma unroll
          for (int e = E - 1; e >= 0; --e) bi = v[q][e] == m ? (q * kRowThreads + tid) * E + e : bi;
    }
    bi = block_min_int(bi, redi);
    if (tid == 0) static_cast<int32_t*>(a.y)[row] = bi == 0x7FFFFFFF ? 0 : bi;
  } else if (OP == ROW_SUM) {
    float s = 0.f;
#pragma unroll
    for (int q = 0; q < VPT; ++q)
      if (ok[q])
#pragma unroll
        for (int e = 0; e < E; ++e) s += v[q][e];
    s = block_sum(s, redf);
    if (tid == 0) V::store1(a.y, row, s);
  } else {  // ROW_MAX, ROW_MIN
    const float sg = OP == ROW_MIN ? -1.f : 1.f;
    float m = -INFINITY;
#pragma unroll
    for (int q = 0; q < VPT; ++q)
      if (ok[q])
#pragma unroll
        for (int e = 0; e < E; ++e) m = xmax(m, sg * v[q][e]);
    m = block_max(m, redf);
    if (tid == 0) V::store1(a.y, row, sg * m);
  }
  }
}

// Streaming row kernel for any cols: scalar strided passes over the row
// (max / sums first, then the output pass re-reads the row).
template <typename T, int OP>
__global__ __launch_bounds__(kRowThreads) void row_stream_kernel(RowArgs a) {
  using V = Vec<T>;
  __shared__ float redf[4];
  __shared__ int redi[4];
  for (int64_t row = blockIdx.x; row < a.rows; row += gridDim.x) {
  const int64_t base = row * a.cols;
  const int tid = threadIdx.x;
  if (OP == ROW_SOFTMAX) {
    float m = -INFINITY;
    for (int64_t c = tid; c < a.cols; c += kRowThreads) m = xmax(m, V::load1(a.x, base + c));
    m = block_max(m, redf);
    float s = 0.f;
    for (int64_t c = tid; c < a.cols; c += kRowThreads) {
      float d = V::load1(a.x, base + c) - m;
      if (V::bf16) d = bf16r(d);
      float ex = __expf(d);
      if (V::bf16) ex = bf16r(ex);
      s += ex;
    }
    s = block_sum(s, redf);
    if (V::bf16) s = bf16r(s);
    const float r = 1.0f / s;
    for (int64_t c = tid; c < a.cols; c += kRowThreads) {
      float d = V::load1(a.x, base + c) - m;
      if (V::bf16) d = bf16r(d);
      float ex = __expf(d);
      if (V::bf16) ex = bf16r(ex);
      float y = ex * r;
      if (V::bf16) y = __builtin_fmaf(__builtin_fmaf(-y, s, ex), r, y);  // the exact quotient, as above
      V::store1(a.y, base + c, y);
    }
  } else if (OP == ROW_RMSNORM) {
    float s = 0.f;
    for (int64_t c = tid; c < a.cols; c += kRowThreads) {
      const float x = V::load1(a.x, base + c);
      s += x * x;
    }
    s = block_sum(s, redf);
    const float r = rsqrtf(s / (float)a.cols + a.eps);
    for (int64_t c = tid; c < a.cols; c += kRowThreads)
      V::store1(a.y, base + c, V::load1(a.x, base + c) * r * V::load1(a.g, c));
  } else if (OP == ROW_ARGMAX) {
    float bv = -INFINITY;
    int bi = 0x7FFFFFFF;
    bool nan = false;
    int nan_i = 0x7FFFFFFF;
    for (int64_t c = tid; c < a.cols; c += kRowThreads) {
      const float x = V::load1(a.x, base + c);
      if (x != x) {
        if (!nan) {
          nan = true;
          nan_i = (int)c;
        }
      } else if (x > bv || bi == 0x7FFFFFFF) {
        bv = x;
        bi = (int)c;
      }
    }
    float rv = nan ? NAN : bv;
    int ri = nan ? nan_i : bi;
    block_argmax(rv, ri, redf, redi);
    if (tid == 0) static_cast<int32_t*>(a.y)[row] = ri == 0x7FFFFFFF ? 0 : ri;
  } else if (OP == ROW_SUM) {
    float s = 0.f;
    for (int64_t c = tid; c < a.cols; c += kRowThreads) s += V::load1(a.x, base + c);
    s = block_sum(s, redf);
    if (tid == 0) V::store1(a.y, row, s);
  } else {  // ROW_MAX, ROW_MIN
    const float sg = OP == ROW_MIN ? -1.f : 1.f;
    float m = -INFINITY;
    for (int64_t c = tid; c < a.cols; c += kRowThreads) m = xmax(m, sg * V::load1(a.x, base + c));
    m = block_max(m, redf);
    if (tid == 0) V::store1(a.y, row, sg * m);
  }
  }
}

}  // namespace mk

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
#include "../capi_internal.h"

namespace {

constexpr int64_t kMaxRowBlocks = 1 << 20;

// MK_ROW_WAVE=0 keeps argmax / max / min on the workgroup-per-row kernels
// (same results).
bool row_wave_enabled() {
  const char* v = getenv("MK_ROW_WAVE");
  return !(v && v[0] == '0');
}

template <typename T, int OP>
hipError_t launch_row(const mk::RowArgs& a, hipStream_t st) {
  constexpr int E = mk::Vec<T>::N;
  const bool aligned = a.cols % E == 0 && ((uintptr_t)a.x % 16 == 0) && ((uintptr_t)a.y % 16 == 0 || OP >= mk::ROW_ARGMAX) &&
                       (OP != mk::ROW_RMSNORM || (uintptr_t)a.g % 16 == 0);
  const int64_t vecs = (a.cols + E - 1) / E;
  const int64_t vpt = (vecs + mk::kRowThreads - 1) / mk::kRowThreads;
  // One workgroup per row up to kMaxRowBlocks rows (2^28 work-items); more
  // rows stride over that grid.
  dim3 grid((unsigned)std::min<int64_t>(a.rows, kMaxRowBlocks)), block(mk::kRowThreads);
  if constexpr (OP == mk::ROW_ARGMAX || OP == mk::ROW_MAX || OP == mk::ROW_MIN) {
    // One wave per row while a lane's share fits 16 vectors (bf16 8192, f32
    // 4096 columns), and bf16 rows up to 32 vectors.  Measured argmax, 10
    // rotating inputs, against the workgroup kernels: bf16 8192^2 28.2 ->
    // 26.3 us, bf16 65536 x 1024 56.2 -> 25.8 us, f32 65536 x 1024 58.3 ->
    // 44.5 us, bf16 8192 x 16384 75.3 -> 49.9 us; f32 8192^2 (32 vectors)
    // 43.5 -> 47.2 us, so f32 rows of 32 vectors stay on the workgroup kernel.
    const int64_t vpw = (vecs + mk::kWave - 1) / mk::kWave;
    if (aligned && (vpw <= 16 || (vpw <= 32 && sizeof(T) == 2)) && row_wave_enabled()) {
      dim3 wgrid((unsigned)std::min<int64_t>((a.rows + 3) / 4, kMaxRowBlocks));
      if (vpw <= 1) hipLaunchKernelGGL((mk::row_wave_kernel<T, OP, 1>), wgrid, block, 0, st, a);
      else if (vpw <= 2) hipLaunchKernelGGL((mk::row_wave_kernel<T, OP, 2>), wgrid, block, 0, st, a);
      else if (vpw <= 4) hipLaunchKernelGGL((mk::row_wave_kernel<T, OP, 4>), wgrid, block, 0, st, a);
      else if (vpw <= 8) hipLaunchKernelGGL((mk::row_wave_kernel<T, OP, 8>), wgrid, block, 0, st, a);
      else if (vpw <= 16) hipLaunchKernelGGL((mk::row_wave_kernel<T, OP, 16>), wgrid, block, 0, st, a);
      else if constexpr (sizeof(T) == 2) hipLaunchKernelGGL((mk::row_wave_kernel<T, OP, 32>), wgrid, block, 0, st, a);
      return hipGetLastError();
    }
  }
  if (aligned && vpt <= 16) {
    if (vpt <= 1) hipLaunchKernelGGL((mk::row_cached_kernel<T, OP, 1>), grid, block, 0, st, a);
    else if (vpt <= 2) hipLaunchKernelGGL((mk::row_cached_kernel<T, OP, 2>), grid, block, 0, st, a);
    else if (vpt <= 4) hipLaunchKernelGGL((mk::row_cached_kernel<T, OP, 4>), grid, block, 0, st, a);
    else if (vpt <= 8) hipLaunchKernelGGL((mk::row_cached_kernel<T, OP, 8>), grid, block, 0, st, a);
    else hipLaunchKernelGGL((mk::row_cached_kernel<T, OP, 16>), grid, block, 0, st, a);
  } else {
    hipLaunchKernelGGL((mk::row_stream_kernel<T, OP>), grid, block, 0, st, a);
  }
  return hipGetLastError();
}

template <int OP>
int run_row(const char* fn, int dtype, const void* x, const void* g, void* y, int64_t rows,
            int64_t cols, float eps, void* stream) {
  mkc::clear_error();
  if (!x || !y || (OP == mk::ROW_RMSNORM && !g)) return mkc::fail(MK_EINVAL, "%s: null pointer argument", fn);
  if (rows <= 0 || cols <= 0) return mkc::fail(MK_EINVAL, "%s: rows and cols must be positive", fn);
  if (rows > 0x7FFFFFFF || cols > 0x7FFFFFFF) return mkc::fail(MK_EINVAL, "%s: shape too large", fn);
  if (dtype != MK_DT_F32 && dtype != MK_DT_BF16) return mkc::fail(MK_EUNSUPPORTED, "%s: dtype %d", fn, dtype);
  mk::RowArgs a{x, g, y, rows, cols, eps};
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipError_t e = dtype == MK_DT_F32 ? launch_row<float, OP>(a, st) : launch_row<uint16_t, OP>(a, st);
  if (e != hipSuccess) return mkc::fail(MK_ELAUNCH, "%s: launch failed: %s", fn, hipGetErrorString(e));
  return MK_OK;
}

}  // namespace

extern "C" int mk_softmax_lastdim(int dtype, const void* x, void* y, int64_t rows, int64_t cols,
                                  void* stream) {
  return run_row<mk::ROW_SOFTMAX>("mk_softmax_lastdim", dtype, x, nullptr, y, rows, cols, 0.f, stream);
}

extern "C" int mk_rmsnorm_lastdim(int dtype, const void* x, const void* g, void* y, int64_t rows,
                                  int64_t cols, float eps, void* stream) {
  return run_row<mk::ROW_RMSNORM>("mk_rmsnorm_lastdim", dtype, x, g, y, rows, cols, eps, stream);
}

extern "C" int mk_argmax_lastdim(int dtype, const void* x, void* out_i32, int64_t rows, int64_t cols,
                                 void* stream) {
  return run_row<mk::ROW_ARGMAX>("mk_argmax_lastdim", dtype, x, nullptr, out_i32, rows, cols, 0.f, stream);
}

extern "C" int mk_reduce_lastdim(int dtype, int op, const void* x, void* y, int64_t rows, int64_t cols,
                                 void* stream) {
  if (op == MK_REDUCE_SUM)
    return run_row<mk::ROW_SUM>("mk_reduce_lastdim", dtype, x, nullptr, y, rows, cols, 0.f, stream);
  if (op == MK_REDUCE_MAX)
    return run_row<mk::ROW_MAX>("mk_reduce_lastdim", dtype, x, nullptr, y, rows, cols, 0.f, stream);
  if (op == MK_REDUCE_MIN)
    return run_row<mk::ROW_MIN>("mk_reduce_lastdim", dtype, x, nullptr, y, rows, cols, 0.f, stream);
  mkc::clear_error();
  return mkc::fail(MK_EUNSUPPORTED, "mk_reduce_lastdim: op %d", op);
}
