// Decode-shaped quantized matmul for gfx950: y[M,N] = x[M,K] @ dequant(W)[K,N].
//
// Workload formats (the jnp programs the plugin recognises; the reference's
// own quantized GEMM is quantized.py:760-958 with W [N, K] uint32 words):
//   int4 g64: W uint8 [K/2, N], low nibble = even k; scale bf16 [K/64, N];
//             zero uint8 [K/64, N].  y = x @ ((W - zero) * scale).
//   int8 pc:  W int8 [K, N]; scale f32 [N].  y = x @ (W * scale).
//
// Design (HBM bound at M <= 16: 29.4 MB of int4 weight per call at the
// workload shape, 4.1 us at 8 TB/s):
//   * One workgroup owns 64 output columns and (normally) all of K, split
//     over its waves; the wave partials are summed through LDS, so no
//     workgroup ever waits on another (no device-scope fences: on gfx950 they
//     write back / invalidate the per-XCD L2).  Only when x does not fit in
//     LDS, or the grid would be too small, is K split across workgroups; the
//     partials then go to a workspace and a second small kernel sums them.
//   * Each lane streams weight bytes as dwords: 4 (int4) or 8 (int8)
//     consecutive W rows x 4 columns, so every W row is read by 16 lanes as
//     64 contiguous bytes and neighbouring column tiles (which share 128-byte
//     lines) run on the same XCD.  Loads are issued kQPF groups ahead.
//   * The bytes are transposed in registers with v_perm_b32 so each lane
//     holds, per column, the consecutive-k run that the MFMA B operand wants,
//     and are turned into bf16 without converts:
//       int4: bf16 bits 0x4300 | q  ==  128 + q     (exact)
//       int8: (w ^ 0x80) = w + 128, u8 -> f32 -> bf16 (exact, 8 bits)
//     The constant offset is removed algebraically with the x row sums:
//       sum_k x (q - z) = sum_k x (128 + q) - (128 + z) * sum_k x
//   * int4 groups: each 64-k group is accumulated by two
//     v_mfma_f32_16x16x32_bf16 from zero, then folded into the running sum
//     with its scale, y += s * (acc - (128 + z) * xsum) -- the scale is
//     applied per group on the 16x16 MFMA tile instead of per weight.
//   * x is staged once per wave in LDS, pre-permuted into the MFMA A-operand
//     order.  The x row sums come from one extra MFMA per step against a B
//     operand of bf16 ones, which lands them directly in the accumulator
//     layout (lane (c, j) holds rows 4j..4j+3).
//
// Numerics: products bf16 x bf16 are exact in the MFMA and accumulate in
// f32.  The dequantised weight (q - z) * s is used exactly; XLA:CPU rounds
// that product to bf16 first (reference ops/registry.h:273-287), which is
// within the workload's bf16 tolerance.
#include "common.h"
#include "epilogue.h"

#include <algorithm>
#include <atomic>
#include <cstring>

namespace mk {

constexpr int kQCols = 64;   // output columns per workgroup
constexpr int kQRows = 16;   // x rows per MFMA row block
constexpr int kQPF = 4;      // weight groups (int4) / steps (int8) in flight

struct QArgs {
  const uint16_t* x;
  const uint8_t* w;
  const void* s;     // int4: bf16 [K/64, N]; int8: f32 [N]
  const uint8_t* z;  // int4 only
  uint16_t* y;
  float* part;       // [rowblocks][ks][16][N] split-K partials (ks > 1)
  int M, K, N;
  int ks;            // workgroups per column tile (split-K)
  int kwave;         // k handled by one wave (multiple of 64)
  int wave_lds;      // bytes of LDS per wave (x staging, then partial y)
  uint32_t* cnt;     // wide kernel, ks > 1: per-tile arrival counters (zero between calls)
  const uint16_t* aux;  // epilogue operand (bf16 [M, N]) or null
  int epi;              // MK_EPI_* applied by every kernel's bf16 store
  int xch_local;        // wide int4 kernel: split-K exchange inside one XCD's L2 (see wide_finish)
};

// Stage this wave's x block [16 rows][kwave] into LDS as 16-byte MFMA A
// fragments, index ((step * 4 + kblock) * 16 + row), permuted within each
// 8-k run by PERM (int4: slots k0 k2 k4 k6 k1 k3 k5 k7; int8: identity).
template <bool PERM>
__device__ __forceinline__ void stage_x(const QArgs& a, u32x4* xl, int lane, int m0, int mrows,
                                        int kbeg) {
  const int chunks_per_row = a.kwave >> 3;
  const int total = kQRows * chunks_per_row;
  for (int q = lane; q < total; q += kWave) {
    const int m = q / chunks_per_row;
    const int kc = q - m * chunks_per_row;
    u32x4 v = {0u, 0u, 0u, 0u};
    if (m < mrows) {
      v = *reinterpret_cast<const u32x4*>(a.x + (size_t)(m0 + m) * a.K + kbeg + 8 * kc);
    }
    if (PERM) {
      u32x4 p;
      p.x = perm(v.y, v.x, 0x05040100u);  // k0, k2
      p.y = perm(v.w, v.z, 0x05040100u);  // k4, k6
      p.z = perm(v.y, v.x, 0x07060302u);  // k1, k3
      p.w = perm(v.w, v.z, 0x07060302u);  // k5, k7
      v = p;
    }
    const int st = kc >> 2, jj = kc & 3;
    xl[(st * 4 + jj) * 16 + m] = v;
  }
}

// 4x4 byte transpose: rows r0..r3 (4 bytes each) -> columns c0..c3, where
// column b holds byte b of r0, r1, r2, r3 in bytes 0..3.
__device__ __forceinline__ void transpose4x4(uint32_t r0, uint32_t r1, uint32_t r2, uint32_t r3,
                                             uint32_t& c0, uint32_t& c1, uint32_t& c2,
                                             uint32_t& c3) {
  const uint32_t x0 = perm(r1, r0, 0x05010400u);  // r0.b0 r1.b0 r0.b1 r1.b1
  const uint32_t x1 = perm(r1, r0, 0x07030602u);  // r0.b2 r1.b2 r0.b3 r1.b3
  const uint32_t y0 = perm(r3, r2, 0x05010400u);
  const uint32_t y1 = perm(r3, r2, 0x07030602u);
  c0 = perm(y0, x0, 0x05040100u);
  c1 = perm(y0, x0, 0x07060302u);
  c2 = perm(y1, x1, 0x05040100u);
  c3 = perm(y1, x1, 0x07060302u);
}

// Column dword t (byte r = W row r: low nibble k = 2r, high nibble 2r + 1)
// -> MFMA B fragment of bf16 (128 + q) in slot order k0 k2 k4 k6 k1 k3 k5 k7.
__device__ __forceinline__ u32x4 unpack_int4(uint32_t t) {
  const uint32_t lo = t & 0x0F0F0F0Fu;
  const uint32_t hi = (t >> 4) & 0x0F0F0F0Fu;
  const uint32_t C = 0x43434343u;
  u32x4 b;
  b.x = perm(C, lo, 0x04010400u);
  b.y = perm(C, lo, 0x04030402u);
  b.z = perm(C, hi, 0x04010400u);
  b.w = perm(C, hi, 0x04030402u);
  return b;
}

template <int B>
__device__ __forceinline__ float ubyte_f32(uint32_t v) {
  return (float)((v >> (8 * B)) & 0xFFu);  // v_cvt_f32_ubyte<B>
}

// Two column dwords (bytes = k 0..3 and 4..7 of int8 weights) -> bf16
// fragment of (w + 128) in natural k order.
__device__ __forceinline__ u32x4 unpack_int8(uint32_t t0, uint32_t t1) {
  t0 ^= 0x80808080u;
  t1 ^= 0x80808080u;
  u32x4 b;
  b.x = pack_bf16x2(ubyte_f32<0>(t0), ubyte_f32<1>(t0));
  b.y = pack_bf16x2(ubyte_f32<2>(t0), ubyte_f32<3>(t0));
  b.z = pack_bf16x2(ubyte_f32<0>(t1), ubyte_f32<1>(t1));
  b.w = pack_bf16x2(ubyte_f32<2>(t1), ubyte_f32<3>(t1));
  return b;
}

// Write this wave's y fragments ([4 tiles][4 rows]) into its LDS region as
// [16][64] f32: lane (c, j) holds rows 4j..4j+3, columns 4c..4c+3.
__device__ __forceinline__ void spill_y(unsigned char* wsm, const f32x4 (&y)[4], int c, int j) {
  float* red = reinterpret_cast<float*>(wsm);
#pragma unroll
  for (int i = 0; i < 4; ++i)
    *reinterpret_cast<f32x4*>(red + (4 * j + i) * kQCols + 4 * c) =
        f32x4{y[0][i], y[1][i], y[2][i], y[3][i]};
}

// Four device-coherent 16-byte loads (sc1: they miss the local L2) in flight
// together.
__device__ __forceinline__ void ld4_sc1(const float* p0, const float* p1, const float* p2, const float* p3,
                                        f32x4& v0, f32x4& v1, f32x4& v2, f32x4& v3) {
  asm volatile(
      "global_load_dwordx4 %0, %4, off sc1\n\t"
      "global_load_dwordx4 %1, %5, off sc1\n\t"
      "global_load_dwordx4 %2, %6, off sc1\n\t"
      "global_load_dwordx4 %3, %7, off sc1\n\t"
      "s_waitcnt vmcnt(0)"
      : "=&v"(v0), "=&v"(v1), "=&v"(v2), "=&v"(v3)
      : "v"(p0), "v"(p1), "v"(p2), "v"(p3)
      : "memory");
}

// Two device-coherent 16-byte loads in flight together.
__device__ __forceinline__ void ld2_sc1(const float* p0, const float* p1, f32x4& v0, f32x4& v1) {
  asm volatile(
      "global_load_dwordx4 %0, %2, off sc1\n\t"
      "global_load_dwordx4 %1, %3, off sc1\n\t"
      "s_waitcnt vmcnt(0)"
      : "=&v"(v0), "=&v"(v1)
      : "v"(p0), "v"(p1)
      : "memory");
}

// Two device-coherent 16-byte stores (sc1: written through past the per-XCD
// L2) and the wait for their acknowledgement, in one block: no instruction
// may overwrite a store's data registers before the store has read them (a
// hazard the compiler does not see inside inline asm).
__device__ __forceinline__ void st2_sc1_wait(float* p0, const f32x4& v0, float* p1, const f32x4& v1) {
  asm volatile(
      "global_store_dwordx4 %0, %2, off sc1\n\t"
      "global_store_dwordx4 %1, %3, off sc1\n\t"
      "s_waitcnt vmcnt(0)" ::"v"(p0),
      "v"(p1), "v"(v0), "v"(v1)
      : "memory");
}

// One device-coherent 16-byte load.
__device__ __forceinline__ f32x4 ld1_sc1(const float* p) {
  f32x4 v;
  asm volatile("global_load_dwordx4 %0, %1, off sc1\n\ts_waitcnt vmcnt(0)" : "=&v"(v) : "v"(p) : "memory");
  return v;
}

// One device-coherent 16-byte store and the wait for its acknowledgement
// (one asm block, as for st2_sc1_wait below).
__device__ __forceinline__ void st1_sc1_wait(float* p, const f32x4& v) {
  asm volatile("global_store_dwordx4 %0, %1, off sc1\n\ts_waitcnt vmcnt(0)" ::"v"(p), "v"(v) : "memory");
}

// Sum the NW wave tiles of the workgroup and emit bf16 y (ks == 1, with the
// int8 per-channel scale when FMT8) or the f32 split-K partial (ks > 1).
// With a.cnt set the split-K partials are combined here, as in the wide
// kernels: device-coherent (sc1) stores of the partial, acknowledged, a
// device-scope arrival count per tile, and the last arriver sums the ks
// partials in k order from 0 (the separate reduce pass's order, so the two
// give the same bits) and stores y.  Without a.cnt a second kernel
// (qmm_splitk_reduce_kernel) does that.
template <int NW, bool FMT8>
__device__ __forceinline__ void reduce_and_store(const QArgs& a, unsigned char* smem, int ksi,
                                                 int rb, int m0, int mrows, int n0) {
  constexpr int kItems = kQRows * (kQCols / 4);
  constexpr int IPT = (kItems + NW * kWave - 1) / (NW * kWave);  // items per thread
  // FMT8: this thread's per-channel scales, loaded before the sums so their
  // latency is not added after the last arriver's partial loads.
  f32x4 scl[FMT8 ? IPT : 1];
  if constexpr (FMT8) {
#pragma unroll
    for (int i = 0; i < IPT; ++i) {
      const int item = threadIdx.x + i * NW * kWave;
      const int n = n0 + 4 * (item % (kQCols / 4));
      scl[i] = f32x4{1.f, 1.f, 1.f, 1.f};
      if (item < kItems && n < a.N) scl[i] = *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(a.s) + n);
    }
  }
  __syncthreads();
  const bool exchange = a.ks > 1 && a.cnt != nullptr;
#pragma unroll
  for (int i = 0; i < IPT; ++i) {
    const int item = threadIdx.x + i * NW * kWave;
    if (item >= kItems) break;
    const int m = item / (kQCols / 4), ch = item % (kQCols / 4);
    const int n = n0 + 4 * ch;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < NW; ++w)
      acc += *reinterpret_cast<const f32x4*>(smem + w * a.wave_lds + (m * kQCols + 4 * ch) * 4);
    if (m >= mrows || n >= a.N) continue;
    float* dst = a.part + ((size_t)(rb * a.ks + ksi) * kQRows + m) * a.N + n;
    if (exchange) {
      st1_sc1_wait(dst, acc);
    } else if (a.ks > 1) {
      *reinterpret_cast<f32x4*>(dst) = acc;
    } else {
      if constexpr (FMT8) acc *= scl[i];
      epi_store_bf16x4(a.y, a.aux, a.epi, (size_t)(m0 + m) * a.N + n, acc);
    }
  }
  if (!exchange) return;
  // Every thread's partial stores are acknowledged, and every wave is done
  // reading the spills, before thread 0 counts this workgroup in.
  __syncthreads();
  volatile uint32_t* flag = reinterpret_cast<volatile uint32_t*>(smem);
  if (threadIdx.x == 0) {
    const int ntiles = (a.N + kQCols - 1) / kQCols;
    uint32_t* ctr = a.cnt + rb * ntiles + n0 / kQCols;
    asm volatile("" : "+v"(ctr));  // per-lane address: a vector atomic
    const uint32_t old = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t last = old == (uint32_t)(a.ks - 1);
    if (last) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *flag = last;
  }
  __syncthreads();
  if (!*flag) return;
#pragma unroll
  for (int i = 0; i < IPT; ++i) {
    const int item = threadIdx.x + i * NW * kWave;
    if (item >= kItems) break;
    const int m = item / (kQCols / 4), ch = item % (kQCols / 4);
    const int n = n0 + 4 * ch;
    if (m >= mrows || n >= a.N) continue;
    const float* src = a.part + ((size_t)rb * a.ks * kQRows + m) * a.N + n;
    const size_t kstride = (size_t)kQRows * a.N;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    int k = 0;
    for (; k + 4 <= a.ks; k += 4) {
      f32x4 v0, v1, v2, v3;
      ld4_sc1(src + k * kstride, src + (k + 1) * kstride, src + (k + 2) * kstride, src + (k + 3) * kstride, v0, v1,
              v2, v3);
      acc += v0;
      acc += v1;
      acc += v2;
      acc += v3;
    }
    for (; k < a.ks; ++k) acc += ld1_sc1(src + k * kstride);
    if constexpr (FMT8) acc *= scl[i];
    epi_store_bf16x4(a.y, a.aux, a.epi, (size_t)(m0 + m) * a.N + n, acc);
  }
}

template <int NW>
__global__ __launch_bounds__(NW * kWave) void int4g64_gemv_kernel(QArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const uint32_t L = xcd_logical_id(blockIdx.x, gridDim.x);
  const int tile = (int)(L / (uint32_t)a.ks);
  const int ksi = (int)(L - (uint32_t)tile * a.ks);
  const int rb = blockIdx.y;
  const int m0 = rb * kQRows;
  const int mrows = min(kQRows, a.M - m0);
  const int n0 = tile * kQCols;
  const int c = lane & 15, j = lane >> 4;
  const int kbeg = ksi * (a.K / a.ks) + wv * a.kwave;
  // Columns past N (last tile) read column N-4 instead: their results are
  // never stored, and every load stays in bounds without a branch.
  const int ncol = min(n0 + 4 * c, a.N - 4);
  const int ngroups = a.kwave >> 6;
  const uint32_t N = (uint32_t)a.N;

  unsigned char* wsm = smem + wv * a.wave_lds;
  u32x4* xl = reinterpret_cast<u32x4*>(wsm);

  // Per-wave (uniform) base pointers plus 32-bit per-lane offsets, so the
  // loads use the scalar-base addressing mode.  Lane rows: kp = kbeg/2 +
  // 32*g + 16*h + 4*j + r for group g, step h.
  const uint8_t* wwave = a.w + (size_t)(kbeg / 2) * N;
  const uint16_t* swave = reinterpret_cast<const uint16_t*>(a.s) + (size_t)(kbeg >> 6) * N;
  const uint8_t* zwave = a.z + (size_t)(kbeg >> 6) * N;
  uint32_t woff[8];
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int q = 0; q < 4; ++q) woff[4 * h + q] = (uint32_t)(16 * h + 4 * j + q) * N + (uint32_t)ncol;

  uint32_t rn[kQPF][8];
  u32x2 sn[kQPF];
  uint32_t zn[kQPF];
  auto load_group = [&](int g, uint32_t (&r)[8], u32x2& sv, uint32_t& zv) {
    const uint8_t* wg = wwave + (size_t)(32 * g) * N;
#pragma unroll
    for (int q = 0; q < 8; ++q) r[q] = *reinterpret_cast<const uint32_t*>(wg + woff[q]);
    sv = *reinterpret_cast<const u32x2*>(swave + (size_t)g * N + ncol);
    zv = *reinterpret_cast<const uint32_t*>(zwave + (size_t)g * N + ncol);
  };
#pragma unroll
  for (int p = 0; p < kQPF; ++p)
    if (p < ngroups) load_group(p, rn[p], sn[p], zn[p]);

  stage_x<true>(a, xl, lane, m0, mrows, kbeg);
  __syncthreads();

  const u32x4 ones = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};  // bf16 1.0
  f32x4 y[4];
#pragma unroll
  for (int w = 0; w < 4; ++w) y[w] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int g0 = 0; g0 < ngroups; g0 += kQPF) {
#pragma unroll
    for (int p = 0; p < kQPF; ++p) {
      const int g = g0 + p;
      if (g >= ngroups) break;
      uint32_t rc[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) rc[q] = rn[p][q];
      const u32x2 sv = sn[p];
      const uint32_t zv = zn[p];
      if (g + kQPF < ngroups) load_group(g + kQPF, rn[p], sn[p], zn[p]);

      f32x4 acc[4], xsum;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const u32x4 A = xl[((2 * g + h) * 4 + j) * 16 + c];
        uint32_t t[4];
        transpose4x4(rc[4 * h + 0], rc[4 * h + 1], rc[4 * h + 2], rc[4 * h + 3], t[0], t[1], t[2],
                     t[3]);
        const f32x4 zero4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int w = 0; w < 4; ++w) acc[w] = mfma16x16x32(A, unpack_int4(t[w]), h == 0 ? zero4 : acc[w]);
        // Row sums of x over the group (every column of this tile equal):
        // lane (c, j) gets sum_k x[4j + i][k] in element i.
        xsum = mfma16x16x32(A, ones, h == 0 ? zero4 : xsum);
      }
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const uint32_t sw = (w < 2) ? sv.x : sv.y;
        const float sf = bf16_to_f32((w & 1) ? (sw >> 16) : (sw & 0xFFFFu));
        const float zf = (float)((zv >> (8 * w)) & 0xFFu);
        const float cz = 128.f + zf;
        y[w] = sf * (acc[w] - cz * xsum) + y[w];
      }
    }
  }

  spill_y(wsm, y, c, j);
  reduce_and_store<NW, false>(a, smem, ksi, rb, m0, mrows, n0);
}

template <int NW>
__global__ __launch_bounds__(NW * kWave) void int8pc_gemv_kernel(QArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const uint32_t L = xcd_logical_id(blockIdx.x, gridDim.x);
  const int tile = (int)(L / (uint32_t)a.ks);
  const int ksi = (int)(L - (uint32_t)tile * a.ks);
  const int rb = blockIdx.y;
  const int m0 = rb * kQRows;
  const int mrows = min(kQRows, a.M - m0);
  const int n0 = tile * kQCols;
  const int c = lane & 15, j = lane >> 4;
  const int kbeg = ksi * (a.K / a.ks) + wv * a.kwave;
  const int ncol = min(n0 + 4 * c, a.N - 4);  // see int4g64_gemv_kernel
  const int nsteps = a.kwave >> 5;
  const uint32_t N = (uint32_t)a.N;

  unsigned char* wsm = smem + wv * a.wave_lds;
  u32x4* xl = reinterpret_cast<u32x4*>(wsm);

  // Lane rows: k = kbeg + 32*step + 8*j + r.
  const uint8_t* wwave = a.w + (size_t)kbeg * N;
  uint32_t woff[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) woff[q] = (uint32_t)(8 * j + q) * N + (uint32_t)ncol;

  uint32_t rn[kQPF][8];
  auto load_step = [&](int st, uint32_t (&r)[8]) {
    const uint8_t* ws = wwave + (size_t)(32 * st) * N;
#pragma unroll
    for (int q = 0; q < 8; ++q) r[q] = *reinterpret_cast<const uint32_t*>(ws + woff[q]);
  };
#pragma unroll
  for (int p = 0; p < kQPF; ++p)
    if (p < nsteps) load_step(p, rn[p]);

  stage_x<false>(a, xl, lane, m0, mrows, kbeg);
  __syncthreads();

  const u32x4 ones = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};  // bf16 1.0
  f32x4 y[4], xsum = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int w = 0; w < 4; ++w) y[w] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int s0 = 0; s0 < nsteps; s0 += kQPF) {
#pragma unroll
    for (int p = 0; p < kQPF; ++p) {
      const int st = s0 + p;
      if (st >= nsteps) break;
      uint32_t rc[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) rc[q] = rn[p][q];
      if (st + kQPF < nsteps) load_step(st + kQPF, rn[p]);
      const u32x4 A = xl[(st * 4 + j) * 16 + c];
      uint32_t lo[4], hi[4];
      transpose4x4(rc[0], rc[1], rc[2], rc[3], lo[0], lo[1], lo[2], lo[3]);
      transpose4x4(rc[4], rc[5], rc[6], rc[7], hi[0], hi[1], hi[2], hi[3]);
#pragma unroll
      for (int w = 0; w < 4; ++w) y[w] = mfma16x16x32(A, unpack_int8(lo[w], hi[w]), y[w]);
      xsum = mfma16x16x32(A, ones, xsum);
    }
  }
  // Remove the +128 offset: y -= 128 * sum_k x over this wave's K range.
#pragma unroll
  for (int w = 0; w < 4; ++w) y[w] = y[w] - 128.f * xsum;
  spill_y(wsm, y, c, j);
  reduce_and_store<NW, true>(a, smem, ksi, rb, m0, mrows, n0);
}

// ---------------------------------------------------------------------------
// Streaming kernels (N % 16 == 0, the workload shapes).
//
// Every operand goes global -> LDS by DMA (global_load_lds_dwordx4: 16 B per
// lane, written at M0 + 16 * lane, no VGPRs): per 32-k step one 1 KB block of
// x fragments and one (int4) or two (int8) 1 KB blocks of weights, through a
// ring of R steps per wave, plus the group scales / zero-points once.  A wave
// thus keeps R steps of weight bytes in flight from its first instructions,
// and since nothing is loaded into registers, every wait is explicit:
// s_waitcnt vmcnt(n) lets exactly the step about to be consumed complete.
// LDS reads are inline asm (ending in lgkmcnt(0)) because the compiler's
// wait-count pass cannot tell which DMA an LDS read depends on and would
// otherwise wait for the whole stream.  Their outputs are early-clobber
// ("=&v"): a load's destination must never share a register with an address
// that a later instruction of the same block still reads.
//
// Weight block = 16 W rows x 64 B.  DMA lane L = 16 r + 4 jj + kk loads row
// (4 jj + r), bytes [16 kk, 16 kk + 16) of the tile, so MFMA lane (c, j),
// which needs rows 4 j + r, bytes 4c..4c+3, reads dwords 64 r + 16 j + c:
// the 64 lanes of each read hit 64 distinct banks.  x block: DMA lane L
// loads MFMA lane L's own A fragment, read back as one contiguous 16 B.
// ---------------------------------------------------------------------------
// One step's LDS reads for MFMA lane (c, j): the 16 B A fragment at xaddr and
// the 4 weight row dwords of a block at waddr (dwords 0, 64, 128, 192).
__device__ __forceinline__ void read_step(uint32_t xaddr, uint32_t waddr, u32x4& A, uint32_t& r0,
                                          uint32_t& r1, uint32_t& r2, uint32_t& r3) {
  u32x2 p, q;
  asm volatile(
      "ds_read_b128 %0, %3\n\t"
      "ds_read2st64_b32 %1, %4 offset1:1\n\t"
      "ds_read2st64_b32 %2, %4 offset0:2 offset1:3\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(A), "=&v"(p), "=&v"(q)
      : "v"(xaddr), "v"(waddr)
      : "memory");
  r0 = p.x;
  r1 = p.y;
  r2 = q.x;
  r3 = q.y;
}

__device__ __forceinline__ void read_rows(uint32_t waddr, uint32_t& r0, uint32_t& r1, uint32_t& r2,
                                          uint32_t& r3) {
  u32x2 p, q;
  asm volatile(
      "ds_read2st64_b32 %0, %2 offset1:1\n\t"
      "ds_read2st64_b32 %1, %2 offset0:2 offset1:3\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(p), "=&v"(q)
      : "v"(waddr)
      : "memory");
  r0 = p.x;
  r1 = p.y;
  r2 = q.x;
  r3 = q.y;
}

__device__ __forceinline__ void read_scale_zero(uint32_t saddr, uint32_t zaddr, u32x2& sv, uint32_t& zv) {
  asm volatile(
      "ds_read_b64 %0, %2\n\t"
      "ds_read_b32 %1, %3\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(sv), "=&v"(zv)
      : "v"(saddr), "v"(zaddr)
      : "memory");
}

template <int S, int R>  // 32-k steps per wave; ring of R steps
__global__ __launch_bounds__(8 * kWave) void int4g64_stream_kernel(QArgs a) {
  constexpr int G = S / 2;
  static_assert(G <= 8 && R <= S, "scale / zero block holds 8 groups");
  extern __shared__ __align__(16) unsigned char smem[];
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const uint32_t L = xcd_logical_id(blockIdx.x, gridDim.x);
  const int tile = (int)(L / (uint32_t)a.ks);
  const int ksi = (int)(L - (uint32_t)tile * a.ks);
  const int rb = blockIdx.y;
  const int m0 = rb * kQRows;
  const int mrows = min(kQRows, a.M - m0);
  const int n0 = tile * kQCols;
  const int c = lane & 15, j = lane >> 4;
  const int kbeg = ksi * (a.K / a.ks) + wv * 32 * S;
  const size_t N = (size_t)a.N;
  // Wave LDS: [R] weight blocks | [R] x blocks | scales (1 KB) | zeros (1 KB).
  unsigned char* wl = smem + wv * a.wave_lds;
  unsigned char* wring = wl;
  unsigned char* xring = wl + R * 1024;
  unsigned char* sblk = wl + 2 * R * 1024;
  unsigned char* zblk = sblk + 1024;

  // Scales: group g row = 64 columns x 2 B = lanes 8g..8g+7; zero-points:
  // 64 B = lanes 4g..4g+3 (lanes 32..63 repeat 0..31).  Groups past G and
  // columns past N repeat valid ones (never consumed / never stored).
  {
    const int gs = min(lane >> 3, G - 1), gz = min((lane >> 2) & 7, G - 1);
    const uint16_t* sp = reinterpret_cast<const uint16_t*>(a.s) + (size_t)((kbeg >> 6) + gs) * N +
                         min(n0 + 8 * (lane & 7), a.N - 8);
    const uint8_t* zp = a.z + (size_t)((kbeg >> 6) + gz) * N + min(n0 + 16 * (lane & 3), a.N - 16);
    dma16(sp, sblk);
    dma16(zp, zblk);
  }
  // Step t: x fragment of MFMA lane (c, j) = lane; weight rows kp =
  // kbeg/2 + 16 t + 4 jj + r for DMA lane 16 r + 4 jj + kk.
  const uint16_t* xsrc = a.x + (size_t)min(m0 + c, a.M - 1) * a.K + kbeg + 8 * j;
  const int r = lane >> 4, jj = (lane >> 2) & 3, kk = lane & 3;
  const uint8_t* wsrc = a.w + (size_t)(kbeg / 2 + 4 * jj + r) * N + min(n0 + 16 * kk, a.N - 16);
  auto issue = [&](int t) {
    dma16(xsrc + 32 * t, xring + (t % R) * 1024);
    dma16(wsrc + (size_t)(16 * t) * N, wring + (t % R) * 1024);
  };
#pragma unroll
  for (int t = 0; t < R; ++t) issue(t);

  const uint32_t xaddr0 = lds_addr(xring) + 16 * lane;
  const uint32_t waddr0 = lds_addr(wring) + 4 * (16 * j + c);
  const uint32_t saddr0 = lds_addr(sblk) + 8 * c;
  const uint32_t zaddr0 = lds_addr(zblk) + 4 * c;
  const u32x4 ones = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};  // bf16 1.0
  const f32x4 zero4 = {0.f, 0.f, 0.f, 0.f};
  f32x4 y[4] = {zero4, zero4, zero4, zero4};
  f32x4 acc[4], xsum;
#pragma unroll
  for (int s = 0; s < S; ++s) {
    const int issued = (s + R < S) ? s + R : S;
    vm_wait(2 * (issued - 1 - s));
    u32x4 v;
    uint32_t r0, r1, r2, r3, t[4];
    read_step(xaddr0 + (s % R) * 1024, waddr0 + (s % R) * 1024, v, r0, r1, r2, r3);
    if (s + R < S) issue(s + R);  // this slot's reads have completed
    transpose4x4(r0, r1, r2, r3, t[0], t[1], t[2], t[3]);
    // x slot order k0 k2 k4 k6 k1 k3 k5 k7 (matches unpack_int4).
    const u32x4 A = {perm(v.y, v.x, 0x05040100u), perm(v.w, v.z, 0x05040100u),
                     perm(v.y, v.x, 0x07060302u), perm(v.w, v.z, 0x07060302u)};
    const bool first = (s & 1) == 0;
#pragma unroll
    for (int w = 0; w < 4; ++w) acc[w] = mfma16x16x32(A, unpack_int4(t[w]), first ? zero4 : acc[w]);
    xsum = mfma16x16x32(A, ones, first ? zero4 : xsum);
    if (!first) {
      const int g = s >> 1;
      u32x2 sv;
      uint32_t zv;
      read_scale_zero(saddr0 + 128 * g, zaddr0 + 64 * g, sv, zv);
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const uint32_t sw = (w < 2) ? sv.x : sv.y;
        const float sf = bf16_to_f32((w & 1) ? (sw >> 16) : (sw & 0xFFFFu));
        const float cz = 128.f + (float)((zv >> (8 * w)) & 0xFFu);
        y[w] = sf * (acc[w] - cz * xsum) + y[w];
      }
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  spill_y(wl, y, c, j);
  reduce_and_store<8, false>(a, smem, ksi, rb, m0, mrows, n0);
}

// ---------------------------------------------------------------------------
// Wide int4 kernel: 256 (or 128) output columns per workgroup.
//
// The 64-column kernel above streams 64-byte strips of every weight row and
// DMAs one 1 KB x slice per 1 KB of weights, so half of its L2->LDS traffic is
// re-reads of x.  Here a workgroup owns a tile of 256 columns (128 when N is
// not a multiple of 256) and K is split over `ks` workgroups to fill the
// chip.  Each wave covers TNW = 256 or 128 columns of the tile over its own G
// groups of 64 k (with the column split, waves w and w + 1 take the two
// 128-column halves of the same k range), with a private DMA ring of R 32-k
// steps: slot = 16 weight rows x TNW bytes, 16-column chunks swizzled so the
// transposing reads below are conflict-free.  ds_read_b64_tr_b8 hands MFMA
// lane (c, j) the bytes of column c of two column blocks in rows 4j..4j+3 of
// a step, i.e. its B fragments for two MFMAs; the bytes become bf16
// (128 + q) in registers as in the kernels above.  Scales and zero points
// come from tr16 / tr8 reads of the wave's scale block, x from two 16-byte
// reads of its x block; all three arrive by LDS DMA ahead of the ring.
//
// Split-K partials are combined in the kernel: every workgroup writes its
// f32 partial, waits for the stores' acknowledgement, and bumps the tile's
// arrival counter with an atomic; the last arriver sums all partials in k
// order (its own from registers, so results do not depend on arrival
// order), writes bf16 y and resets the counter.  No workgroup waits on
// another and no cache-wide fence is needed.  When the grid deals each
// tile's workgroups to one XCD (checked once per device by a probe) the
// exchange stays in that XCD's L2; otherwise it goes through device-coherent
// (sc1) stores and loads.
// ---------------------------------------------------------------------------
constexpr int kWideTN = 256;
constexpr int kWideSlot = 4 * 1024;   // one 32-k step: 16 weight rows x 256 B
constexpr int kWideRedStride = kWideTN + 4;  // padded f32 row of the y spill
constexpr int kWideCounters = 16384;  // counter slots at the start of the workspace
constexpr size_t kWidePartOffset = 64 * 1024;

// LDS position of weight chunk ch (16 columns) in slot row r:
// ch ^ (r & 7) ^ 8 (ch & 1).  A transposing read of the chunk pair (b, b+1),
// b even, then touches 16 distinct positions across rows 0..7 (conflict-free),
// and wide_pos(hi, r) is the lane constant K with position = b ^ K for
// chunk b + hi.
__device__ __forceinline__ int wide_pos(int hi, int r) { return hi ^ (r & 7) ^ (8 * hi); }
// Inverse: the chunk stored at position p of row r.
__device__ __forceinline__ int wide_chunk(int p, int r) {
  const int c0 = (p ^ r) & 1;
  return p ^ (r & 7) ^ (8 * c0);
}

// Eight transposing byte reads.
__device__ __forceinline__ void lds_tr8x8(const uint32_t (&ad)[8], u32x2 (&o)[8]) {
  asm volatile(
      "ds_read_b64_tr_b8 %0, %8\n\t"
      "ds_read_b64_tr_b8 %1, %9\n\t"
      "ds_read_b64_tr_b8 %2, %10\n\t"
      "ds_read_b64_tr_b8 %3, %11\n\t"
      "ds_read_b64_tr_b8 %4, %12\n\t"
      "ds_read_b64_tr_b8 %5, %13\n\t"
      "ds_read_b64_tr_b8 %6, %14\n\t"
      "ds_read_b64_tr_b8 %7, %15\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(o[0]), "=&v"(o[1]), "=&v"(o[2]), "=&v"(o[3]), "=&v"(o[4]), "=&v"(o[5]), "=&v"(o[6]),
        "=&v"(o[7])
      : "v"(ad[0]), "v"(ad[1]), "v"(ad[2]), "v"(ad[3]), "v"(ad[4]), "v"(ad[5]), "v"(ad[6]), "v"(ad[7])
      : "memory");
}

// Four transposing byte reads (the column split's 8 blocks) and their wait.
// One 16-byte LDS read and its wait.
__device__ __forceinline__ u32x4 lds_read_b128(uint32_t a0) {
  u32x4 v;
  asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=&v"(v) : "v"(a0) : "memory");
  return v;
}

// Two 16-byte LDS reads and their wait (x fragments of one 64-k group).
__device__ __forceinline__ void lds_read2_b128(uint32_t a0, uint32_t a1, u32x4& v0, u32x4& v1) {
  asm volatile(
      "ds_read_b128 %0, %2\n\t"
      "ds_read_b128 %1, %3\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(v0), "=&v"(v1)
      : "v"(a0), "v"(a1)
      : "memory");
}

__device__ __forceinline__ void lds_tr8x4(const uint32_t (&ad)[4], u32x2 (&o)[4]) {
  asm volatile(
      "ds_read_b64_tr_b8 %0, %4\n\t"
      "ds_read_b64_tr_b8 %1, %5\n\t"
      "ds_read_b64_tr_b8 %2, %6\n\t"
      "ds_read_b64_tr_b8 %3, %7\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(o[0]), "=&v"(o[1]), "=&v"(o[2]), "=&v"(o[3])
      : "v"(ad[0]), "v"(ad[1]), "v"(ad[2]), "v"(ad[3])
      : "memory");
}

// Scales and zero points of one group for 8 column blocks (2 tr16 reads, 1
// tr8 read): sv[0], sv[1] and zv[0] as lds_scale_zero fills them.
__device__ __forceinline__ void lds_scale_zero_half(uint32_t sa, uint32_t za, u32x2 (&sv)[4], u32x2 (&zv)[2]) {
  asm volatile(
      "ds_read_b64_tr_b16 %0, %3\n\t"
      "ds_read_b64_tr_b16 %1, %3 offset:128\n\t"
      "ds_read_b64_tr_b8 %2, %4\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(sv[0]), "=&v"(sv[1]), "=&v"(zv[0])
      : "v"(sa), "v"(za)
      : "memory");
  sv[2] = sv[0];
  sv[3] = sv[1];
  zv[1] = zv[0];
}

// Scales of one group for all 16 column blocks (4 tr16 reads: 4 blocks
// each) and its zero points (2 tr8 reads: 8 blocks each).
__device__ __forceinline__ void lds_scale_zero(uint32_t sa, uint32_t za, u32x2 (&sv)[4], u32x2 (&zv)[2]) {
  asm volatile(
      "ds_read_b64_tr_b16 %0, %6\n\t"
      "ds_read_b64_tr_b16 %1, %6 offset:128\n\t"
      "ds_read_b64_tr_b16 %2, %6 offset:256\n\t"
      "ds_read_b64_tr_b16 %3, %6 offset:384\n\t"
      "ds_read_b64_tr_b8 %4, %7\n\t"
      "ds_read_b64_tr_b8 %5, %7 offset:128\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(sv[0]), "=&v"(sv[1]), "=&v"(sv[2]), "=&v"(sv[3]), "=&v"(zv[0]), "=&v"(zv[1])
      : "v"(sa), "v"(za)
      : "memory");
}

// y quads of this thread = the KS split-K partials (this workgroup's among
// them, already acknowledged) summed in k order.
template <int NW, int KS, int TN = kWideTN>
__device__ __forceinline__ void wide_sum_partials(const float* tile_part, f32x4 (&own)[TN / 16 / NW]) {
  constexpr int IT = TN / 16 / NW;  // quads per thread: 16 rows x TN/4 quads over NW waves
  f32x4 v[IT][KS];
  const float* src[IT][KS];
#pragma unroll
  for (int it = 0; it < IT; ++it)
#pragma unroll
    for (int k2 = 0; k2 < KS; ++k2)
      src[it][k2] = tile_part + (size_t)k2 * kQRows * TN + 4 * (threadIdx.x + NW * kWave * it);
  if constexpr (KS == 2 && IT == 1) {
    ld2_sc1(src[0][0], src[0][1], v[0][0], v[0][1]);
  } else if constexpr (KS == 2) {
#pragma unroll
    for (int it = 0; it < IT; it += 2)
      ld4_sc1(src[it][0], src[it][1], src[it + 1][0], src[it + 1][1], v[it][0], v[it][1], v[it + 1][0],
              v[it + 1][1]);
  } else {
#pragma unroll
    for (int it = 0; it < IT; ++it)
#pragma unroll
      for (int k2 = 0; k2 < KS; k2 += 4)
        ld4_sc1(src[it][k2], src[it][k2 + 1], src[it][k2 + 2], src[it][k2 + 3], v[it][k2], v[it][k2 + 1],
                v[it][k2 + 2], v[it][k2 + 3]);
  }
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    f32x4 acc = v[it][0];
#pragma unroll
    for (int k2 = 1; k2 < KS; ++k2) acc += v[it][k2];
    own[it] = acc;
  }
}

#ifndef XCH_STORE_POLICY
#define XCH_STORE_POLICY kSc1
#endif
// The sum for the exchange inside one XCD's L2: loads served by the L2
// (first touch of these lines on this CU), through the tile's buffer
// resource `rs`, with this
// workgroup's own partial (split ksi) taken from registers: it was never
// stored.  The sum is the device-scope path's k-order sum, bit for bit.
template <int NW, int KS, int TN>
__device__ __forceinline__ void wide_sum_partials_l2_own(__amdgpu_buffer_rsrc_t rs, int ksi,
                                                         f32x4 (&own)[TN / 16 / NW]) {
  constexpr int IT = TN / 16 / NW;
  // v[it][i]: split i + (i >= ksi), every load in flight together (no
  // branches between them).
  u32x4 v[IT][KS - 1];
#pragma unroll
  for (int it = 0; it < IT; ++it)
#pragma unroll
    for (int i = 0; i < KS - 1; ++i)
      v[it][i] = __builtin_amdgcn_raw_buffer_load_b128(
          rs, ((i + (i >= ksi)) * kQRows * TN + 4 * (threadIdx.x + NW * kWave * it)) * 4, 0, kSc0);
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    f32x4 p[KS];
#pragma unroll
    for (int k2 = 0; k2 < KS; ++k2) {
      const f32x4 below = __builtin_bit_cast(f32x4, v[it][k2 < KS - 1 ? k2 : KS - 2]);
      const f32x4 above = __builtin_bit_cast(f32x4, v[it][k2 > 0 ? k2 - 1 : 0]);
      p[k2] = k2 < ksi ? below : (k2 == ksi ? own[it] : above);
    }
    f32x4 acc = p[0];
#pragma unroll
    for (int k2 = 1; k2 < KS; ++k2) acc += p[k2];
    own[it] = acc;
  }
}


// The end of both wide kernels.  Sum the 8 waves' y tiles through LDS;
// with ks > 1 combine the split-K partials across workgroups (the last of a
// tile's workgroups to arrive sums them in k order); store bf16 y, times the
// int8 per-channel scale when FMT8.  Every DMA of the calling wave must have
// landed: y is spilled into its own LDS region, over its ring.
// CS = 1: every wave holds all TN columns of its k range.  CS = 2: wave w
// holds columns [128 (w % 2), +128) of its k range (NB = 8 blocks), and each
// output column sums the NW / 2 waves of its half.  TN: the tile's columns
// (256, or 128 for the narrow tiles, whose waves all hold the whole tile).
template <int NW, bool FMT8, int CS = 1, int TN = kWideTN>
__device__ __forceinline__ void wide_finish(const QArgs& a, unsigned char* smem, unsigned char* wl,
                                            const f32x4 (&y)[TN / 16 / CS], int tile, int ksi, int rb, int m0,
                                            int mrows, int n0, int c, int j) {
  constexpr int NB = TN / 16 / CS, QPR = TN / 4;  // y blocks per wave; output quads per row
  constexpr int RS = TN + 4;                      // padded f32 row of the y spill
  constexpr int IT = 16 * QPR / (NW * kWave);     // output quads per thread
  const size_t N = (size_t)a.N;
  const f32x4 zero4 = {0.f, 0.f, 0.f, 0.f};
  // FMT8: the per-channel scales of this thread's output quads, loaded now
  // so that their latency hides under the wave sum and the exchange instead
  // of following the last arriver's partial loads (int8 headline shape
  // 16.52-16.72 -> 16.19-16.27 us).
  f32x4 scl[FMT8 ? IT : 1];
  if constexpr (FMT8) {
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      const int q = threadIdx.x + NW * kWave * it;
      scl[it] = *reinterpret_cast<const f32x4*>(static_cast<const float*>(a.s) + n0 + 4 * (q % QPR));
    }
  }
  // Sum the waves: each spills y as [16 m][TN] f32 (padded rows; its own
  // columns only) into its own region; lane (c, j) holds column
  // col0 + 16b + c, rows 4j..4j+3.
  float* red = reinterpret_cast<float*>(wl);
  const int col0 = CS == 1 ? 0 : (TN / CS) * ((threadIdx.x >> 6) % CS);
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int i = 0; i < 4; ++i) red[(4 * j + i) * RS + col0 + 16 * b + c] = y[b][i];
  __syncthreads();
  f32x4 own[IT];
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    const int q = threadIdx.x + NW * kWave * it;  // quad index: 16 rows x QPR quads
    const int m = q / QPR, n = 4 * (q % QPR);
    const int wh = CS == 1 ? 0 : n / (TN / CS);  // the waves holding column n: wh, wh + CS, ...
    f32x4 acc = zero4;
#pragma unroll
    for (int w = 0; w < NW / CS; ++w)
      acc += *reinterpret_cast<const f32x4*>(smem + (CS * w + wh) * a.wave_lds + (m * RS + n) * 4);
    own[it] = acc;
  }
  const int ntiles = a.N / TN;
  uint32_t* ctr = a.cnt + rb * ntiles + tile;
  asm volatile("" : "+v"(ctr));  // per-lane address: a vector atomic
  if (a.ks > 1 && a.xch_local) {
    // Every workgroup of this tile runs on this XCD (the host checked that
    // the grid deals each tile's ks workgroups to one XCD), so the exchange
    // stays in its L2: stores acknowledged by the L2, a workgroup-scope
    // atomic (performed in the L2), and loads the L2 serves (the CU's L1
    // holds no line of the tile's partials: it starts the kernel
    // invalidated, and only the tile's last arriver loads them, once).  The
    // ordering argument is the device-scope one below with the L2 as the
    // common coherence point; the last arriver takes its own partial from
    // registers.
    const size_t tbase = ((size_t)(rb * ntiles + tile) * a.ks) * kQRows * TN;
    float* tp = a.part + tbase;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(tp, 0, a.ks * kQRows * TN * 4, kBufWord3);
#pragma unroll
    for (int it = 0; it < IT; ++it)
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, own[it]), rs,
                                             (ksi * kQRows * TN + 4 * (threadIdx.x + NW * kWave * it)) * 4, 0,
                                             XCH_STORE_POLICY);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // every partial store acknowledged
    __syncthreads();  // (also: every wave is done reading the spills)
    volatile uint32_t* flag = reinterpret_cast<volatile uint32_t*>(smem);
    if (threadIdx.x == 0) {
      const uint32_t old = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      const uint32_t last = old == (uint32_t)(a.ks - 1);
      if (last) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      *flag = last;
    }
    __syncthreads();
    if (!*flag) return;
    switch (a.ks) {
      case 2: wide_sum_partials_l2_own<NW, 2, TN>(rs, ksi, own); break;
      case 4: wide_sum_partials_l2_own<NW, 4, TN>(rs, ksi, own); break;
      default: wide_sum_partials_l2_own<NW, 8, TN>(rs, ksi, own); break;
    }
  } else if (a.ks > 1) {
    const size_t tbase = ((size_t)(rb * ntiles + tile) * a.ks) * kQRows * TN;
    // Device-coherent stores of the partial, acknowledged.
    float* dst = a.part + tbase + (size_t)ksi * kQRows * TN + 4 * threadIdx.x;
    if constexpr (IT == 1) {
      st1_sc1_wait(dst, own[0]);
    } else {
#pragma unroll
      for (int it = 0; it < IT; it += 2)
        st2_sc1_wait(dst + 4 * NW * kWave * it, own[it], dst + 4 * NW * kWave * (it + 1), own[it + 1]);
    }
    __syncthreads();  // (also: every wave is done reading the spills)
    // The flag lives in dynamic LDS: a static __shared__ would shift the
    // dynamic base off the 256-byte alignment the swizzled addressing needs.
    volatile uint32_t* flag = reinterpret_cast<volatile uint32_t*>(smem);
    if (threadIdx.x == 0) {
      const uint32_t old = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const uint32_t last = old == (uint32_t)(a.ks - 1);
      if (last) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      *flag = last;
    }
    __syncthreads();
    if (!*flag) return;
    // Device-coherent 16-byte loads (sc1: miss the local L2) of every
    // partial, then the sum in k order.
    switch (a.ks) {
      case 2: wide_sum_partials<NW, 2, TN>(a.part + tbase, own); break;
      case 4: wide_sum_partials<NW, 4, TN>(a.part + tbase, own); break;
      default: wide_sum_partials<NW, 8, TN>(a.part + tbase, own); break;
    }
  }
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    const int q = threadIdx.x + NW * kWave * it;
    const int m = q / QPR, n = n0 + 4 * (q % QPR);
    if (m >= mrows) continue;
    if constexpr (FMT8) own[it] *= scl[it];
    epi_store_bf16x4(a.y, a.aux, a.epi, (size_t)(m0 + m) * N + n, own[it]);
  }
}

// Column split CS = 2: 128-byte slot rows (8 chunks), chunk ch of slot row r
// at position ch ^ (r & 2).  The transposing read of chunk pair (b, b+1),
// b even, takes rows 4j .. 4j+3: rows 4j, 4j+2 put the pair at positions
// {b, b+1} and {b^2, b^3} and rows 4j+1, 4j+3 lie 128 bytes further (the
// other half of the 64 banks), so a 16-lane group touches 16 distinct
// 8-byte bank pairs.
__device__ __forceinline__ int wide2_swz(int r) { return r & 2; }

// NW waves; G 64-k groups per wave; ring of R 32-k steps; column split CS;
// tile of TN columns (TNW = TN / CS per wave: 256 or 128).
template <int NW, int G, int R, int CS, int TN = kWideTN>
__global__ __launch_bounds__(NW * kWave) void int4g64_wide_kernel(QArgs a) {
  constexpr int TNW = TN / CS, NB = TNW / 16, S = 2 * G;
  constexpr int DPS = TNW / 64;                             // weight DMAs per step
  constexpr int SLOT = 16 * TNW;                            // one 32-k step: 16 weight rows x TNW bytes
  constexpr int LPR = TNW / 16, RPD = 64 / LPR;             // DMA lanes per slot row, slot rows per DMA
  constexpr int SB = ((G * TNW * 2 + 1023) / 1024) * 1024;  // scale block bytes
  constexpr int ZB = ((G * TNW + 1023) / 1024) * 1024;      // zero-point block bytes
  constexpr int XB = G * 2048;                              // x block bytes: [G][16 rows][64 k] bf16
  static_assert((CS == 1 || CS == 2) && (TNW == 256 || TNW == 128), "128 or 256 columns per wave");
  static_assert(R >= 2 && R <= S && G <= 4, "ring holds both steps of a group");
  extern __shared__ __align__(16) unsigned char smem[];
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  // Column split: the second wave of each SIMD (wv >= NW / 2) issues its
  // first loads at a raised priority (dropped after them).  Without it those
  // waves start their streams 0.6 us after the first four and end their K
  // loop 1 us later; the age-ordered issue of the K loop then favours the
  // first four, which evens them out (headline shape 11.31 -> 11.05 us on
  // one box, 11.35-11.44 -> 11.16-11.28 on another, same bits; the
  // 128-column tiles measured 0.8 % slower with it).
  constexpr bool PR = CS == 2;
  if (PR && __builtin_amdgcn_readfirstlane(wv) >= NW / 2) __builtin_amdgcn_s_setprio(1);
  const uint32_t L = xcd_logical_id(blockIdx.x, gridDim.x);
  const int tile = (int)(L / (uint32_t)a.ks);
  const int ksi = (int)(L - (uint32_t)tile * a.ks);
  const int rb = blockIdx.y;
  const int m0 = rb * kQRows;
  const int mrows = min(kQRows, a.M - m0);
  const int n0 = tile * TN;
  const int c = lane & 15, j = lane >> 4;
  // wave wv: columns [TNW (wv % CS), +TNW) of the tile, k part wv / CS
  const int n0w = n0 + TNW * (wv % CS);
  const int kbeg = ksi * (a.K / a.ks) + (wv / CS) * 64 * G;
  const size_t N = (size_t)a.N;
  unsigned char* wl = smem + wv * a.wave_lds;
  unsigned char* ring = wl;
  unsigned char* sblk = wl + R * SLOT;
  unsigned char* zblk = sblk + SB;
  unsigned char* xblk = zblk + ZB;

  // k order inside each 64-k group g: MFMA lane group j, half h (of the two
  // MFMAs) covers k = kbeg + 64 g + 16 j + 8 h .. +7, so a lane's x for a
  // group is 16 contiguous bf16 and a row of x is read as whole lines.  x
  // comes by LDS DMA like everything else the wave streams (issued first),
  // so every load of the wave is one kind and the ring's counted waits
  // cover it: block [G][16 rows][8 chunks of 16 B], chunk q of row r at
  // position q ^ (r & 7), which makes the two 16-byte reads per lane below
  // conflict-free.  Rows past M repeat row M - 1 (never stored).
  {
    const int r = lane >> 3, q = (lane & 7) ^ (lane >> 3);
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int hb = 0; hb < 2; ++hb)
        dma16(a.x + (size_t)min(m0 + r + 8 * hb, a.M - 1) * a.K + kbeg + 64 * g + 8 * q,
              xblk + g * 2048 + hb * 1024);
  }
  const uint32_t xoff = lds_addr(xblk) + (uint32_t)(c * 128);
  const uint32_t xlo = 16u * (uint32_t)((2 * j) ^ (c & 7)), xhi = 16u * (uint32_t)((2 * j + 1) ^ (c & 7));
  // Scale rows [G][TN] bf16 and zero rows [G][TN] u8 of this wave's groups
  // (rows past G repeat the last one; never used).
#pragma unroll
  for (int q = 0; q < SB / 1024; ++q) {
    const int b = q * 1024 + 16 * lane;
    const int g = min(b / (2 * TNW), G - 1), col = (b % (2 * TNW)) / 2;
    dma16(reinterpret_cast<const uint16_t*>(a.s) + (size_t)((kbeg >> 6) + g) * N + n0w + col, sblk + q * 1024);
  }
#pragma unroll
  for (int q = 0; q < ZB / 1024; ++q) {
    const int b = q * 1024 + 16 * lane;
    const int g = min(b / TNW, G - 1), col = b % TNW;
    dma16(a.z + (size_t)((kbeg >> 6) + g) * N + n0w + col, zblk + q * 1024);
  }

  // Step t = 2g + h: weight DMA q lane L fills slot row rr = RPD q + L/LPR,
  // chunk position p = L % LPR, from W row kbeg/2 + 32 g + 4 h + 8 (rr/4)
  // + rr%4 (slot rows 4j .. 4j+3 are MFMA lane group j's) at the global
  // chunk stored in position p of row rr.
  const uint8_t* wsrc[DPS];
#pragma unroll
  for (int q = 0; q < DPS; ++q) {
    const int rr = RPD * q + lane / LPR, pp = lane % LPR;
    const int ch = TNW == 256 ? wide_chunk(pp, rr) : (pp ^ wide2_swz(rr));
    wsrc[q] = a.w + (size_t)(kbeg / 2 + 8 * (rr >> 2) + (rr & 3)) * N + n0w + 16 * ch;
  }
  auto issue = [&](int t) {
    unsigned char* slot = ring + (t % R) * SLOT;
    const int g = t >> 1, h = t & 1;
#pragma unroll
    for (int q = 0; q < DPS; ++q) dma16(wsrc[q] + (size_t)(32 * g + 4 * h) * N, slot + q * 1024);
  };
#pragma unroll
  for (int t = 0; t < R; ++t) issue(t);
  if (PR) __builtin_amdgcn_s_setprio(0);

  // Per-lane LDS offsets.  Transposing weight read of lane (c, j) for the
  // column-block pair (b, b+1), b even: lane pair (2r, 2r+1) of each 16-lane
  // group names the two 8-byte halves of row r; rows r < 4 are slot row
  // 4j + r at chunk b, rows r >= 4 slot row 4j + r - 4 at chunk b + 1.  The
  // chunk position is then b ^ (a lane constant), so the address of pair b
  // is wbase ^ (16 b).
  const int r8 = (lane & 15) >> 1, hi = r8 >> 2;
  const int wrow = 4 * j + (r8 & 3);
  const uint32_t woff =
      (uint32_t)(wrow * TNW + 8 * (lane & 1) + 16 * (TNW == 256 ? wide_pos(hi, wrow) : (hi ^ wide2_swz(wrow))));
  const uint32_t ring0 = lds_addr(ring);
  // Scale tr16 read: lane 4r + q of a group names row (block) r, columns 4q..4q+3.
  const uint32_t soff = lds_addr(sblk) + (uint32_t)(((lane & 15) >> 2) * 32 + 8 * (lane & 3));
  const uint32_t zoff = lds_addr(zblk) + (uint32_t)(r8 * 16 + 8 * (lane & 1));

  const u32x4 ones = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};  // bf16 1.0
  const f32x4 zero4 = {0.f, 0.f, 0.f, 0.f};
  f32x4 y[NB], acc[NB], xs;
  u32x4 xg[2];
#pragma unroll
  for (int b = 0; b < NB; ++b) y[b] = zero4;

#pragma unroll
  for (int t = 0; t < S; ++t) {
    const int g = t >> 1, h = t & 1;
    const int issued = (R + t < S) ? R + t : S;  // steps issued before this wait
    vm_wait(DPS * (issued - (t + 1)));
    const uint32_t wb = ring0 + (uint32_t)((t % R) * SLOT) + woff;
    u32x2 w2[NB / 2];
    {
      uint32_t ad[NB / 2];
#pragma unroll
      for (int p = 0; p < NB / 2; ++p) ad[p] = wb ^ (uint32_t)(32 * p);
      if constexpr (TNW == 256) lds_tr8x8(ad, w2);
      else lds_tr8x4(ad, w2);
    }
    // This step's slot is read: refill it.
    if (t + R < S) issue(t + R);

    // x slot order k0 k2 k4 k6 k1 k3 k5 k7 (matches unpack_int4).
    if (h == 0) lds_read2_b128(xoff + (uint32_t)(g * 2048) + xlo, xoff + (uint32_t)(g * 2048) + xhi, xg[0], xg[1]);
    const u32x4 v = xg[h];
    const u32x4 A = {perm(v.y, v.x, 0x05040100u), perm(v.w, v.z, 0x05040100u), perm(v.y, v.x, 0x07060302u),
                     perm(v.w, v.z, 0x07060302u)};
    xs = mfma16x16x32(A, ones, h ? xs : zero4);
#pragma unroll
    for (int b = 0; b < NB; ++b)
      acc[b] = mfma16x16x32(A, unpack_int4((b & 1) ? w2[b >> 1].y : w2[b >> 1].x), h ? acc[b] : zero4);
    if (h) {
      u32x2 sv[4], zv[2];
      if constexpr (TNW == 256) lds_scale_zero(soff + (uint32_t)(g * 2 * TNW), zoff + (uint32_t)(g * TNW), sv, zv);
      else lds_scale_zero_half(soff + (uint32_t)(g * 2 * TNW), zoff + (uint32_t)(g * TNW), sv, zv);
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const uint32_t sw = (b & 2) ? sv[b >> 2].y : sv[b >> 2].x;
        const float sf = __uint_as_float((b & 1) ? (sw & 0xFFFF0000u) : (sw << 16));
        const uint32_t zw = (b & 4) ? zv[b >> 3].y : zv[b >> 3].x;
        const float cz = 128.f + (float)((zw >> (8 * (b & 3))) & 0xFFu);
#pragma unroll
        for (int i = 0; i < 4; ++i) y[b][i] = fmaf(sf, fmaf(-cz, xs[i], acc[b][i]), y[b][i]);
      }
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  wide_finish<NW, false, CS, TN>(a, smem, wl, y, tile, ksi, rb, m0, mrows, n0, c, j);
}

// ---------------------------------------------------------------------------
// Wide int8 kernel: the wide int4 kernel's layout for per-channel int8
// weights.  The 64-column streaming kernel reads 64-byte strips of every
// weight row, which HBM serves at about half the rate of 256-byte segments;
// here a workgroup owns 256 output columns and K is split over `ks`
// workgroups.  Each of the 8 waves covers all 256 columns over its own S
// steps of 32 k with a private DMA ring of R steps: slot = 32 weight rows x
// 256 B, 16-column chunk c of row r at position c ^ (r & 15), so a
// transposing read of one chunk across 16 consecutive rows touches 16
// distinct positions (conflict-free).  ds_read_b64_tr_b8 hands MFMA lane
// (c, j) column c of one column block in rows 8j..8j+7 -- its B fragment of
// that block, in natural k order.  Bytes become bf16 (w + 128) as in the
// 64-column kernel; the offset is removed with the x row sums and the
// per-channel scale is applied at the store.
// ---------------------------------------------------------------------------
constexpr int kWide8Slot = 8 * 1024;  // one 32-k step: 32 weight rows x 256 B

// Sixteen transposing byte reads (one per column block) and their wait.
__device__ __forceinline__ void lds_tr8x16(uint32_t wb, u32x2 (&o)[16]) {
  asm volatile(
      "ds_read_b64_tr_b8 %0, %16\n\t"
      "ds_read_b64_tr_b8 %1, %17\n\t"
      "ds_read_b64_tr_b8 %2, %18\n\t"
      "ds_read_b64_tr_b8 %3, %19\n\t"
      "ds_read_b64_tr_b8 %4, %20\n\t"
      "ds_read_b64_tr_b8 %5, %21\n\t"
      "ds_read_b64_tr_b8 %6, %22\n\t"
      "ds_read_b64_tr_b8 %7, %23\n\t"
      "ds_read_b64_tr_b8 %8, %24\n\t"
      "ds_read_b64_tr_b8 %9, %25\n\t"
      "ds_read_b64_tr_b8 %10, %26\n\t"
      "ds_read_b64_tr_b8 %11, %27\n\t"
      "ds_read_b64_tr_b8 %12, %28\n\t"
      "ds_read_b64_tr_b8 %13, %29\n\t"
      "ds_read_b64_tr_b8 %14, %30\n\t"
      "ds_read_b64_tr_b8 %15, %31\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(o[0]), "=&v"(o[1]), "=&v"(o[2]), "=&v"(o[3]), "=&v"(o[4]), "=&v"(o[5]), "=&v"(o[6]),
        "=&v"(o[7]), "=&v"(o[8]), "=&v"(o[9]), "=&v"(o[10]), "=&v"(o[11]), "=&v"(o[12]), "=&v"(o[13]),
        "=&v"(o[14]), "=&v"(o[15])
      : "v"(wb), "v"(wb ^ 16u), "v"(wb ^ 32u), "v"(wb ^ 48u), "v"(wb ^ 64u), "v"(wb ^ 80u), "v"(wb ^ 96u),
        "v"(wb ^ 112u), "v"(wb ^ 128u), "v"(wb ^ 144u), "v"(wb ^ 160u), "v"(wb ^ 176u), "v"(wb ^ 192u),
        "v"(wb ^ 208u), "v"(wb ^ 224u), "v"(wb ^ 240u)
      : "memory");
}

// Eight transposing byte reads (the column-split waves' 128-column slots).
__device__ __forceinline__ void lds_tr8x8(uint32_t wb, u32x2 (&o)[8]) {
  asm volatile(
      "ds_read_b64_tr_b8 %0, %8\n\t"
      "ds_read_b64_tr_b8 %1, %9\n\t"
      "ds_read_b64_tr_b8 %2, %10\n\t"
      "ds_read_b64_tr_b8 %3, %11\n\t"
      "ds_read_b64_tr_b8 %4, %12\n\t"
      "ds_read_b64_tr_b8 %5, %13\n\t"
      "ds_read_b64_tr_b8 %6, %14\n\t"
      "ds_read_b64_tr_b8 %7, %15\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(o[0]), "=&v"(o[1]), "=&v"(o[2]), "=&v"(o[3]), "=&v"(o[4]), "=&v"(o[5]), "=&v"(o[6]), "=&v"(o[7])
      : "v"(wb), "v"(wb ^ 16u), "v"(wb ^ 32u), "v"(wb ^ 48u), "v"(wb ^ 64u), "v"(wb ^ 80u), "v"(wb ^ 96u),
        "v"(wb ^ 112u)
      : "memory");
}

// CS = 2 (column split, as in the wide int4 kernel): wave w covers columns
// [128 (w % 2), +128) of the tile over twice the k steps; a slot row is then
// 128 B and chunk c of row r sits at position c ^ ((r / 2) % 8), which keeps
// one transposing read (8 rows per 16-lane group, 32 rows per wave) on
// distinct 16-byte bank groups.
template <int S, int R, int CS = 1>  // 32-k steps per wave; ring of R steps; column split
__global__ __launch_bounds__(8 * kWave) void int8pc_wide_kernel(QArgs a) {
  constexpr int TN = kWideTN, TNW = TN / CS, NB = TNW / 16;
  constexpr int SLOT = 32 * TNW;          // one 32-k step: 32 weight rows x TNW bytes
  constexpr int DPS = SLOT / 1024;        // weight DMAs per step
  static_assert(CS == 1 || CS == 2, "256 or 128 columns per wave");
  static_assert(R >= 1 && R <= S, "ring of at most S steps");
  extern __shared__ __align__(16) unsigned char smem[];
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  // Waves 4-7 issue their first loads at a raised priority, as in the int4
  // kernel (M = 16, K = 4096: N = 14336 16.68-16.71 -> 16.52-16.68 us, N =
  // 8192 9.59-9.64 -> 9.53-9.56 us; same bits).
  if (__builtin_amdgcn_readfirstlane(wv) >= 4) __builtin_amdgcn_s_setprio(1);
  const uint32_t L = xcd_logical_id(blockIdx.x, gridDim.x);
  const int tile = (int)(L / (uint32_t)a.ks);
  const int ksi = (int)(L - (uint32_t)tile * a.ks);
  const int rb = blockIdx.y;
  const int m0 = rb * kQRows;
  const int mrows = min(kQRows, a.M - m0);
  const int n0 = tile * TN;
  const int c = lane & 15, j = lane >> 4;
  const int kbeg = ksi * (a.K / a.ks) + (wv / CS) * 32 * S;
  const int n0w = n0 + TNW * (wv % CS);
  const size_t N = (size_t)a.N;
  unsigned char* wl = smem + wv * a.wave_lds;

  // x of every step, issued first: lane (c, j) uses x[m0 + c][kbeg + 32 t +
  // 8 j .. +7], its A fragment of step t.  With S <= 4 it comes by LDS DMA
  // like the weights (every load of the wave one kind, so the ring's counted
  // waits cover it; with register loads in flight beside LDS DMAs the
  // compiler waits for all of them before the first step): block
  // [S][16 rows][4 chunks of 16 B], chunk q of row r at position
  // q ^ ((r >> 2) & 3), which makes the 16-byte reads conflict-free.  Longer
  // waves keep it in registers (the LDS would not hold it).
  constexpr bool XL = CS == 1 ? S <= 4 : S <= 8;
  unsigned char* xblk = wl + R * SLOT;
  u32x4 xr[XL ? 1 : S];
  if constexpr (XL) {
    const int r = lane >> 2, q = (lane & 3) ^ ((lane >> 4) & 3);
#pragma unroll
    for (int t = 0; t < S; ++t)
      dma16(a.x + (size_t)min(m0 + r, a.M - 1) * a.K + kbeg + 32 * t + 8 * q, xblk + t * 1024);
  } else {
    const uint16_t* xp = a.x + (size_t)min(m0 + c, a.M - 1) * a.K + kbeg + 8 * j;
#pragma unroll
    for (int t = 0; t < S; ++t) xr[t] = *reinterpret_cast<const u32x4*>(xp + 32 * t);
  }
  const uint32_t xa = lds_addr(xblk) + (uint32_t)(c * 64 + 16 * (j ^ ((c >> 2) & 3)));
  // Step t, DMA q: lane L fills slot row rr = 4 q + L / 16 (W row
  // kbeg + 32 t + rr), position L % 16, from chunk (L % 16) ^ (rr & 15);
  // with 128-byte rows, row 8 q + L / 8, position L % 8, from chunk
  // (L % 8) ^ ((rr / 2) % 8).
  const uint8_t* wsrc[DPS];
#pragma unroll
  for (int q = 0; q < DPS; ++q) {
    if constexpr (CS == 1) {
      const int rr = 4 * q + (lane >> 4);
      wsrc[q] = a.w + (size_t)(kbeg + rr) * N + n0w + 16 * ((lane & 15) ^ (rr & 15));
    } else {
      const int rr = 8 * q + (lane >> 3);
      wsrc[q] = a.w + (size_t)(kbeg + rr) * N + n0w + 16 * ((lane & 7) ^ ((rr >> 1) & 7));
    }
  }
  auto issue = [&](int t) {
    unsigned char* slot = wl + (t % R) * SLOT;
#pragma unroll
    for (int q = 0; q < DPS; ++q) dma16(wsrc[q] + (size_t)(32 * t) * N, slot + q * 1024);
  };
#pragma unroll
  for (int t = 0; t < R; ++t) issue(t);
  __builtin_amdgcn_s_setprio(0);

  // Transposing read of lane (c, j): lane pair (2r, 2r + 1) of the 16-lane
  // group names the two 8-byte halves of chunk b in slot row 8 j + r, at
  // position b ^ (row & 15): the address of block b is wb ^ (16 b).
  const int wrow = 8 * j + ((lane & 15) >> 1);
  const uint32_t woff = CS == 1 ? (uint32_t)(wrow * TNW + 16 * (wrow & 15) + 8 * (lane & 1))
                                : (uint32_t)(wrow * TNW + 16 * ((wrow >> 1) & 7) + 8 * (lane & 1));
  const uint32_t ring0 = lds_addr(wl);

  const u32x4 ones = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};  // bf16 1.0
  const f32x4 zero4 = {0.f, 0.f, 0.f, 0.f};
  f32x4 acc[NB], xs = zero4;
#pragma unroll
  for (int b = 0; b < NB; ++b) acc[b] = zero4;
#pragma unroll
  for (int t = 0; t < S; ++t) {
    const int issued = (R + t < S) ? R + t : S;  // steps issued before this wait
    vm_wait(DPS * (issued - (t + 1)));
    u32x2 w8[NB];
    if constexpr (CS == 1) lds_tr8x16(ring0 + (uint32_t)((t % R) * SLOT) + woff, w8);
    else lds_tr8x8(ring0 + (uint32_t)((t % R) * SLOT) + woff, w8);
    // This step's slot is read: refill it.
    if (t + R < S) issue(t + R);
    u32x4 A;
    if constexpr (XL) A = lds_read_b128(xa + (uint32_t)(t * 1024));
    else A = xr[t];
    xs = mfma16x16x32(A, ones, xs);
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[b] = mfma16x16x32(A, unpack_int8(w8[b].x, w8[b].y), acc[b]);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  f32x4 y[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) y[b] = acc[b] - 128.f * xs;
  wide_finish<8, true, CS>(a, smem, wl, y, tile, ksi, rb, m0, mrows, n0, c, j);
}

template <int S, int R>  // 32-k steps per wave, ring of R steps (3 KB each)
__global__ __launch_bounds__(8 * kWave) void int8pc_stream_kernel(QArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const uint32_t L = xcd_logical_id(blockIdx.x, gridDim.x);
  const int tile = (int)(L / (uint32_t)a.ks);
  const int ksi = (int)(L - (uint32_t)tile * a.ks);
  const int rb = blockIdx.y;
  const int m0 = rb * kQRows;
  const int mrows = min(kQRows, a.M - m0);
  const int n0 = tile * kQCols;
  const int c = lane & 15, j = lane >> 4;
  const int kbeg = ksi * (a.K / a.ks) + wv * 32 * S;
  const size_t N = (size_t)a.N;
  // Wave LDS: [R] x (weight block h = 0, weight block h = 1, x block).
  unsigned char* wl = smem + wv * a.wave_lds;

  // Step t: weight rows kbeg + 32 t + 8 jj + 4 h + r in block h (DMA lane
  // 16 r + 4 jj + kk), x fragment of MFMA lane (c, j) = lane.
  const uint16_t* xsrc = a.x + (size_t)min(m0 + c, a.M - 1) * a.K + kbeg + 8 * j;
  const int r = lane >> 4, jj = (lane >> 2) & 3, kk = lane & 3;
  const uint8_t* wsrc = a.w + (size_t)(kbeg + 8 * jj + r) * N + min(n0 + 16 * kk, a.N - 16);
  auto issue = [&](int t) {
    unsigned char* dst = wl + (t % R) * 3072;
    dma16(wsrc + (size_t)(32 * t) * N, dst);
    dma16(wsrc + (size_t)(32 * t + 4) * N, dst + 1024);
    dma16(xsrc + 32 * t, dst + 2048);
  };
#pragma unroll
  for (int t = 0; t < R; ++t) issue(t);

  const uint32_t base = lds_addr(wl);
  const uint32_t waddr0 = base + 4 * (16 * j + c);
  const uint32_t xaddr0 = base + 2048 + 16 * lane;
  const u32x4 ones = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};  // bf16 1.0
  const f32x4 zero4 = {0.f, 0.f, 0.f, 0.f};
  f32x4 y[4] = {zero4, zero4, zero4, zero4};
  f32x4 xsum = zero4;
#pragma unroll
  for (int s = 0; s < S; ++s) {
    const int issued = (s + R < S) ? s + R : S;
    vm_wait(3 * (issued - 1 - s));
    u32x4 A;
    uint32_t q[8], lo[4], hi[4];
    read_step(xaddr0 + (s % R) * 3072, waddr0 + (s % R) * 3072, A, q[0], q[1], q[2], q[3]);
    read_rows(waddr0 + (s % R) * 3072 + 1024, q[4], q[5], q[6], q[7]);
    if (s + R < S) issue(s + R);  // this slot's reads have completed
    transpose4x4(q[0], q[1], q[2], q[3], lo[0], lo[1], lo[2], lo[3]);
    transpose4x4(q[4], q[5], q[6], q[7], hi[0], hi[1], hi[2], hi[3]);
#pragma unroll
    for (int w = 0; w < 4; ++w) y[w] = mfma16x16x32(A, unpack_int8(lo[w], hi[w]), y[w]);
    xsum = mfma16x16x32(A, ones, xsum);
  }
#pragma unroll
  for (int w = 0; w < 4; ++w) y[w] = y[w] - 128.f * xsum;
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  spill_y(wl, y, c, j);
  reduce_and_store<8, true>(a, smem, ksi, rb, m0, mrows, n0);
}

// Second pass when K was split across workgroups: y = sum_ks part (in ks
// order, deterministic), times the int8 per-channel scale when FMT8.
template <bool FMT8>
__global__ __launch_bounds__(256) void qmm_splitk_reduce_kernel(QArgs a) {
  const int64_t chunks = (int64_t)a.M * (a.N / 4);
  for (int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x; q < chunks; q += (int64_t)gridDim.x * 256) {
    const int m = (int)(q / (a.N / 4));
    const int n = (int)(q - (int64_t)m * (a.N / 4)) * 4;
    const int rb = m / kQRows, mr = m % kQRows;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int k = 0; k < a.ks; ++k)
      acc += *reinterpret_cast<const f32x4*>(a.part + ((size_t)(rb * a.ks + k) * kQRows + mr) * a.N + n);
    if (FMT8) acc *= *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(a.s) + n);
    epi_store_bf16x4(a.y, a.aux, a.epi, (size_t)m * a.N + n, acc);
  }
}

// Large-M path, first pass: the dequantised weight as bf16 [K, N] (into the
// workspace), which the bf16 GEMM then multiplies.  int4: (q - z) * s is
// exact in f32 (at most 12 significant bits) and rounded once to bf16 (RNE);
// int8: w * s is rounded to f32, then to bf16.  One thread: 8
// columns of RPT packed rows (int4: k = 2r and 2r + 1) or k rows (int8);
// every load and store is a whole 8- or 16-byte vector.  wd rows are ldd
// elements apart.  The paired form (below) writes a SwiGLU product's gate
// and up weights into one [K, 2N] buffer, column n of the gate at
// 32 (n / 16) + n % 16 and of the up 16 further: the 16-column interleave
// the MK_EPI_SWIGLU_PAIRS epilogue reads (8-column groups never straddle a
// 16-column block).
// Rows per thread of the dequantise kernels (RPT; it divides 32, so a
// thread's rows share an int4 64-k group).  Medians of one process, us,
// RPT 1 / 2 / 4 / 8:
//   int4 4096 x 14336            30.6 / 28.4 / 29.3 / 28.5
//   int4 2048 x 2048 and 8192 x 2048 (mixed)  10.5 / 10.0 / 9.5 / 9.0
//   int4 2048 x 6144              8.6 / 8.6 / 8.1 / 8.4
//   int4 pair 2048 x 2 x 8192    19.4 / 19.5 / 22.8 / 27.2
//   int8 4096 x 14336            43.0 / 33.5 / 35.0 / 37.9
// so 8 for an int4 weight, 2 for the pair (two weights per thread) and for
// int8.  MK_QMM_DEQ_RPT forces one.
inline int dequant_rpt(bool int4, bool pair) {
  if (const char* e = getenv("MK_QMM_DEQ_RPT")) {
    const int r = atoi(e);
    if (r == 1 || r == 2 || r == 4 || r == 8) return r;
  }
  return int4 && !pair ? 8 : 2;
}

// Grid: 256 column chunks of 8 by RPT rows.
inline dim3 dequant_grid(bool int4, int64_t K, int64_t N, int rpt) {
  const int64_t rows = int4 ? K / 2 : K;
  return dim3((unsigned)((N / 8 + 255) / 256), (unsigned)std::min<int64_t>((rows + rpt - 1) / rpt, 65535));
}

// One thread's share of a weight: 8 columns c0..c0+7 of RPT rows from r0
// (every row < rows), the scales (and int4 zero points, whose 64-k group
// the rows share) loaded once.
template <bool INT4, int RPT>
struct DeqRows {
  u32x2 wb[RPT];
  float sv[8];
  int zv[8];

  __device__ __forceinline__ void load(const QArgs& a, int r0, int rows, int c0) {
#pragma unroll
    for (int i = 0; i < RPT; ++i)
      if (r0 + i < rows) wb[i] = *reinterpret_cast<const u32x2*>(a.w + (int64_t)(r0 + i) * a.N + c0);
    if (INT4) {
      const int g = r0 / 32;  // 64-k group of rows 2r, 2r + 1 (RPT divides 32)
      const u32x4 sb = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(a.s) + (int64_t)g * a.N + c0);
      const u32x2 zb = *reinterpret_cast<const u32x2*>(a.z + (int64_t)g * a.N + c0);
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const uint32_t sw = (c < 2 ? sb.x : c < 4 ? sb.y : c < 6 ? sb.z : sb.w) >> (16 * (c & 1));
        sv[c] = bf16_to_f32(sw & 0xffffu);
        zv[c] = (int)(((c < 4 ? zb.x : zb.y) >> (8 * (c & 3))) & 0xffu);
      }
    } else {
      const float* sp = static_cast<const float*>(a.s) + c0;
      const f32x4 s0 = *reinterpret_cast<const f32x4*>(sp), s1 = *reinterpret_cast<const f32x4*>(sp + 4);
      sv[0] = s0.x; sv[1] = s0.y; sv[2] = s0.z; sv[3] = s0.w;
      sv[4] = s1.x; sv[5] = s1.y; sv[6] = s1.z; sv[7] = s1.w;
    }
  }

  // Rows of wd are ldd elements apart; this thread's 8 columns start at d0.
  __device__ __forceinline__ void emit(int r0, int rows, uint16_t* wd, int64_t ldd, int64_t d0) const {
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      if (r0 + i >= rows) break;
      const int64_t r = r0 + i;
      if (INT4) {
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int j = 0; j < 8; j += 2) {
          float e[2], o[2];
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int c = j + h;
            const uint32_t byte = ((c < 4 ? wb[i].x : wb[i].y) >> (8 * (c & 3))) & 0xffu;
            e[h] = (float)((int)(byte & 15u) - zv[c]) * sv[c];
            o[h] = (float)((int)(byte >> 4) - zv[c]) * sv[c];
          }
          lo[j / 2] = pack_bf16x2(e[0], e[1]);
          hi[j / 2] = pack_bf16x2(o[0], o[1]);
        }
        *reinterpret_cast<u32x4*>(wd + (2 * r) * ldd + d0) = u32x4{lo[0], lo[1], lo[2], lo[3]};
        *reinterpret_cast<u32x4*>(wd + (2 * r + 1) * ldd + d0) = u32x4{hi[0], hi[1], hi[2], hi[3]};
      } else {
        uint32_t out[4];
#pragma unroll
        for (int j = 0; j < 8; j += 2) {
          const int8_t b0 = (int8_t)(((j < 4 ? wb[i].x : wb[i].y) >> (8 * (j & 3))) & 0xffu);
          const int8_t b1 = (int8_t)(((j < 4 ? wb[i].x : wb[i].y) >> (8 * ((j + 1) & 3))) & 0xffu);
          out[j / 2] = pack_bf16x2((float)b0 * sv[j], (float)b1 * sv[j + 1]);
        }
        *reinterpret_cast<u32x4*>(wd + r * ldd + d0) = u32x4{out[0], out[1], out[2], out[3]};
      }
    }
  }
};

template <bool INT4, int RPT>
__global__ __launch_bounds__(256) void qmm_dequant_kernel(QArgs a, uint16_t* wd, int64_t ldd) {
  const int N8 = a.N / 8;
  const int rows = INT4 ? a.K / 2 : a.K;
  const int c8 = blockIdx.x * 256 + threadIdx.x;
  if (c8 >= N8) return;
  const int c0 = c8 * 8;
  const int64_t d0 = c0;
  for (int r0 = blockIdx.y * RPT; r0 < rows; r0 += gridDim.y * RPT) {
    DeqRows<INT4, RPT> d;
    d.load(a, r0, rows, c0);
    d.emit(r0, rows, wd, ldd, d0);
  }
}

// The gate and up weights of a paired SwiGLU product into one [K, 2N]
// buffer in one pass.  Lanes 2b and 2b + 1 write one whole 64-byte piece of
// a row between them, where two passes (one per weight) each wrote every
// other 32 bytes: 37 against 2 x 22.5 us for the decoder's 2048 x 8192
// weights.
template <bool INT4, int RPT>
__global__ __launch_bounds__(256) void qmm_dequant_pair_kernel(QArgs g, QArgs u, uint16_t* wd, int64_t ldd) {
  const int N8 = g.N / 8;
  const int rows = INT4 ? g.K / 2 : g.K;
  const int c8 = blockIdx.x * 256 + threadIdx.x;
  if (c8 >= N8) return;
  const int c0 = c8 * 8;
  const int64_t d0 = 32 * (c0 / 16) + c0 % 16;
  for (int r0 = blockIdx.y * RPT; r0 < rows; r0 += gridDim.y * RPT) {
    DeqRows<INT4, RPT> dg, du;
    dg.load(g, r0, rows, c0);
    du.load(u, r0, rows, c0);
    dg.emit(r0, rows, wd, ldd, d0);
    du.emit(r0, rows, wd, ldd, d0 + 16);
  }
}

}  // namespace mk

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
#include "../capi_internal.h"
#include "qgemm.h"

namespace {

constexpr size_t kMaxLds = 160 * 1024;

struct QPlan {
  int ks, nw, kwave, ntiles, rowblocks, wave_lds;
  int stream_steps;  // > 0: streaming kernel with this many 32-k steps per wave
  int ring;          // int8 streaming kernel: ring slots
  int wide_groups;   // > 0: wide int4 kernel with this many 64-k groups per wave
  int wide_cs;       // wide int4 kernel: column split (1: waves split K only; 2: also the columns in halves)
  int wide_tn;       // wide int4 kernel: tile columns (256, or 128 for narrow tiles)
  int wide8_steps;   // > 0: wide int8 kernel with this many 32-k steps per wave
  int wide8_cs;      // its column split (1: every wave over all 256 columns; 2: halves)
  int deq;           // 1: dequantise W to bf16 in the workspace, then the bf16 GEMM
  int qg;            // 1: the many-row kernel of qgemm.hip (K split ks ways)
  size_t lds_bytes;
  int64_t part_bytes;
};

int env_int(const char* name, int dflt) {
  const char* v = getenv(name);
  return v ? atoi(v) : dflt;
}

bool fill_plan(int fmt, int64_t K, int ks, int nw, QPlan* p) {
  const int groups = (int)(K / 64);
  if (ks < 1 || nw < 1 || groups % (ks * nw) != 0) return false;
  p->ks = ks;
  p->nw = nw;
  p->kwave = (int)(K / (ks * nw));
  const int xbytes = p->kwave * 32;          // 16 rows x kwave bf16
  const int ybytes = mk::kQRows * mk::kQCols * 4;
  p->wave_lds = xbytes > ybytes ? xbytes : ybytes;
  p->lds_bytes = (size_t)nw * p->wave_lds;
  return p->lds_bytes <= kMaxLds;
}

// Pick waves per workgroup (nw) and split-K (ks).  K stays whole inside a
// workgroup whenever x fits in LDS and the grid already covers ~192+ CUs;
// otherwise the smallest split that does.  Every wave gets a whole number of
// 64-k groups.  MK_QMM_KS / MK_QMM_NW force a choice (tuning sweeps).
// Streaming kernels: 8 waves, K = ks * 8 * 32 * S with S in {16, 8, 4, 2}
// (int4 needs S even), N % 16 == 0.  Prefer the fewest splits that still
// give >= 192 workgroups.
bool plan_stream(int fmt, int64_t K, int64_t N, QPlan* p) {
  if (N % 16 != 0 || N < 16 || getenv("MK_QMM_GENERIC")) return false;
  const int ks_env = env_int("MK_QMM_KS", 0);
  const int steps[4] = {16, 8, 4, 2};
  for (int ks = 1; ks <= 64; ks *= 2) {
    if (ks_env > 0 && ks != ks_env) continue;
    for (int i = 0; i < 4; ++i) {
      const int S = steps[i];
      if (K != (int64_t)ks * 8 * 32 * S) continue;
      if ((int64_t)p->ntiles * p->rowblocks * ks < 192 && ks_env <= 0 && 2 * ks <= 64 &&
          K % ((int64_t)2 * ks * 8 * 32 * 2) == 0)
        break;  // a larger split would still divide K: try it for more workgroups
      p->ks = ks;
      p->nw = 8;
      p->kwave = 32 * S;
      p->stream_steps = S;
      p->ring = fmt == MK_QFMT_INT4_G64 ? (S < 8 ? S : 8) : (S < 4 ? S : 4);
      p->wave_lds = fmt == MK_QFMT_INT4_G64 ? (2 * p->ring + 2) * 1024 : p->ring * 3072;
      p->lds_bytes = (size_t)8 * p->wave_lds;
      return true;
    }
  }
  return false;
}

// Wide int4 kernel: N % 128 == 0, K = ks * (NW / CS) * 64 * G with G in
// {1, 2, 4}; the fewest splits that give >= 192 workgroups (the most the
// 64 KB counter region and G >= 1 allow).  Grids below 128 workgroups stay
// on the 64-column kernels.  MK_QMM_WIDE=0 disables it.
// Ring depth (32-k steps in flight per wave) of the wide kernel with NW
// waves of G groups; MK_QMM_WIDE_RING overrides it (sweeps), and it is
// halved until the workgroup's LDS fits.  At the headline (8 waves, column
// split, ks 4, G 4), one box, one run: 2 steps in flight 11.37 us, 4 steps
// 11.79; 128-column tiles (ks 2) 11.55 us (2 steps) and 11.92 (ks 4);
// unsplit 256-column waves 12.47 us; 4 waves 13.11 us; ks 8 17.0 us.  The
// x block by LDS DMA instead of register loads took the column split from
// 12.02 to 11.43 us: with register loads in flight beside LDS DMAs the
// compiler waits for every outstanding load before the first step.
constexpr int kWideWaves = 8;
constexpr int kWideColumnSplit = 2;
constexpr int kWideTileColumns = 256;
// LDS bytes of one wave of the wide int4 kernel: ring, scale and zero-point
// blocks, x block; at least the y spill of a tile of tnw * cs columns.
int wide_wave_lds(int G, int tnw, int cs, int R) {
  const int sb = ((G * tnw * 2 + 1023) / 1024) * 1024, zb = ((G * tnw + 1023) / 1024) * 1024;
  const int wl = std::max(R * 16 * tnw + sb + zb + G * 2048, mk::kQRows * (tnw * cs + 4) * 4);
  return (wl + 255) & ~255;
}

int wide_ring(int nw, int G, int tnw = 256, int cs = 1) {
  int r = env_int("MK_QMM_WIDE_RING", 0);
  if (!(r >= 2 && r <= 2 * G && (r == 2 || r == 4 || r == 8))) {
    if (tnw == 128) r = 2;
    else if (nw == 4) r = G == 4 ? 4 : 2 * G;
    else r = G == 4 ? 4 : G == 2 ? 2 : 2 * G;
  }
  while (r > 2 && (size_t)nw * wide_wave_lds(G, tnw, cs, r) > kMaxLds) r /= 2;  // what fits
  return r;
}

bool plan_wide(int fmt, int64_t M, int64_t K, int64_t N, QPlan* p) {
  const char* env = getenv("MK_QMM_WIDE");
  if (fmt != MK_QFMT_INT4_G64 || N % 128 != 0 || (env && env[0] == '0')) return false;
  const int nw = env_int("MK_QMM_WIDE_NW", kWideWaves);
  // 256-column tiles where N allows, else 128 (MK_QMM_WIDE_TN forces one).
  int tn = nw == 8 ? env_int("MK_QMM_WIDE_TN", N % kWideTileColumns == 0 ? kWideTileColumns : 128) : mk::kWideTN;
  if (tn != 128 && tn != 256) return false;
  const int cs = nw == 8 && tn == 256 ? env_int("MK_QMM_WIDE_CS", kWideColumnSplit) : 1;
  if ((nw != 4 && nw != 8) || (cs != 1 && cs != 2) || N % tn != 0) return false;
  const int64_t kunit = (int64_t)(nw / cs) * 64;  // k per workgroup and group-per-wave
  if (K % kunit != 0) return false;
  const int ntiles = (int)(N / tn);
  const int rb = (int)((M + mk::kQRows - 1) / mk::kQRows);
  const int ks_env = env_int("MK_QMM_KS", 0);
  int best = 0;
  for (int ks = 1; ks <= 8; ks *= 2) {
    if (ks_env > 0 && ks != ks_env) continue;
    if (K % ((int64_t)ks * kunit) != 0) break;
    const int64_t G = K / ((int64_t)ks * kunit);
    if (G > 4) continue;
    if (G != 1 && G != 2 && G != 4) continue;
    if (ks > 1 && (int64_t)rb * ntiles > mk::kWideCounters) break;
    best = ks;
    if ((int64_t)ntiles * rb * ks >= 192) break;
  }
  if (best == 0 || (int64_t)ntiles * rb * best < 128) return false;
  const int G = (int)(K / ((int64_t)best * kunit));
  const int tnw = tn / cs;
  const int R = wide_ring(nw, G, tnw, cs);
  const int wl = wide_wave_lds(G, tnw, cs, R);
  p->ks = best;
  p->nw = nw;
  p->wide_cs = cs;
  p->wide_tn = tn;
  p->ntiles = ntiles;
  p->rowblocks = rb;
  p->wide_groups = G;
  p->kwave = 64 * G;
  p->wave_lds = wl;
  p->lds_bytes = (size_t)nw * wl;
  p->part_bytes = best > 1 ? (int64_t)mk::kWidePartOffset + (int64_t)rb * ntiles * best * mk::kQRows * tn * 4 : 0;
  return p->lds_bytes <= kMaxLds;
}

// Wide int8 kernel: N % 256 == 0, K = ks * 8 * 32 * S with S in {4, 8, 16};
// the fewest splits that give >= 192 workgroups, as for int4 (the same
// counter region bounds ks > 1).  A 2-step ring: 16 KB per wave, the size of
// its y spill.  MK_QMM_WIDE=0 disables it.
constexpr int kWide8Ring = 2;
// Waves split over two 128-column halves (twice the k steps each), as in
// the wide int4 kernel: M = 16 17.33 -> 16.54 us, M = 1 16.8 -> 16.0 us (one
// box, three interleaved repeats).  MK_QMM_WIDE8_CS overrides.
constexpr int kWide8ColumnSplit = 2;

bool plan_wide8(int fmt, int64_t M, int64_t K, int64_t N, QPlan* p) {
  const char* env = getenv("MK_QMM_WIDE");
  if (fmt != MK_QFMT_INT8_PC || N % mk::kWideTN != 0 || K % 1024 != 0 || (env && env[0] == '0')) return false;
  const int ntiles = (int)(N / mk::kWideTN);
  const int rb = (int)((M + mk::kQRows - 1) / mk::kQRows);
  const int ks_env = env_int("MK_QMM_KS", 0);
  const int cs = env_int("MK_QMM_WIDE8_CS", kWide8ColumnSplit);
  if (cs != 1 && cs != 2) return false;
  int best = 0;
  for (int ks = 1; ks <= 8; ks *= 2) {
    if (ks_env > 0 && ks != ks_env) continue;
    if (K % ((int64_t)ks * 1024) != 0) break;
    const int64_t S = K * cs / ((int64_t)ks * 256);
    if (S != 4 && S != 8 && S != 16) continue;
    if (ks > 1 && (int64_t)rb * ntiles > mk::kWideCounters) break;
    best = ks;
    if ((int64_t)ntiles * rb * ks >= 192) break;
  }
  if (best == 0 || (int64_t)ntiles * rb * best < 128) return false;
  const int64_t S = K * cs / ((int64_t)best * 256);
  // ring, the x block when the kernel stages x in LDS (S <= 4, or 8 with
  // the column split), the y spill
  const bool xl = cs == 1 ? S <= 4 : S <= 8;
  int wl = std::max(kWide8Ring * mk::kWide8Slot / cs + (xl ? (int)S * 1024 : 0), mk::kQRows * mk::kWideRedStride * 4);
  wl = (wl + 255) & ~255;
  p->ks = best;
  p->nw = 8;
  p->ntiles = ntiles;
  p->rowblocks = rb;
  p->wide8_steps = (int)S;
  p->wide8_cs = cs;
  p->kwave = 32 * p->wide8_steps;
  p->wave_lds = wl;
  p->lds_bytes = (size_t)8 * wl;
  p->part_bytes = best > 1 ? (int64_t)mk::kWidePartOffset + (int64_t)rb * ntiles * best * mk::kQRows * mk::kWideTN * 4
                           : 0;
  return p->lds_bytes <= kMaxLds;
}

// Many rows.  The streaming kernels re-read the weights once per 16 rows;
// from kQgMinRows rows the qgemm.hip kernel (weights read once per 256 rows,
// dequantised in LDS) takes over, and from kDeqMinRows rows W is dequantised
// to bf16 in the workspace once and multiplied by the bf16 GEMM, whose wider
// tiles win there (measured crossover between 512 and 768 rows at K = 4096,
// N = 14336).  Shapes qgemm does not take use the GEMM path from
// kDeqFallbackRows.  MK_QMM_QG_M / MK_QMM_DEQ_M override the thresholds; 0
// disables that path.
constexpr int kQgMinRows = 128;
constexpr int kDeqMinRows = 768;
constexpr int kDeqFallbackRows = 256;

// qg_cap bounds the workspace the many-row kernel's K split may use (the
// no-allocation entry point passes its array's size; the kernel then runs
// unsplit rather than ask for more).
bool plan_q(int fmt, int64_t M, int64_t K, int64_t N, QPlan* p, int64_t qg_cap = INT64_MAX) {
  *p = QPlan{};
  const int qg_m = env_int("MK_QMM_QG_M", kQgMinRows);
  const int deq_m = env_int("MK_QMM_DEQ_M", kDeqMinRows);
  const bool deq = deq_m > 0 && (M >= deq_m || M >= std::min(deq_m, kDeqFallbackRows));
  if (qg_m > 0 && M >= qg_m && !(deq_m > 0 && M >= deq_m) && mkq::qgemm_supported(M, K, N)) {
    p->qg = 1;
    p->ks = mkq::qgemm_ks(M, K, N, qg_cap);
    p->part_bytes = mkq::qgemm_workspace_bytes(M, K, N, p->ks);
    return true;
  }
  if (deq) {
    p->deq = 1;
    p->part_bytes = (int64_t)mk::kWidePartOffset + K * N * 2;
    return true;
  }
  if (plan_wide(fmt, M, K, N, p)) return true;
  p->wide_groups = 0;
  if (plan_wide8(fmt, M, K, N, p)) return true;
  p->wide8_steps = 0;
  p->ntiles = (int)((N + mk::kQCols - 1) / mk::kQCols);
  p->rowblocks = (int)((M + mk::kQRows - 1) / mk::kQRows);
  if (plan_stream(fmt, K, N, p)) {
    p->part_bytes = p->ks > 1 ? (int64_t)mk::kWidePartOffset + (int64_t)p->rowblocks * p->ks * mk::kQRows * N * 4 : 0;
    return true;
  }
  const int ks_env = env_int("MK_QMM_KS", 0), nw_env = env_int("MK_QMM_NW", 0);
  const int nws[4] = {8, 4, 2, 1};
  QPlan best;
  bool have = false;
  for (int ks = 1; ks <= 64; ks *= 2) {
    if (ks_env > 0 && ks != ks_env) continue;
    for (int i = 0; i < 4; ++i) {
      if (nw_env > 0 && nws[i] != nw_env) continue;
      QPlan q = *p;
      if (!fill_plan(fmt, K, ks, nws[i], &q)) continue;
      if (!have) {
        best = q;
        have = true;
      }
      if ((int64_t)p->ntiles * p->rowblocks * ks >= 192) {
        *p = q;
        goto done;
      }
      break;  // widest nw that fits for this ks
    }
  }
  if (!have) return false;
  *p = best;
  // Grid too small even at the largest split tried: keep the first plan that
  // fits (fewest partials) rather than fail.
done:
  p->part_bytes = p->ks > 1 ? (int64_t)mk::kWidePartOffset + (int64_t)p->rowblocks * p->ks * mk::kQRows * N * 4 : 0;
  return true;
}

// Kernels that need more than the default 64 KB of dynamic LDS must opt in.
hipError_t lds_opt_in(const void* fn, size_t bytes) {
  if (bytes <= 64 * 1024) return hipSuccess;
  return hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
}

hipError_t launch_reduce(int fmt, const mk::QArgs& a, hipStream_t st);

template <int NW, int G, int R, int CS, int TN>
hipError_t launch_wide_nwgr(const mk::QArgs& a, const QPlan& p, hipStream_t st) {
  dim3 grid(p.ntiles * p.ks, p.rowblocks), block(NW * mk::kWave);
  hipError_t e = lds_opt_in((const void*)mk::int4g64_wide_kernel<NW, G, R, CS, TN>, p.lds_bytes);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((mk::int4g64_wide_kernel<NW, G, R, CS, TN>), grid, block, p.lds_bytes, st, a);
  return hipGetLastError();
}

template <int NW, int G, int CS = 1, int TN = mk::kWideTN>
hipError_t launch_wide(const mk::QArgs& a, const QPlan& p, hipStream_t st) {
  switch (wide_ring(NW, G, TN / CS, CS)) {
    case 2: return launch_wide_nwgr<NW, G, 2, CS, TN>(a, p, st);
    case 4: if constexpr (2 * G >= 4) return launch_wide_nwgr<NW, G, 4, CS, TN>(a, p, st); break;
    case 8: if constexpr (2 * G >= 8) return launch_wide_nwgr<NW, G, 8, CS, TN>(a, p, st); break;
  }
  return hipErrorInvalidValue;
}

template <int S, int CS>
hipError_t launch_wide8(const mk::QArgs& a, const QPlan& p, hipStream_t st) {
  dim3 grid(p.ntiles * p.ks, p.rowblocks), block(8 * mk::kWave);
  hipError_t e = lds_opt_in((const void*)mk::int8pc_wide_kernel<S, kWide8Ring, CS>, p.lds_bytes);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((mk::int8pc_wide_kernel<S, kWide8Ring, CS>), grid, block, p.lds_bytes, st, a);
  return hipGetLastError();
}

template <int S>
hipError_t launch_stream(int fmt, const mk::QArgs& a, const QPlan& p, hipStream_t st) {
  dim3 grid(p.ntiles * p.ks, p.rowblocks), block(8 * mk::kWave);
  const void* fn = fmt == MK_QFMT_INT4_G64 ? (const void*)mk::int4g64_stream_kernel<S, (S < 8 ? S : 8)>
                                           : (const void*)mk::int8pc_stream_kernel<S, (S < 4 ? S : 4)>;
  hipError_t e = lds_opt_in(fn, p.lds_bytes);
  if (e != hipSuccess) return e;
  if (fmt == MK_QFMT_INT4_G64)
    hipLaunchKernelGGL((mk::int4g64_stream_kernel<S, (S < 8 ? S : 8)>), grid, block, p.lds_bytes, st, a);
  else
    hipLaunchKernelGGL((mk::int8pc_stream_kernel<S, (S < 4 ? S : 4)>), grid, block, p.lds_bytes, st, a);
  e = hipGetLastError();
  if (e != hipSuccess || p.ks == 1 || a.cnt) return e;
  return launch_reduce(fmt, a, st);
}

template <int NW>
hipError_t launch_q(int fmt, const mk::QArgs& a, const QPlan& p, hipStream_t st) {
  dim3 grid(p.ntiles * p.ks, p.rowblocks), block(NW * mk::kWave);
  const void* fn = fmt == MK_QFMT_INT4_G64 ? (const void*)mk::int4g64_gemv_kernel<NW>
                                           : (const void*)mk::int8pc_gemv_kernel<NW>;
  hipError_t e = lds_opt_in(fn, p.lds_bytes);
  if (e != hipSuccess) return e;
  if (fmt == MK_QFMT_INT4_G64) {
    hipLaunchKernelGGL(mk::int4g64_gemv_kernel<NW>, grid, block, p.lds_bytes, st, a);
  } else {
    hipLaunchKernelGGL(mk::int8pc_gemv_kernel<NW>, grid, block, p.lds_bytes, st, a);
  }
  e = hipGetLastError();
  if (e != hipSuccess || p.ks == 1 || a.cnt) return e;
  return launch_reduce(fmt, a, st);
}

hipError_t launch_reduce(int fmt, const mk::QArgs& a, hipStream_t st) {
  const int64_t chunks = (int64_t)a.M * (a.N / 4);
  const int blocks = (int)std::min<int64_t>((chunks + 255) / 256, 4096);
  if (fmt == MK_QFMT_INT4_G64)
    hipLaunchKernelGGL(mk::qmm_splitk_reduce_kernel<false>, dim3(blocks), dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL(mk::qmm_splitk_reduce_kernel<true>, dim3(blocks), dim3(256), 0, st, a);
  return hipGetLastError();
}

// Workgroup placement.  The wide int4 kernel's split-K exchange can stay in
// one XCD's L2 when every workgroup of a tile runs on the same XCD.  In the
// GPU's single-partition mode the dispatcher deals workgroups to the 8 XCDs
// round-robin (linear workgroup id i on XCD i % 8); with gridDim.x % 8 == 0
// and (gridDim.x / 8) % ks == 0, xcd_logical_id then gives each tile's ks
// workgroups one XCD.  That dealing is checked once per device, outside graph
// capture, by a probe launch of the same grid shape that compares each
// workgroup's hardware XCC id with its linear id; until a probe has passed
// (and under MK_QMM_XCH=device) the exchange goes through device scope.
__global__ void xcd_probe_kernel(uint32_t* bad) {
  uint32_t xcc;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
  const uint32_t lin = blockIdx.x + blockIdx.y * gridDim.x;
  if (threadIdx.x == 0 && (xcc & 7u) != (lin & 7u)) atomicOr(bad, 1u);
}

constexpr int kXcdMaxDevices = 64;
std::atomic<int> g_xcd_state[kXcdMaxDevices];  // 0 unknown, 1 round-robin, 2 other

// True when workgroups of `grid` are dealt round-robin to the 8 XCDs on the
// current device.  Probes (synchronously on `st`, using the first word of
// `word` as scratch) the first time it is asked outside graph capture.
bool xcd_round_robin(dim3 grid, hipStream_t st, uint32_t* word) {
  const char* env = getenv("MK_QMM_XCH");
  if (env && std::strcmp(env, "device") == 0) return false;
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kXcdMaxDevices) return false;
  const int state = g_xcd_state[dev].load(std::memory_order_acquire);
  if (state != 0) return state == 1;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return false;
  uint32_t bad = 1;
  if (hipMemsetAsync(word, 0, sizeof(uint32_t), st) != hipSuccess) return false;
  hipLaunchKernelGGL(xcd_probe_kernel, grid, dim3(64), 0, st, word);
  if (hipGetLastError() != hipSuccess) return false;
  if (hipMemcpyAsync(&bad, word, sizeof(uint32_t), hipMemcpyDeviceToHost, st) != hipSuccess ||
      hipStreamSynchronize(st) != hipSuccess)
    return false;
  g_xcd_state[dev].store(bad == 0 ? 1 : 2, std::memory_order_release);
  return bad == 0;
}

// The dequantise pass: W [K, N] -> bf16 rows of N (up == null), or the
// gate (a) and up weights into one interleaved [K, 2N] buffer.
hipError_t launch_dequant(bool int4, const mk::QArgs& a, const mk::QArgs* up, uint16_t* wd, int64_t N, int64_t K,
                          hipStream_t st) {
  const int rpt = mk::dequant_rpt(int4, up != nullptr);
  const dim3 grid = mk::dequant_grid(int4, K, N, rpt);
#define MK_DEQ_LAUNCH(I4, R)                                                                                      \
  if (up)                                                                                                        \
    hipLaunchKernelGGL((mk::qmm_dequant_pair_kernel<I4, R>), grid, dim3(256), 0, st, a, *up, wd, 2 * N);          \
  else                                                                                                           \
    hipLaunchKernelGGL((mk::qmm_dequant_kernel<I4, R>), grid, dim3(256), 0, st, a, wd, N);
  switch ((int4 ? 16 : 0) + rpt) {
    case 16 + 8: MK_DEQ_LAUNCH(true, 8) break;
    case 16 + 4: MK_DEQ_LAUNCH(true, 4) break;
    case 16 + 2: MK_DEQ_LAUNCH(true, 2) break;
    case 16 + 1: MK_DEQ_LAUNCH(true, 1) break;
    case 8: MK_DEQ_LAUNCH(false, 8) break;
    case 4: MK_DEQ_LAUNCH(false, 4) break;
    case 2: MK_DEQ_LAUNCH(false, 2) break;
    default: MK_DEQ_LAUNCH(false, 1) break;
  }
#undef MK_DEQ_LAUNCH
  return hipGetLastError();
}

int run_q(int fmt, const void* x, const void* w, const void* s, const void* z, void* y, int64_t M,
          int64_t K, int64_t N, void* ws, int64_t ws_bytes, void* stream, const void* aux = nullptr,
          int epi = MK_EPI_NONE, int64_t qg_cap = INT64_MAX) {
  const char* fn = fmt == MK_QFMT_INT4_G64 ? "mk_int4g64_matmul_bf16" : "mk_int8pc_matmul_bf16";
  if (epi != MK_EPI_NONE && epi != MK_EPI_ADD && epi != MK_EPI_SWIGLU && epi != MK_EPI_SWIGLU_PAIRS)
    return mkc::fail(MK_EINVAL, "%s: unknown epilogue %d", fn, epi);
  if (epi != MK_EPI_NONE && epi != MK_EPI_SWIGLU_PAIRS && !aux)
    return mkc::fail(MK_EINVAL, "%s: the epilogue needs aux", fn);
  if (!x || !w || !s || !y || (fmt == MK_QFMT_INT4_G64 && !z))
    return mkc::fail(MK_EINVAL, "%s: null pointer argument", fn);
  if (M <= 0 || K <= 0 || N <= 0)
    return mkc::fail(MK_EINVAL, "%s: M, K, N must be positive (got %lld, %lld, %lld)", fn,
                     (long long)M, (long long)K, (long long)N);
  if (K % 64 != 0 || N % 8 != 0)
    return mkc::fail(MK_EINVAL, "%s: need K %% 64 == 0 and N %% 8 == 0 (got K=%lld, N=%lld)", fn,
                     (long long)K, (long long)N);
  if (M > (1 << 20) || K > (1 << 24) || N > (1 << 26) || (M * K) > (int64_t)1 << 31)
    return mkc::fail(MK_EINVAL, "%s: shape too large", fn);
  QPlan p;
  if (!plan_q(fmt, M, K, N, &p, qg_cap))
    return mkc::fail(MK_EUNSUPPORTED, "%s: no launch configuration for K=%lld", fn, (long long)K);
  // The paired SwiGLU (interleaved gate / up columns, y [M, N/2]) is an
  // epilogue of the bf16 GEMM only: it needs the dequantise-then-GEMM route.
  if (epi == MK_EPI_SWIGLU_PAIRS && !p.deq)
    return mkc::fail(MK_EUNSUPPORTED, "%s: paired SwiGLU needs the dequantise-then-GEMM route (M >= %d)", fn,
                     kDeqMinRows);
  if (p.part_bytes > 0 && (!ws || ws_bytes < p.part_bytes))
    return mkc::fail(MK_EWORKSPACE, "%s: workspace of %lld bytes needed, %lld given", fn,
                     (long long)p.part_bytes, (long long)ws_bytes);
  mk::QArgs a;
  a.x = static_cast<const uint16_t*>(x);
  a.w = static_cast<const uint8_t*>(w);
  a.s = s;
  a.z = static_cast<const uint8_t*>(z);
  a.y = static_cast<uint16_t*>(y);
  // Workspace: [0, 64 KB) arrival counters of the wide kernel (zero between
  // calls), then split-K partials for whichever kernel runs.
  a.part = p.part_bytes > 0 ? reinterpret_cast<float*>(static_cast<unsigned char*>(ws) + mk::kWidePartOffset)
                            : nullptr;
  a.M = (int)M;
  a.K = (int)K;
  a.N = (int)N;
  a.ks = p.ks;
  a.kwave = p.kwave;
  a.wave_lds = p.wave_lds;
  a.cnt = nullptr;
  a.xch_local = 0;
  a.aux = static_cast<const uint16_t*>(aux);
  a.epi = epi;
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipError_t e;
  if (p.qg) {
    // The split-K exchange stays in one XCD's L2 when the placement probe
    // has seen round-robin dealing (as for the wide kernel below).
    const unsigned gx = mkq::qgemm_grid(M, N, p.ks);
    const bool local = p.ks > 1 && mkq::qgemm_tile_on_one_xcd(gx, p.ks) &&
                       xcd_round_robin(dim3(gx), st, reinterpret_cast<uint32_t*>(a.part));
    e = mkq::qgemm_launch(fmt == MK_QFMT_INT4_G64, x, w, s, z, y, M, K, N, aux, epi, p.ks, ws, st, local);
    if (e != hipSuccess) return mkc::fail(MK_ELAUNCH, "%s: launch failed: %s", fn, hipGetErrorString(e));
    return MK_OK;
  }
  if (p.deq) {
    uint16_t* wd = reinterpret_cast<uint16_t*>(a.part);
    e = launch_dequant(fmt == MK_QFMT_INT4_G64, a, nullptr, wd, N, K, st);
    if (e != hipSuccess) return mkc::fail(MK_ELAUNCH, "%s: dequantise launch failed: %s", fn, hipGetErrorString(e));
    const int rc = epi == MK_EPI_NONE ? mk_gemm_bf16(x, wd, y, 1, M, N, K, 0, stream)
                                      : mk_gemm_bf16_epilogue(x, wd, y, aux, epi, 1, M, N, K, stream);
    if (rc != MK_OK) return rc;
    return MK_OK;
  }
  if (p.wide_groups > 0) {
    if (p.part_bytes > 0) a.cnt = static_cast<uint32_t*>(ws);
    const int gx = p.ntiles * p.ks;
    a.xch_local = p.ks > 1 && gx % 8 == 0 && (gx / 8) % p.ks == 0 &&
                  xcd_round_robin(dim3(gx, p.rowblocks), st, reinterpret_cast<uint32_t*>(a.part));
    if (p.wide_tn == 128) {
      switch (p.wide_groups) {
        case 1: e = launch_wide<8, 1, 1, 128>(a, p, st); break;
        case 2: e = launch_wide<8, 2, 1, 128>(a, p, st); break;
        default: e = launch_wide<8, 4, 1, 128>(a, p, st); break;
      }
    } else if (p.wide_cs == 2) {
      switch (p.wide_groups) {
        case 1: e = launch_wide<8, 1, 2>(a, p, st); break;
        case 2: e = launch_wide<8, 2, 2>(a, p, st); break;
        default: e = launch_wide<8, 4, 2>(a, p, st); break;
      }
    } else {
      switch (p.wide_groups * (p.nw == 4 ? -1 : 1)) {
        case 1: e = launch_wide<8, 1>(a, p, st); break;
        case 2: e = launch_wide<8, 2>(a, p, st); break;
        case 4: e = launch_wide<8, 4>(a, p, st); break;
        case -1: e = launch_wide<4, 1>(a, p, st); break;
        case -2: e = launch_wide<4, 2>(a, p, st); break;
        default: e = launch_wide<4, 4>(a, p, st); break;
      }
    }
  } else if (p.wide8_steps > 0) {
    if (p.part_bytes > 0) a.cnt = static_cast<uint32_t*>(ws);
    switch (p.wide8_steps * 4 + p.wide8_cs) {
      case 4 * 4 + 1: e = launch_wide8<4, 1>(a, p, st); break;
      case 8 * 4 + 1: e = launch_wide8<8, 1>(a, p, st); break;
      case 16 * 4 + 1: e = launch_wide8<16, 1>(a, p, st); break;
      case 4 * 4 + 2: e = launch_wide8<4, 2>(a, p, st); break;
      case 8 * 4 + 2: e = launch_wide8<8, 2>(a, p, st); break;
      default: e = launch_wide8<16, 2>(a, p, st); break;
    }
  } else if (p.stream_steps > 0) {
    // Split-K partials combined in the kernel (the counters live in the
    // workspace's first 64 KB), else by a second, reduce kernel
    // (MK_QMM_REDUCE_PASS=1 forces the latter; same results, bit for bit).
    if (p.ks > 1 && (int64_t)p.rowblocks * p.ntiles <= mk::kWideCounters && !env_int("MK_QMM_REDUCE_PASS", 0))
      a.cnt = static_cast<uint32_t*>(ws);
    switch (p.stream_steps) {
      case 16: e = launch_stream<16>(fmt, a, p, st); break;
      case 8: e = launch_stream<8>(fmt, a, p, st); break;
      case 4: e = launch_stream<4>(fmt, a, p, st); break;
      default: e = launch_stream<2>(fmt, a, p, st); break;
    }
  } else {
    if (p.ks > 1 && (int64_t)p.rowblocks * p.ntiles <= mk::kWideCounters && !env_int("MK_QMM_REDUCE_PASS", 0))
      a.cnt = static_cast<uint32_t*>(ws);
    switch (p.nw) {
    case 1: e = launch_q<1>(fmt, a, p, st); break;
    case 2: e = launch_q<2>(fmt, a, p, st); break;
    case 4: e = launch_q<4>(fmt, a, p, st); break;
    default: e = launch_q<8>(fmt, a, p, st); break;
    }
  }
  if (e != hipSuccess) return mkc::fail(MK_ELAUNCH, "%s: launch failed: %s", fn, hipGetErrorString(e));
  return MK_OK;
}

}  // namespace

extern "C" int64_t mk_qmatmul_workspace_bytes(int fmt, int64_t M, int64_t K, int64_t N) {
  if ((fmt != MK_QFMT_INT4_G64 && fmt != MK_QFMT_INT8_PC) || M <= 0 || K <= 0 || N <= 0 ||
      K % 64 != 0)
    return -1;
  QPlan p;
  if (!plan_q(fmt, M, K, N, &p)) return -1;
  return p.part_bytes;
}

extern "C" int mk_qmatmul_epilogue_supported(int fmt, int64_t M, int64_t K, int64_t N, int epilogue) {
  if (mk_qmatmul_workspace_bytes(fmt, M, K, N) < 0) return 0;
  if (epilogue == MK_EPI_NONE || epilogue == MK_EPI_ADD || epilogue == MK_EPI_SWIGLU) return 1;
  if (epilogue != MK_EPI_SWIGLU_PAIRS) return 0;
  QPlan p;
  return plan_q(fmt, M, K, N, &p) && p.deq && M % 256 == 0 && N % 256 == 0 ? 1 : 0;
}

extern "C" int mk_int4g64_matmul_bf16(const void* x, const void* w_packed, const void* scale,
                                      const void* zero, void* y, int64_t M, int64_t K, int64_t N,
                                      void* workspace, int64_t workspace_bytes, void* stream) {
  mkc::clear_error();
  return run_q(MK_QFMT_INT4_G64, x, w_packed, scale, zero, y, M, K, N, workspace, workspace_bytes,
               stream);
}

extern "C" int mk_int8pc_matmul_bf16(const void* x, const void* w, const void* scale, void* y,
                                     int64_t M, int64_t K, int64_t N, void* workspace,
                                     int64_t workspace_bytes, void* stream) {
  mkc::clear_error();
  return run_q(MK_QFMT_INT8_PC, x, w, scale, nullptr, y, M, K, N, workspace, workspace_bytes,
               stream);
}

extern "C" int mk_int4g64_matmul_epilogue_bf16(const void* x, const void* w_packed, const void* scale,
                                               const void* zero, void* y, const void* aux, int epilogue,
                                               int64_t M, int64_t K, int64_t N, void* workspace,
                                               int64_t workspace_bytes, void* stream) {
  mkc::clear_error();
  return run_q(MK_QFMT_INT4_G64, x, w_packed, scale, zero, y, M, K, N, workspace, workspace_bytes, stream, aux,
               epilogue);
}

extern "C" int mk_int8pc_matmul_epilogue_bf16(const void* x, const void* w, const void* scale, void* y,
                                              const void* aux, int epilogue, int64_t M, int64_t K, int64_t N,
                                              void* workspace, int64_t workspace_bytes, void* stream) {
  mkc::clear_error();
  return run_q(MK_QFMT_INT8_PC, x, w, scale, nullptr, y, M, K, N, workspace, workspace_bytes, stream, aux,
               epilogue);
}

// ---------------------------------------------------------------------------
// Paired SwiGLU product from two separate weights, silu(x @ Wg) * (x @ Wu):
// both weights dequantised into one bf16 [K, 2N] buffer in the workspace,
// their 16-column blocks interleaved (gate, up, gate, up, ...), then one bf16
// GEMM whose MK_EPI_SWIGLU_PAIRS store writes silu(gate) * up.  The
// dequantised values, the GEMM's k order and the epilogue's roundings are
// those of the two products followed by the SwiGLU program, so the result is
// bit-identical to that form; it saves the gate product's bf16 round trip
// through HBM and one GEMM launch.  Many-row shapes only (the
// dequantise-then-GEMM route, M % 256 == 0, N % 128 == 0).
// ---------------------------------------------------------------------------
namespace {

int64_t pair_workspace(int fmt, int64_t M, int64_t K, int64_t N) {
  if ((fmt != MK_QFMT_INT4_G64 && fmt != MK_QFMT_INT8_PC) || M <= 0 || K <= 0 || N <= 0 || K % 64 != 0 ||
      N % 128 != 0 || M % 256 != 0)
    return -1;
  QPlan p;
  if (!plan_q(fmt, M, K, N, &p) || !p.deq) return -1;
  return (int64_t)mk::kWidePartOffset + K * (2 * N) * 2;
}

int run_pair(int fmt, const void* x, const void* wg, const void* sg, const void* zg, const void* wu, const void* su,
             const void* zu, void* y, int64_t M, int64_t K, int64_t N, void* ws, int64_t ws_bytes, void* stream) {
  const char* fn = fmt == MK_QFMT_INT4_G64 ? "mk_int4g64_matmul_swiglu_pair_bf16" : "mk_int8pc_matmul_swiglu_pair_bf16";
  if (!x || !wg || !sg || !wu || !su || !y || (fmt == MK_QFMT_INT4_G64 && (!zg || !zu)))
    return mkc::fail(MK_EINVAL, "%s: null pointer argument", fn);
  if (M <= 0 || K <= 0 || N <= 0)
    return mkc::fail(MK_EINVAL, "%s: M, K, N must be positive (got %lld, %lld, %lld)", fn, (long long)M,
                     (long long)K, (long long)N);
  if (M > (1 << 20) || K > (1 << 24) || N > (1 << 25) || (M * K) > (int64_t)1 << 31)
    return mkc::fail(MK_EINVAL, "%s: shape too large", fn);
  const int64_t need = pair_workspace(fmt, M, K, N);
  if (need < 0)
    return mkc::fail(MK_EUNSUPPORTED, "%s: needs the many-row route with M %% 256 == 0, N %% 128 == 0, "
                     "K %% 64 == 0 (got M=%lld, K=%lld, N=%lld)", fn, (long long)M, (long long)K, (long long)N);
  if (!ws || ws_bytes < need)
    return mkc::fail(MK_EWORKSPACE, "%s: workspace of %lld bytes needed, %lld given", fn, (long long)need,
                     (long long)ws_bytes);
  uint16_t* wd = reinterpret_cast<uint16_t*>(static_cast<unsigned char*>(ws) + mk::kWidePartOffset);
  hipStream_t st = static_cast<hipStream_t>(stream);
  mk::QArgs ag{}, au{};
  for (int half = 0; half < 2; ++half) {
    mk::QArgs& a = half ? au : ag;
    a.w = static_cast<const uint8_t*>(half ? wu : wg);
    a.s = half ? su : sg;
    a.z = static_cast<const uint8_t*>(half ? zu : zg);
    a.M = (int)M;
    a.K = (int)K;
    a.N = (int)N;
  }
  const hipError_t e = launch_dequant(fmt == MK_QFMT_INT4_G64, ag, &au, wd, N, K, st);
  if (e != hipSuccess) return mkc::fail(MK_ELAUNCH, "%s: dequantise launch failed: %s", fn, hipGetErrorString(e));
  return mk_gemm_bf16_epilogue(x, wd, y, nullptr, MK_EPI_SWIGLU_PAIRS, 1, M, 2 * N, K, stream);
}

}  // namespace

extern "C" int64_t mk_qmatmul_swiglu_pair_workspace_bytes(int fmt, int64_t M, int64_t K, int64_t N) {
  return pair_workspace(fmt, M, K, N);
}

extern "C" int mk_int4g64_matmul_swiglu_pair_bf16(const void* x, const void* wg_packed, const void* g_scale,
                                                  const void* g_zero, const void* wu_packed, const void* u_scale,
                                                  const void* u_zero, void* y, int64_t M, int64_t K, int64_t N,
                                                  void* workspace, int64_t workspace_bytes, void* stream) {
  mkc::clear_error();
  return run_pair(MK_QFMT_INT4_G64, x, wg_packed, g_scale, g_zero, wu_packed, u_scale, u_zero, y, M, K, N, workspace,
                  workspace_bytes, stream);
}

extern "C" int mk_int8pc_matmul_swiglu_pair_bf16(const void* x, const void* wg, const void* g_scale, const void* wu,
                                                 const void* u_scale, void* y, int64_t M, int64_t K, int64_t N,
                                                 void* workspace, int64_t workspace_bytes, void* stream) {
  mkc::clear_error();
  return run_pair(MK_QFMT_INT8_PC, x, wg, g_scale, nullptr, wu, u_scale, nullptr, y, M, K, N, workspace,
                  workspace_bytes, stream);
}

// ---------------------------------------------------------------------------
// No-allocation entry point: the workspace is a file-scope device array.
//
// Each GPU the library runs on holds its own copy of `scratch` until the
// process ends.  In host code the array's name is only a host-side stand-in,
// so every host use goes through the per-device address that
// hipGetSymbolAddress returns at set-up.  The first 64 KB are the wide
// kernel's arrival counters, which must read zero before a call: set-up
// clears them once per device with a fill kernel (not a memset node, so the
// call can sit inside a captured graph), and every completed call leaves them
// at zero again.  All calls on one GPU share the array: calls that overlap in
// time on one GPU (different streams without ordering) race on it.
// ---------------------------------------------------------------------------
#include <mutex>

namespace {

constexpr int64_t kNoAllocScratchBytes = 8ll << 20;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

__global__ void scratch_clear_kernel(uint32_t* p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The calling thread's device's copy of `scratch`, set up on first use:
// its address, and its counter region cleared on `stream`.
int scratch_for_current_device(hipStream_t stream, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return mkc::fail(MK_ELAUNCH, "mk_int4g64_matmul_bf16_noalloc: no current device (%s)", hipGetErrorString(e));
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      return mkc::fail(MK_ELAUNCH, "mk_int4g64_matmul_bf16_noalloc: hipGetSymbolAddress failed on device %d: %s",
                       dev, hipGetErrorString(e));
    const int words = (int)(mk::kWidePartOffset / 4);
    hipLaunchKernelGGL(scratch_clear_kernel, dim3((words + 255) / 256), dim3(256), 0, stream,
                       static_cast<uint32_t*>(ptr), words);
    e = hipGetLastError();
    if (e != hipSuccess)
      return mkc::fail(MK_ELAUNCH, "mk_int4g64_matmul_bf16_noalloc: scratch clear failed: %s", hipGetErrorString(e));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return MK_OK;
}

}  // namespace

extern "C" int mk_int4g64_matmul_bf16_noalloc(const void* x, const void* w_packed, const void* scale,
                                              const void* zero, void* y, int64_t M, int64_t K, int64_t N,
                                              void* stream) {
  mkc::clear_error();
  // The plan this entry point runs: the many-row kernel's K split only when
  // its partials fit the array.
  QPlan cp;
  const int64_t need = (M > 0 && K > 0 && N > 0 && K % 64 == 0 &&
                        plan_q(MK_QFMT_INT4_G64, M, K, N, &cp, kNoAllocScratchBytes))
                           ? cp.part_bytes
                           : -1;
  if (need > kNoAllocScratchBytes)
    return mkc::fail(MK_EWORKSPACE,
                     "mk_int4g64_matmul_bf16_noalloc: M=%lld K=%lld N=%lld needs %lld bytes of workspace; "
                     "the no-allocation entry point holds %lld (use mk_int4g64_matmul_bf16 with a workspace)",
                     (long long)M, (long long)K, (long long)N, (long long)need, (long long)kNoAllocScratchBytes);
  // Shapes the plan rejects (need < 0) fail in run_q with its own message,
  // before anything is set up or launched.
  if (need < 0)
    return run_q(MK_QFMT_INT4_G64, x, w_packed, scale, zero, y, M, K, N, nullptr, 0, stream);
  hipStream_t st = static_cast<hipStream_t>(stream);
  void* ws = nullptr;
  const int rc = scratch_for_current_device(st, &ws);
  if (rc != MK_OK) return rc;
  return run_q(MK_QFMT_INT4_G64, x, w_packed, scale, zero, y, M, K, N, ws, kNoAllocScratchBytes, stream, nullptr,
               MK_EPI_NONE, kNoAllocScratchBytes);
}
