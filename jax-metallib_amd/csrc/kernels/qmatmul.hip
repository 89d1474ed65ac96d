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

#include <algorithm>

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

// Sum the NW wave tiles of the workgroup and emit bf16 y (ks == 1, with the
// int8 per-channel scale when FMT8) or the f32 split-K partial (ks > 1).
template <int NW, bool FMT8>
__device__ __forceinline__ void reduce_and_store(const QArgs& a, const unsigned char* smem, int ksi,
                                                 int rb, int m0, int mrows, int n0) {
  __syncthreads();
  for (int item = threadIdx.x; item < kQRows * (kQCols / 4); item += NW * kWave) {
    const int m = item / (kQCols / 4), ch = item % (kQCols / 4);
    const int n = n0 + 4 * ch;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < NW; ++w)
      acc += *reinterpret_cast<const f32x4*>(smem + w * a.wave_lds + (m * kQCols + 4 * ch) * 4);
    if (m >= mrows || n >= a.N) continue;
    if (a.ks > 1) {
      *reinterpret_cast<f32x4*>(a.part + ((size_t)(rb * a.ks + ksi) * kQRows + m) * a.N + n) = acc;
    } else {
      if (FMT8) acc *= *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(a.s) + n);
      *reinterpret_cast<u32x2*>(a.y + (size_t)(m0 + m) * a.N + n) =
          u32x2{pack_bf16x2(acc.x, acc.y), pack_bf16x2(acc.z, acc.w)};
    }
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
typedef __attribute__((address_space(3))) void* lds_vptr;
typedef __attribute__((address_space(1))) const void* glb_cptr;

__device__ __forceinline__ void dma16(const void* g, void* lds_uniform) {
  __builtin_amdgcn_global_load_lds((glb_cptr)g, (lds_vptr)lds_uniform, 16, 0, 0);
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(lds_vptr)p;
}

// s_waitcnt vmcnt(n) for a value the unrolled loops fold to a constant.
__device__ __forceinline__ void vm_wait(int n) {
  switch (n) {
    case 0: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
    case 1: asm volatile("s_waitcnt vmcnt(1)" ::: "memory"); break;
    case 2: asm volatile("s_waitcnt vmcnt(2)" ::: "memory"); break;
    case 3: asm volatile("s_waitcnt vmcnt(3)" ::: "memory"); break;
    case 4: asm volatile("s_waitcnt vmcnt(4)" ::: "memory"); break;
    case 5: asm volatile("s_waitcnt vmcnt(5)" ::: "memory"); break;
    case 6: asm volatile("s_waitcnt vmcnt(6)" ::: "memory"); break;
    case 7: asm volatile("s_waitcnt vmcnt(7)" ::: "memory"); break;
    case 8: asm volatile("s_waitcnt vmcnt(8)" ::: "memory"); break;
    case 9: asm volatile("s_waitcnt vmcnt(9)" ::: "memory"); break;
    case 10: asm volatile("s_waitcnt vmcnt(10)" ::: "memory"); break;
    case 11: asm volatile("s_waitcnt vmcnt(11)" ::: "memory"); break;
    case 12: asm volatile("s_waitcnt vmcnt(12)" ::: "memory"); break;
    case 13: asm volatile("s_waitcnt vmcnt(13)" ::: "memory"); break;
    case 14: asm volatile("s_waitcnt vmcnt(14)" ::: "memory"); break;
    case 15: asm volatile("s_waitcnt vmcnt(15)" ::: "memory"); break;
    case 16: asm volatile("s_waitcnt vmcnt(16)" ::: "memory"); break;
    case 17: asm volatile("s_waitcnt vmcnt(17)" ::: "memory"); break;
    case 18: asm volatile("s_waitcnt vmcnt(18)" ::: "memory"); break;
    case 19: asm volatile("s_waitcnt vmcnt(19)" ::: "memory"); break;
    case 20: asm volatile("s_waitcnt vmcnt(20)" ::: "memory"); break;
    case 21: asm volatile("s_waitcnt vmcnt(21)" ::: "memory"); break;
    case 22: asm volatile("s_waitcnt vmcnt(22)" ::: "memory"); break;
    case 23: asm volatile("s_waitcnt vmcnt(23)" ::: "memory"); break;
    case 24: asm volatile("s_waitcnt vmcnt(24)" ::: "memory"); break;
    case 25: asm volatile("s_waitcnt vmcnt(25)" ::: "memory"); break;
    case 26: asm volatile("s_waitcnt vmcnt(26)" ::: "memory"); break;
    case 27: asm volatile("s_waitcnt vmcnt(27)" ::: "memory"); break;
    case 28: asm volatile("s_waitcnt vmcnt(28)" ::: "memory"); break;
    case 29: asm volatile("s_waitcnt vmcnt(29)" ::: "memory"); break;
    case 30: asm volatile("s_waitcnt vmcnt(30)" ::: "memory"); break;
    case 31: asm volatile("s_waitcnt vmcnt(31)" ::: "memory"); break;
    case 32: asm volatile("s_waitcnt vmcnt(32)" ::: "memory"); break;
    case 33: asm volatile("s_waitcnt vmcnt(33)" ::: "memory"); break;
    case 34: asm volatile("s_waitcnt vmcnt(34)" ::: "memory"); break;
    case 35: asm volatile("s_waitcnt vmcnt(35)" ::: "memory"); break;
    case 36: asm volatile("s_waitcnt vmcnt(36)" ::: "memory"); break;
    case 37: asm volatile("s_waitcnt vmcnt(37)" ::: "memory"); break;
    case 38: asm volatile("s_waitcnt vmcnt(38)" ::: "memory"); break;
    case 39: asm volatile("s_waitcnt vmcnt(39)" ::: "memory"); break;
    case 40: asm volatile("s_waitcnt vmcnt(40)" ::: "memory"); break;
    case 41: asm volatile("s_waitcnt vmcnt(41)" ::: "memory"); break;
    case 42: asm volatile("s_waitcnt vmcnt(42)" ::: "memory"); break;
    case 43: asm volatile("s_waitcnt vmcnt(43)" ::: "memory"); break;
    case 44: asm volatile("s_waitcnt vmcnt(44)" ::: "memory"); break;
    case 45: asm volatile("s_waitcnt vmcnt(45)" ::: "memory"); break;
    case 46: asm volatile("s_waitcnt vmcnt(46)" ::: "memory"); break;
    case 47: asm volatile("s_waitcnt vmcnt(47)" ::: "memory"); break;
    case 48: asm volatile("s_waitcnt vmcnt(48)" ::: "memory"); break;
    case 49: asm volatile("s_waitcnt vmcnt(49)" ::: "memory"); break;
    case 50: asm volatile("s_waitcnt vmcnt(50)" ::: "memory"); break;
    case 51: asm volatile("s_waitcnt vmcnt(51)" ::: "memory"); break;
    case 52: asm volatile("s_waitcnt vmcnt(52)" ::: "memory"); break;
    case 53: asm volatile("s_waitcnt vmcnt(53)" ::: "memory"); break;
    case 54: asm volatile("s_waitcnt vmcnt(54)" ::: "memory"); break;
    case 55: asm volatile("s_waitcnt vmcnt(55)" ::: "memory"); break;
    case 56: asm volatile("s_waitcnt vmcnt(56)" ::: "memory"); break;
    case 57: asm volatile("s_waitcnt vmcnt(57)" ::: "memory"); break;
    case 58: asm volatile("s_waitcnt vmcnt(58)" ::: "memory"); break;
    case 59: asm volatile("s_waitcnt vmcnt(59)" ::: "memory"); break;
    case 60: asm volatile("s_waitcnt vmcnt(60)" ::: "memory"); break;
    case 61: asm volatile("s_waitcnt vmcnt(61)" ::: "memory"); break;
    case 62: asm volatile("s_waitcnt vmcnt(62)" ::: "memory"); break;
    case 63: asm volatile("s_waitcnt vmcnt(63)" ::: "memory"); break;
    default: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
  }
}

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
    *reinterpret_cast<u32x2*>(a.y + (size_t)m * a.N + n) =
        u32x2{pack_bf16x2(acc.x, acc.y), pack_bf16x2(acc.z, acc.w)};
  }
}

}  // namespace mk

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
#include "../capi_internal.h"

namespace {

constexpr size_t kMaxLds = 160 * 1024;

struct QPlan {
  int ks, nw, kwave, ntiles, rowblocks, wave_lds;
  int stream_steps;  // > 0: streaming kernel with this many 32-k steps per wave
  int ring;          // int8 streaming kernel: ring slots
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
// Streaming kernels: 8 waves, K = ks * 8 * 32 * S with S in {16, 8, 4}
// (int4 needs S even), N % 16 == 0.  Prefer the fewest splits that still
// give >= 192 workgroups.
bool plan_stream(int fmt, int64_t K, int64_t N, QPlan* p) {
  if (N % 16 != 0 || N < 16 || getenv("MK_QMM_GENERIC")) return false;
  const int ks_env = env_int("MK_QMM_KS", 0);
  const int steps[3] = {16, 8, 4};
  for (int ks = 1; ks <= 64; ks *= 2) {
    if (ks_env > 0 && ks != ks_env) continue;
    for (int i = 0; i < 3; ++i) {
      const int S = steps[i];
      if (K != (int64_t)ks * 8 * 32 * S) continue;
      if ((int64_t)p->ntiles * p->rowblocks * ks < 192 && ks_env <= 0 && 2 * ks <= 64 &&
          K % ((int64_t)2 * ks * 8 * 32 * 4) == 0)
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

bool plan_q(int fmt, int64_t M, int64_t K, int64_t N, QPlan* p) {
  p->ntiles = (int)((N + mk::kQCols - 1) / mk::kQCols);
  p->rowblocks = (int)((M + mk::kQRows - 1) / mk::kQRows);
  p->stream_steps = 0;
  p->ring = 0;
  if (plan_stream(fmt, K, N, p)) {
    p->part_bytes = p->ks > 1 ? (int64_t)p->rowblocks * p->ks * mk::kQRows * N * 4 : 0;
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
  p->part_bytes = p->ks > 1 ? (int64_t)p->rowblocks * p->ks * mk::kQRows * N * 4 : 0;
  return true;
}

// Kernels that need more than the default 64 KB of dynamic LDS must opt in.
hipError_t lds_opt_in(const void* fn, size_t bytes) {
  if (bytes <= 64 * 1024) return hipSuccess;
  return hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
}

hipError_t launch_reduce(int fmt, const mk::QArgs& a, hipStream_t st);

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
  if (e != hipSuccess || p.ks == 1) return e;
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
  if (e != hipSuccess || p.ks == 1) return e;
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

int run_q(int fmt, const void* x, const void* w, const void* s, const void* z, void* y, int64_t M,
          int64_t K, int64_t N, void* ws, int64_t ws_bytes, void* stream) {
  const char* fn = fmt == MK_QFMT_INT4_G64 ? "mk_int4g64_matmul_bf16" : "mk_int8pc_matmul_bf16";
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
  if (!plan_q(fmt, M, K, N, &p))
    return mkc::fail(MK_EUNSUPPORTED, "%s: no launch configuration for K=%lld", fn, (long long)K);
  if (p.part_bytes > 0 && (!ws || ws_bytes < p.part_bytes))
    return mkc::fail(MK_EWORKSPACE, "%s: workspace of %lld bytes needed, %lld given", fn,
                     (long long)p.part_bytes, (long long)ws_bytes);
  mk::QArgs a;
  a.x = static_cast<const uint16_t*>(x);
  a.w = static_cast<const uint8_t*>(w);
  a.s = s;
  a.z = static_cast<const uint8_t*>(z);
  a.y = static_cast<uint16_t*>(y);
  a.part = p.part_bytes > 0 ? static_cast<float*>(ws) : nullptr;
  a.M = (int)M;
  a.K = (int)K;
  a.N = (int)N;
  a.ks = p.ks;
  a.kwave = p.kwave;
  a.wave_lds = p.wave_lds;
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipError_t e;
  if (p.stream_steps > 0) {
    switch (p.stream_steps) {
      case 16: e = launch_stream<16>(fmt, a, p, st); break;
      case 8: e = launch_stream<8>(fmt, a, p, st); break;
      default: e = launch_stream<4>(fmt, a, p, st); break;
    }
  } else switch (p.nw) {
    case 1: e = launch_q<1>(fmt, a, p, st); break;
    case 2: e = launch_q<2>(fmt, a, p, st); break;
    case 4: e = launch_q<4>(fmt, a, p, st); break;
    default: e = launch_q<8>(fmt, a, p, st); break;
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
