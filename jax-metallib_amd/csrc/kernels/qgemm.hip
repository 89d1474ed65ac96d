// Quantized matmul for many rows (M >= 128) on gfx950: y[M, N] = x[M, K] @
// dequant(W)[K, N] in one kernel, weights read once per row tile straight
// from their packed form.
//
// Formats are those of qmatmul.hip (the workload's jnp programs; the
// reference's own quantized GEMM is quantized.py:760-958):
//   int4 g64: W uint8 [K/2, N] (low nibble = even k), scale bf16 [K/64, N],
//             zero uint8 [K/64, N]; y = x @ ((W - zero) * scale).
//   int8 pc:  W int8 [K, N], scale f32 [N]; y = x @ (W * scale).
//
// Tile: 256 rows x 128 columns per workgroup, 4 waves of 64 rows x 128
// columns each, 64 k (one int4 scale group) per step; v_mfma_f32_16x16x32_bf16,
// 4 x 8 tiles per wave (128 f32 accumulators per lane).  The x fragments go
// straight from L2 into registers and each one feeds 8 MFMAs; the earlier
// 64-column tile fed 4, and re-reading x from L2 (about 450 MB per call at
// M = 256, K = 4096, N = 14336) was what bound it.  Per step:
//   * every thread loads its share of the packed weight tile (int4: 2 packed
//     rows x 8 columns plus their 8 scales and zero points; int8: 32 bytes of
//     one k row) into registers kQgAhead steps ahead;
//   * all 256 threads dequantise the next step's tile into a bf16 [64 k][128 n]
//     LDS buffer (double-buffered), each weight once per workgroup:
//       int4: w = (q - z) * s, exact in f32 (q * s is exact inside the FMA and
//             z * s has at most 16 significant bits), then rounded to bf16;
//       int8: w exactly as bf16 (8 significant bits); the per-channel scale
//             multiplies the f32 accumulator in the epilogue instead;
//   * each wave reads its B fragments with ds_read_b64_tr_b16 (conflict-free
//     through an XOR swizzle of the 16-byte chunks); its x fragments are
//     loaded right after the MFMAs of two steps before have read that
//     register set.
// One barrier per step.  Rows past M are clamped on load and not stored.
//
// Split K.  At M = 256 the grid has 112 tiles for 256 CUs, so the K range is
// split in two (ks = 2, 224 workgroups).  Each workgroup stores its f32
// partial with device-coherent (sc1) buffer stores -- plain compiler-visible
// instructions, so the compiler keeps their data registers intact until they
// are read -- waits for their acknowledgement, and bumps the tile's arrival
// counter with a device-scope atomic; the second arriver loads the other
// partial with sc1 loads, adds it to its own (two addends: the sum does not
// depend on which one arrives last), applies the epilogue and resets the
// counter.  No workgroup waits on another.
//
// Numerics vs. the f32 reference: int8 is exact up to f32 accumulation; int4
// rounds each dequantised weight to bf16 once (relative 2^-9), well inside
// the workload's bf16 tolerance.
#include "common.h"
#include "epilogue.h"
#include "qgemm.h"

#include <stdlib.h>

#include <algorithm>

namespace mk {

constexpr int kQgRows = 256;
constexpr int kQgCols = 128;
constexpr int kQgAhead = 3;                // weight loads run this many steps ahead
constexpr int kQgBuf = 64 * kQgCols * 2;   // bf16 [64 k][128 n] tile
constexpr int kQgPart = kQgRows * kQgCols;  // f32 per partial tile

struct QgArgs {
  const uint16_t* x;
  const uint8_t* w;
  const void* s;
  const uint8_t* z;
  uint16_t* y;
  const uint16_t* aux;  // epilogue operand or null
  int epi;
  int M, K, N;
  int ks;          // K split (1 or 2)
  float* part;     // ks > 1: partial tiles [tile][ks][32][256 threads][4]
  uint32_t* cnt;   // ks > 1: per-tile arrival counters (zero between calls)
  int xch_local;   // ks > 1: every tile's K parts run on one XCD (exchange in its L2)
};

typedef short qg_s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) qg_s16x4* qg_lds_s16x4_ptr;

// Chunk swizzle of the bf16 tile (rows of 256 B = 16 chunks of 16 B): chunk
// c of k row k sits at c ^ (2 (k % 4) + 8 (k / 8 % 2)).  A transposing read
// (k rows 8g + r (+4), g, r < 4; two chunks per row) then uses every bank
// exactly twice, and a dequantisation store (4 rows x 16 chunks) four times.
__device__ __forceinline__ int qg_swz(int k, int c) { return c ^ ((2 * (k & 3)) | (((k >> 3) & 1) << 3)); }

// Two floats to bf16 (RNE) in one v_cvt_pk_bf16_f32, lo in the low half.
typedef float qg_f2 __attribute__((ext_vector_type(2)));
typedef __bf16 qg_b2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t qg_pack(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((qg_f2){lo, hi}, qg_b2));
}

// One thread's share of a step's packed weights.
//   int4: packed rows 2 pp, 2 pp + 1 at columns 8 cq .. +7 (w0, w1), their 8
//         bf16 scales (s) and 8 zero points (z).
//   int8: 32 bytes of k row kr at columns 32 cc .. +31 (v0, v1).
struct QgW {
  u32x2 w0, w1, z;
  u32x4 s;
  u32x4 v0, v1;
};

// Dequantise one step's share of thread `pt` (0..255) of the weights in r
// into the bf16 [64 k][128 n] tile dst (swizzled):
//   int4: rows k = 4 pp + {0..3} (pp = pt / 16) at columns 8 cq .. +7
//         (cq = pt % 16): w = (q - z) * s, exact in f32 (q * s is exact
//         inside the FMA and z * s has at most 16 significant bits), then
//         rounded to bf16;
//   int8: row kr = pt / 4 at columns 32 cc .. +31 (cc = pt % 4): w exactly
//         as bf16 (8 significant bits).
template <bool INT4>
__device__ __forceinline__ void qg_dequant(unsigned char* dst, const QgW& r, int pt) {
  const int pp = pt >> 4, cq = pt & 15;
  const int kr = pt >> 2, cc = pt & 3;
  if (INT4) {
    float s[8], s16[8], zs[8];
    const uint32_t sw[4] = {r.s.x, r.s.y, r.s.z, r.s.w};
    const uint32_t zw[2] = {r.z.x, r.z.y};
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      s[c] = bf16_to_f32((sw[c >> 1] >> (16 * (c & 1))) & 0xffffu);
      s16[c] = s[c] * 0.0625f;
      zs[c] = (float)((zw[c >> 2] >> (8 * (c & 3))) & 0xffu) * s[c];
    }
    // Rows k = 4 pp + {0, 1, 2, 3}: low / high nibbles of packed rows 2 pp
    // and 2 pp + 1.  High nibbles are converted as 16 q and scaled by s/16.
    uint32_t lo[4] = {r.w0.x & 0x0f0f0f0fu, r.w0.y & 0x0f0f0f0fu, r.w1.x & 0x0f0f0f0fu, r.w1.y & 0x0f0f0f0fu};
    uint32_t hi[4] = {r.w0.x & 0xf0f0f0f0u, r.w0.y & 0xf0f0f0f0u, r.w1.x & 0xf0f0f0f0u, r.w1.y & 0xf0f0f0f0u};
    // Keep the masked words as they are, so each byte converts with one
    // v_cvt_f32_ubyteN instead of a bit-field extract and a convert.
    asm volatile("" : "+v"(lo[0]), "+v"(lo[1]), "+v"(lo[2]), "+v"(lo[3]));
    asm volatile("" : "+v"(hi[0]), "+v"(hi[1]), "+v"(hi[2]), "+v"(hi[3]));
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int wsel = 2 * (kk >> 1);  // words of packed row 2 pp + kk / 2
      float v[8];
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const uint32_t src = (kk & 1) ? hi[wsel + (c >> 2)] : lo[wsel + (c >> 2)];
        const float q = (float)((src >> (8 * (c & 3))) & 0xffu);
        v[c] = __builtin_fmaf(q, (kk & 1) ? s16[c] : s[c], -zs[c]);
      }
      const int k = 4 * pp + kk;
      *reinterpret_cast<u32x4*>(dst + 256 * k + 16 * qg_swz(k, cq)) =
          u32x4{qg_pack(v[0], v[1]), qg_pack(v[2], v[3]), qg_pack(v[4], v[5]), qg_pack(v[6], v[7])};
    }
  } else {
    const uint32_t wv[8] = {r.v0.x, r.v0.y, r.v0.z, r.v0.w, r.v1.x, r.v1.y, r.v1.z, r.v1.w};
#pragma unroll
    for (int h = 0; h < 4; ++h) {  // chunk 4 cc + h: columns 32 cc + 8 h .. +7
      uint32_t o[4];
#pragma unroll
      for (int d = 0; d < 2; ++d) {
        const uint32_t b = wv[2 * h + d] ^ 0x80808080u;  // w + 128 as u8
        float f[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) f[e] = (float)((b >> (8 * e)) & 0xffu) - 128.0f;
        o[2 * d] = qg_pack(f[0], f[1]);
        o[2 * d + 1] = qg_pack(f[2], f[3]);
      }
      *reinterpret_cast<u32x4*>(dst + 256 * kr + 16 * qg_swz(kr, 4 * cc + h)) = u32x4{o[0], o[1], o[2], o[3]};
    }
  }
}

template <bool INT4>
__global__ __launch_bounds__(256) void qgemm_kernel(QgArgs a) {
  constexpr int P = kQgAhead;
  __shared__ __attribute__((aligned(16))) unsigned char bbuf[2][kQgBuf];
  __shared__ uint32_t last_flag;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int N = a.N, K = a.K, M = a.M;
  const int tiles_n = N / kQgCols, tiles_m = (M + kQgRows - 1) / kQgRows;
  // Logical id -> (column tile, row tile, K part): the row tiles of one
  // column tile (which read the same weights) and the K parts of one tile
  // are consecutive, and xcd_logical_id keeps consecutive ids on one XCD.
  const uint32_t L = xcd_logical_id(blockIdx.x, gridDim.x);
  const int ksi = (int)(L % (uint32_t)a.ks);
  const int tile = (int)(L / (uint32_t)a.ks);
  const int tn = tile / tiles_m, tm = tile - tn * tiles_m;
  const int m0 = tm * kQgRows, n0 = tn * kQgCols;
  const int KT = K / a.ks / 64;       // steps of this workgroup
  const int kt0 = ksi * KT;           // its first step (64-k group)

  // ---- weight loads (steps past the end reload the last one).  Every
  //      address is a wave-uniform per-step base plus a per-lane 32-bit byte
  //      offset. ----
  const int pp = tid >> 4, cq = tid & 15;  // int4
  const int kr = tid >> 2, cc = tid & 3;   // int8
  const uint32_t woff = INT4 ? (uint32_t)(2 * pp * N + n0 + 8 * cq) : (uint32_t)(kr * N + n0 + 32 * cc);
  const uint32_t soff = (uint32_t)(2 * (n0 + 8 * cq)), zoff = (uint32_t)(n0 + 8 * cq);
  auto load_w = [&](int st, QgW& r) {
    st = kt0 + (st < KT ? st : KT - 1);
    if (INT4) {
      const uint32_t o = (uint32_t)st * (uint32_t)(32 * N) + woff;
      r.w0 = *reinterpret_cast<const u32x2*>(a.w + o);
      r.w1 = *reinterpret_cast<const u32x2*>(a.w + (o + (uint32_t)N));
      r.s = *reinterpret_cast<const u32x4*>(static_cast<const uint8_t*>(a.s) + ((uint32_t)st * (uint32_t)(2 * N) + soff));
      r.z = *reinterpret_cast<const u32x2*>(a.z + ((uint32_t)st * (uint32_t)N + zoff));
    } else {
      const uint32_t o = (uint32_t)st * (uint32_t)(64 * N) + woff;
      r.v0 = *reinterpret_cast<const u32x4*>(a.w + o);
      r.v1 = *reinterpret_cast<const u32x4*>(a.w + o + 16);
    }
  };

  // ---- x fragments: tile i, half hh: row m0 + 64 wave + 16 i + lane%16,
  //      k = 64 (kt0 + t) + 32 hh + 8 (lane/16) .. +7 ----
  uint32_t xoff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = std::min(m0 + 64 * wave + 16 * i + (lane & 15), M - 1);
    xoff[i] = (uint32_t)(2 * (r * K + 64 * kt0 + 8 * (lane >> 4)));
  }
  auto load_x = [&](int t, u32x4 (&xa)[8]) {
    t = t < KT ? t : KT - 1;
    const uint8_t* xb = reinterpret_cast<const uint8_t*>(a.x);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t o = (uint32_t)t * 128u + xoff[i];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) xa[4 * hh + i] = *reinterpret_cast<const u32x4*>(xb + o + 64 * hh);
    }
  };

  // ---- dequantisation of one step into bbuf[t & 1] ----
  auto dequant = [&](int t, const QgW& r) {
    qg_dequant<INT4>(bbuf[t & 1], r, tid);
  };

  // ---- B fragment offsets: tile j; the k half h of 32-row block hh adds
  //      the uniform 256 (32 hh + 4 h).  The swizzle term depends only on
  //      bits of the lane's k row 8g + r that 32 hh + 4 h does not change. ----
  int boff[8];
  {
    const int g = lane >> 4, r = (lane & 15) >> 2, q = lane & 3;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int k = 8 * g + r, col = 16 * j + 4 * q;
      boff[j] = 256 * k + 16 * qg_swz(k, col >> 3) + 2 * (col & 7);
    }
  }

  f32x4 acc[4][8];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Both k halves' B fragments are read up front, so the second half's LDS
  // latency runs under the first half's MFMAs.
  auto mma = [&](int t, const u32x4 (&xa)[8]) {
    const unsigned char* b = bbuf[t & 1];
    u32x4 bf[2][8];
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const qg_s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((qg_lds_s16x4_ptr)(b + boff[j] + 8192 * hh));
        const qg_s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((qg_lds_s16x4_ptr)(b + boff[j] + 8192 * hh + 1024));
        const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
        bf[hh][j] = u32x4{l2.x, l2.y, h2.x, h2.y};
      }
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] = mfma16x16x32(bf[hh][j], xa[4 * hh + i], acc[i][j]);
  };

  // ---- prologue: weights of steps 0 .. P-1, x of steps 0 and 1, step 0
  //      dequantised ----
  QgW wr[P];
#pragma unroll
  for (int u = 0; u < P; ++u) load_w(u, wr[u]);
  u32x4 xa[2][8];
  load_x(0, xa[0]);
  load_x(1, xa[1]);
  dequant(0, wr[0]);
  load_w(P, wr[0]);

  // Iteration t: barrier (bbuf[t & 1] complete, bbuf[(t + 1) & 1] free);
  // MFMAs of step t, then x of step t + 2 into the registers they read;
  // dequantise step t + 1 (its VALU work overlaps the MFMAs) and load the
  // weights of step t + 1 + P into its register set.  The loads and the
  // dequantisation run unconditionally (past the end they repeat the last
  // step, into a buffer nobody reads): with no branch in the loop body the
  // compiler's wait counts see the full prefetch distance.
  auto iter = [&](int t, QgW& wn, u32x4 (&xc)[8]) {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    mma(t, xc);
    load_x(t + 2, xc);
    dequant(t + 1, wn);
    load_w(t + 1 + P, wn);
  };
  static_assert(P == 3, "the main loop is unrolled for 3 weight and 2 x register sets");
  int t = 0;
  for (; t + 6 <= KT; t += 6) {
    iter(t, wr[1], xa[0]);
    iter(t + 1, wr[2], xa[1]);
    iter(t + 2, wr[0], xa[0]);
    iter(t + 3, wr[1], xa[1]);
    iter(t + 4, wr[2], xa[0]);
    iter(t + 5, wr[0], xa[1]);
  }
  // The same sequence for the last KT % 6 steps.
  if (t < KT) iter(t, wr[1], xa[0]);
  if (t + 1 < KT) iter(t + 1, wr[2], xa[1]);
  if (t + 2 < KT) iter(t + 2, wr[0], xa[0]);
  if (t + 3 < KT) iter(t + 3, wr[1], xa[1]);
  if (t + 4 < KT) iter(t + 4, wr[2], xa[0]);

  // ---- split K: exchange the partials ----
  if (a.ks > 1) {
    // Partial (i, j) of thread tid at float offset 4 * ((32 ksi + 8 i + j) * 256 + tid)
    // of the tile's region; every store and load below stays inside it
    // (the resource's size bounds the accesses as well).
    float* tp = a.part + (size_t)tile * a.ks * kQgPart;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(tp, 0, a.ks * kQgPart * 4, kBufWord3);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc[i][j]), rs,
                                               ((32 * ksi + 8 * i + j) * 256 + tid) * 16, 0, kSc1);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // every partial store acknowledged
    __syncthreads();
    if (tid == 0) {
      uint32_t* ctr = a.cnt + tile;
      asm volatile("" : "+v"(ctr));  // per-lane address: a vector atomic
      // Local exchange: both K parts run on this XCD, so the atomic is
      // performed in its L2 at workgroup scope; otherwise at device scope.
      const uint32_t old = a.xch_local ? __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)
                                       : __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const uint32_t last = old == (uint32_t)(a.ks - 1);
      if (last) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      last_flag = last;
    }
    __syncthreads();
    if (!last_flag) return;
    // The other partial (ks == 2), added to ours.  Device scope: sc1 loads
    // (they miss this XCD's L2).  Local: loads the L2 serves -- this CU's L1
    // holds no line of the tile's partials (it starts the kernel
    // invalidated and only the tile's second arriver loads them, once).
    const int other = 1 - ksi;
    if (a.xch_local) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rs, ((32 * other + 8 * i + j) * 256 + tid) * 16, 0, 0);
          acc[i][j] += __builtin_bit_cast(f32x4, v);
        }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rs, ((32 * other + 8 * i + j) * 256 + tid) * 16, 0,
                                                                kSc1);
          acc[i][j] += __builtin_bit_cast(f32x4, v);
        }
    }
  }

  // ---- epilogue: lane owns row m, columns n .. n + 3 of each tile ----
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = m0 + 64 * wave + 16 * i + (lane & 15);
    if (m >= M) continue;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int n = n0 + 16 * j + 4 * (lane >> 4);
      f32x4 v = acc[i][j];
      if (!INT4) {
        const f32x4 sc = *reinterpret_cast<const f32x4*>(static_cast<const float*>(a.s) + n);
        v = f32x4{v.x * sc.x, v.y * sc.y, v.z * sc.z, v.w * sc.w};
      }
      epi_store_bf16x4(a.y, a.aux, a.epi, (size_t)m * N + n, v);
    }
  }
}

// ---------------------------------------------------------------------------
// Warp-specialised variant: the same tile (256 rows x 128 columns), steps,
// B swizzle, dequantisation and MFMA order as qgemm_kernel -- the results
// are bit-identical -- with 8 waves.  Waves 0-3 (consumers) hold the
// accumulators and do nothing but read fragments from LDS and issue MFMAs;
// waves 4-7 (producers) stream every operand by LDS DMA and dequantise.  The
// dispatcher puts wave w on SIMD w % 4, so each SIMD runs one consumer and
// one producer, and the producer's VALU work overlaps the consumer's MFMAs
// (the one-wave-per-SIMD kernel above serialises them).  LDS:
//   bbuf [2][64 k][128 n] bf16    the dequantised weights (as above)
//   xbuf [3][256 rows][64 k] bf16 x, 16-byte chunk q of row r at q ^ (r & 7)
//                                 (conflict-free 16-byte fragment reads)
//   wst  [4 producers][2][...]    each producer's own share of the packed
//                                 weights, scales and zero points
// Iteration t (between barriers): consumers multiply step t (bbuf[t % 2],
// xbuf[t % 3]); producers issue the DMAs of step t + 2, wait for their own
// DMAs of step t + 1, and dequantise it into bbuf[(t + 1) % 2].  Every DMA a
// producer waits for is its own (it dequantises exactly the weights it
// fetched), so the one barrier per step is the only cross-wave
// synchronisation, as in the kernel above.
// ---------------------------------------------------------------------------
constexpr int kQgXBuf = kQgRows * 64 * 2;  // bf16 x [256 rows][64 k]
constexpr int kQgWSt = 2048 + 512;         // packed weights (int4 1 KB, int8 2 KB) + scales 256 B + zeros 128 B
constexpr int kQgWsLds = 2 * kQgBuf + 3 * kQgXBuf + 4 * 2 * kQgWSt + 16 + kQgCols * 4;

template <bool INT4>
__global__ __launch_bounds__(512) void qgemm_ws_kernel(QgArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  unsigned char* bbuf = smem;                      // [2][kQgBuf]
  unsigned char* xbuf = smem + 2 * kQgBuf;         // [3][kQgXBuf]
  unsigned char* wst = xbuf + 3 * kQgXBuf;         // [4][2][kQgWSt]
  volatile uint32_t* last_flag = reinterpret_cast<volatile uint32_t*>(wst + 4 * 2 * kQgWSt);
  float* scl = reinterpret_cast<float*>(wst + 4 * 2 * kQgWSt + 16);  // int8: the tile's per-channel scales

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const bool producer = wave >= 4;
  const int N = a.N, K = a.K, M = a.M;
  const int tiles_m = (M + kQgRows - 1) / kQgRows;
  const uint32_t L = xcd_logical_id(blockIdx.x, gridDim.x);
  const int ksi = (int)(L % (uint32_t)a.ks);
  const int tile = (int)(L / (uint32_t)a.ks);
  const int tn = tile / tiles_m, tm = tile - tn * tiles_m;
  const int m0 = tm * kQgRows, n0 = tn * kQgCols;
  const int KT = K / a.ks / 64;
  const int kt0 = ksi * KT;

  f32x4 acc[4][8];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  if (producer) {
    // ---- producers: every operand by LDS DMA, then the dequantisation ----
    const int pw = wave - 4;   // producer index
    const int pt = tid - 256;  // producer thread 0..255
    unsigned char* mywst = wst + pw * 2 * kQgWSt;
    const int xq = (lane & 7) ^ (lane >> 3);  // x chunk of this lane (row & 7 == lane / 8)
    const uint8_t* xbase = reinterpret_cast<const uint8_t*>(a.x) + 2 * ((size_t)64 * kt0 + 8 * xq);
    // weights: int4 packed rows 8 pw .. +7 (1 KB), int8 k rows 16 pw .. +15
    // (2 KB), natural layout; int4 scales (256 B) and zero points (128 B).
    const uint8_t* wsrc = a.w + (size_t)((INT4 ? 8 : 16) * pw + (lane >> 3)) * N + n0 + 16 * (lane & 7) +
                          (size_t)kt0 * (INT4 ? 32 * N : 64 * N);
    const uint8_t* szsrc = lane < 16 ? static_cast<const uint8_t*>(a.s) + 2 * ((size_t)kt0 * N + n0) + 16 * lane
                                     : a.z + ((size_t)kt0 * N + n0) + 16 * (lane - 16);
    // DMAs of step st into stage buffer st % 2 and
    // xbuf[st % 3]: 8 of x (rows 64 pw + 8 d + lane / 8, position lane % 8
    // holding chunk xq) and 2 of weights (int4: weights, scales and zero
    // points; int8: weights).
    auto issue = [&](int st) {
      unsigned char* xb = xbuf + (st % 3) * kQgXBuf + (64 * pw) * 128;
#pragma unroll
      for (int d = 0; d < 8; ++d) {
        const int r = std::min(m0 + 64 * pw + 8 * d + (lane >> 3), M - 1);
        dma16(xbase + 2 * (size_t)r * K + (size_t)st * 128, xb + d * 1024);
      }
      unsigned char* wb = mywst + (st & 1) * kQgWSt;
      if (INT4) {
        dma16(wsrc + (size_t)st * 32 * N, wb);
        if (lane < 24) dma16(szsrc + (size_t)st * (lane < 16 ? 2 * N : N), wb + 2048);
      } else {
        dma16(wsrc + (size_t)st * 64 * N, wb);
        dma16(wsrc + (size_t)st * 64 * N + (size_t)8 * N, wb + 1024);
      }
    };
    // Read this thread's share of stage st % 2 and dequantise it.
    auto dequant = [&](int st) {
      const unsigned char* wb = mywst + (st & 1) * kQgWSt;
      QgW r;
      if (INT4) {
        const int ppl = (pt >> 4) & 3, cq = pt & 15;  // packed rows 2 ppl, 2 ppl + 1 of this producer's 8
        r.w0 = *reinterpret_cast<const u32x2*>(wb + (2 * ppl) * 128 + 8 * cq);
        r.w1 = *reinterpret_cast<const u32x2*>(wb + (2 * ppl + 1) * 128 + 8 * cq);
        r.s = *reinterpret_cast<const u32x4*>(wb + 2048 + 16 * cq);
        r.z = *reinterpret_cast<const u32x2*>(wb + 2048 + 256 + 8 * cq);
      } else {
        const int krl = (pt >> 2) & 15, cc = pt & 3;  // k row of this producer's 16, 32 columns
        r.v0 = *reinterpret_cast<const u32x4*>(wb + krl * 128 + 32 * cc);
        r.v1 = *reinterpret_cast<const u32x4*>(wb + krl * 128 + 32 * cc + 16);
      }
      qg_dequant<INT4>(bbuf + (st & 1) * kQgBuf, r, pt);
    };
    constexpr int kDmaPerStep = 10;  // 8 for x, 2 for the weights (the DMA counter is per wave)
    issue(0);
    if (KT > 1) issue(1);
    vm_wait(KT > 1 ? kDmaPerStep : 0);  // own DMAs of step 0 landed (step 1's may not have)
    dequant(0);
    for (int t = 0; t < KT; ++t) {
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      if (t + 2 < KT) issue(t + 2);
      vm_wait(t + 2 < KT ? kDmaPerStep : 0);  // own DMAs of step t + 1 landed
      if (t + 1 < KT) dequant(t + 1);
    }
  } else {
    // ---- consumers: fragments from LDS, MFMAs ----
    // int8: the tile's 128 per-channel scales go to LDS now, so the epilogue
    // reads them from LDS instead of loading them after the exchange (many
    // barriers separate this write from those reads).
    if (!INT4 && wave == 0 && lane < kQgCols / 4)
      *reinterpret_cast<f32x4*>(scl + 4 * lane) =
          *reinterpret_cast<const f32x4*>(static_cast<const float*>(a.s) + n0 + 4 * lane);
    // B fragment of column block j: k row 8 g + r (g = lane / 16,
    // r = lane % 16 / 4), columns 16 j + 4 q .. +3 (q = lane % 4); the
    // swizzled address is bbase ^ (32 j) (the bits of 32 j and of the
    // lane's swizzle term do not overlap any other part of the address).
    uint32_t bbase;
    {
      const int g = lane >> 4, r = (lane & 15) >> 2, q = lane & 3;
      const int k = 8 * g + r, col = 4 * q;
      bbase = (uint32_t)(256 * k + 16 * qg_swz(k, col >> 3) + 2 * (col & 7));
    }
    // x fragment (row block i, k half hh): row 64 wave + 16 i + lane % 16,
    // chunk 4 hh + lane / 16 at position chunk ^ (lane % 8).
    const uint32_t xrow = (uint32_t)((64 * wave + (lane & 15)) * 128);
    const uint32_t xpos0 = 16u * (uint32_t)((lane >> 4) ^ (lane & 7)), xpos1 = 16u * (uint32_t)((4 + (lane >> 4)) ^ (lane & 7));
    for (int t = 0; t < KT; ++t) {
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      const unsigned char* b = bbuf + (t & 1) * kQgBuf;
      const unsigned char* xb = xbuf + (t % 3) * kQgXBuf;
      u32x4 bf[2][8], xa[8];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const uint32_t o = (bbase ^ (uint32_t)(32 * j)) + 8192u * hh;
          const qg_s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((qg_lds_s16x4_ptr)(b + o));
          const qg_s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((qg_lds_s16x4_ptr)(b + o + 1024));
          const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
          bf[hh][j] = u32x4{l2.x, l2.y, h2.x, h2.y};
        }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        xa[i] = *reinterpret_cast<const u32x4*>(xb + xrow + 2048 * i + xpos0);
        xa[4 + i] = *reinterpret_cast<const u32x4*>(xb + xrow + 2048 * i + xpos1);
      }
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 8; ++j) acc[i][j] = mfma16x16x32(bf[hh][j], xa[4 * hh + i], acc[i][j]);
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // ---- split K: exchange the partials (consumers' threads 0..255 hold them) ----
  if (a.ks > 1) {
    float* tp = a.part + (size_t)tile * a.ks * kQgPart;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(tp, 0, a.ks * kQgPart * 4, kBufWord3);
    if (!producer) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j)
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc[i][j]), rs,
                                                 ((32 * ksi + 8 * i + j) * 256 + tid) * 16, 0, kSc1);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // every partial store acknowledged
    }
    __syncthreads();
    if (tid == 0) {
      uint32_t* ctr = a.cnt + tile;
      asm volatile("" : "+v"(ctr));  // per-lane address: a vector atomic
      const uint32_t old = a.xch_local ? __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)
                                       : __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const uint32_t last = old == (uint32_t)(a.ks - 1);
      if (last) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      *last_flag = last;
    }
    __syncthreads();
    if (!*last_flag || producer) return;
    const int other = 1 - ksi;
    const int pol = a.xch_local ? 0 : kSc1;  // local: the L2 serves it (first touch on this CU)
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const u32x4 v = pol ? __builtin_amdgcn_raw_buffer_load_b128(rs, ((32 * other + 8 * i + j) * 256 + tid) * 16, 0, kSc1)
                            : __builtin_amdgcn_raw_buffer_load_b128(rs, ((32 * other + 8 * i + j) * 256 + tid) * 16, 0, 0);
        acc[i][j] += __builtin_bit_cast(f32x4, v);
      }
  }
  if (producer) return;

  // ---- epilogue: lane owns row m, columns n .. n + 3 of each tile ----
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = m0 + 64 * wave + 16 * i + (lane & 15);
    if (m >= M) continue;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int n = n0 + 16 * j + 4 * (lane >> 4);
      f32x4 v = acc[i][j];
      if (!INT4) {
        const f32x4 sc = *reinterpret_cast<const f32x4*>(scl + (n - n0));
        v = f32x4{v.x * sc.x, v.y * sc.y, v.z * sc.z, v.w * sc.w};
      }
      epi_store_bf16x4(a.y, a.aux, a.epi, (size_t)m * N + n, v);
    }
  }
}

}  // namespace mk

namespace mkq {

unsigned qgemm_grid(int64_t M, int64_t N, int ks) {
  return (unsigned)(((M + mk::kQgRows - 1) / mk::kQgRows) * (N / mk::kQgCols) * ks);
}

bool qgemm_tile_on_one_xcd(unsigned gx, int ks) {
  // xcd_logical_id runs of gx / 8 consecutive ids share an XCD when the
  // dispatcher deals round-robin; a tile's ks consecutive ids stay in one run.
  return gx % 8 == 0 && (gx / 8) % (unsigned)ks == 0;
}

bool qgemm_supported(int64_t M, int64_t K, int64_t N) {
  // Per-lane offsets are 32-bit: the weight matrix and x stay under 2 GiB.
  return M >= 1 && K >= 64 && K % 64 == 0 && N >= mk::kQgCols && N % mk::kQgCols == 0 &&
         K * N < ((int64_t)1 << 31) && M * K * 2 < ((int64_t)1 << 31);
}

int qgemm_ks(int64_t M, int64_t K, int64_t N, int64_t workspace_cap) {
  const int64_t tiles = ((M + mk::kQgRows - 1) / mk::kQgRows) * (N / mk::kQgCols);
  const char* env = getenv("MK_QG_KS");
  int ks = (tiles < 192 && K % 128 == 0 && K >= 256) ? 2 : 1;
  if (env && (env[0] == '1' || env[0] == '2') && env[1] == '\0') ks = env[0] - '0';
  if (ks == 2 && (K % 128 != 0 || tiles > kQgCounters || qgemm_workspace_bytes(M, K, N, 2) > workspace_cap)) ks = 1;
  return ks;
}

int64_t qgemm_workspace_bytes(int64_t M, int64_t K, int64_t N, int ks) {
  if (ks <= 1) return 0;
  const int64_t tiles = ((M + mk::kQgRows - 1) / mk::kQgRows) * (N / mk::kQgCols);
  return kQgPartOffset + tiles * ks * mk::kQgPart * 4;
}

hipError_t qgemm_launch(bool int4, const void* x, const void* w, const void* s, const void* z, void* y, int64_t M,
                        int64_t K, int64_t N, const void* aux, int epi, int ks, void* workspace,
                        hipStream_t stream, bool xch_local) {
  mk::QgArgs a;
  a.x = static_cast<const uint16_t*>(x);
  a.w = static_cast<const uint8_t*>(w);
  a.s = s;
  a.z = static_cast<const uint8_t*>(z);
  a.y = static_cast<uint16_t*>(y);
  a.aux = static_cast<const uint16_t*>(aux);
  a.epi = epi;
  a.M = (int)M;
  a.K = (int)K;
  a.N = (int)N;
  a.ks = ks;
  a.cnt = ks > 1 ? static_cast<uint32_t*>(workspace) : nullptr;
  a.part = ks > 1 ? reinterpret_cast<float*>(static_cast<unsigned char*>(workspace) + kQgPartOffset) : nullptr;
  const dim3 grid(qgemm_grid(M, N, ks));
  a.xch_local = ks > 1 && xch_local && qgemm_tile_on_one_xcd(grid.x, ks);
  const char* ws_env = getenv("MK_QG_WS");
  if (!(ws_env && ws_env[0] == '0')) {
    // Warp-specialised kernel (8 waves, 140 KB of LDS).
    const void* fn = int4 ? (const void*)mk::qgemm_ws_kernel<true> : (const void*)mk::qgemm_ws_kernel<false>;
    hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, mk::kQgWsLds);
    if (e != hipSuccess) return e;
    if (int4)
      hipLaunchKernelGGL(mk::qgemm_ws_kernel<true>, grid, dim3(512), mk::kQgWsLds, stream, a);
    else
      hipLaunchKernelGGL(mk::qgemm_ws_kernel<false>, grid, dim3(512), mk::kQgWsLds, stream, a);
    return hipGetLastError();
  }
  if (int4)
    hipLaunchKernelGGL(mk::qgemm_kernel<true>, grid, dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL(mk::qgemm_kernel<false>, grid, dim3(256), 0, stream, a);
  return hipGetLastError();
}

}  // namespace mkq
