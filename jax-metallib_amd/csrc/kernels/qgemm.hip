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
// Tile: 256 rows x 64 columns per workgroup, 4 waves of 64 rows each, 64 k
// (one int4 scale group) per step; v_mfma_f32_16x16x32_bf16, 4 x 4 tiles per
// wave.  Per step:
//   * every thread loads its share of the packed weight tile (int4: 2 packed
//     rows x 4 columns plus their 4 scales and zero points; int8: 16 bytes of
//     one k row) into registers kQgAhead steps ahead -- plain loads, so the
//     compiler's own wait counts cover them;
//   * all 256 threads dequantise the next step's tile into a bf16 [64 k][64 n]
//     LDS buffer (double-buffered), each weight once per workgroup:
//       int4: w = (q - z) * s, exact in f32 (q * s is exact inside the FMA and
//             z * s has at most 16 significant bits), then rounded to bf16;
//       int8: w exactly as bf16 (8 significant bits); the per-channel scale
//             multiplies the f32 accumulator in the epilogue instead;
//   * each wave reads its B fragments with ds_read_b64_tr_b16 (conflict-free
//     through an XOR swizzle of the 16-byte chunks); its x fragments come
//     straight from global memory into registers, loaded right after the
//     MFMAs of two steps before have read that register set (x is shared by
//     every workgroup of a row tile, so it is mostly served from L2).
// One barrier per step.  Rows past M are clamped on load and not stored.
//
// Numerics vs. the f32 reference: int8 is exact up to f32 accumulation; int4
// rounds each dequantised weight to bf16 once (relative 2^-9), well inside
// the workload's bf16 tolerance.
#include "common.h"
#include "epilogue.h"
#include "qgemm.h"

#include <algorithm>

namespace mk {

constexpr int kQgAhead = 3;      // weight loads run this many steps ahead
constexpr int kQgBuf = 64 * 128;  // bf16 [64 k][64 n] tile

struct QgArgs {
  const uint16_t* x;
  const uint8_t* w;
  const void* s;
  const uint8_t* z;
  uint16_t* y;
  const uint16_t* aux;  // epilogue operand or null
  int epi;
  int M, K, N;
};

typedef short qg_s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) qg_s16x4* qg_lds_s16x4_ptr;

// Chunk swizzle of the bf16 tile (rows of 128 B = 8 chunks of 16 B).  With
// it the 64 lanes of one ds_read_b64_tr_b16 (k rows 8g + r (+4), g, r < 4)
// touch every bank exactly twice.
__device__ __forceinline__ int qg_swz(int k, int c) { return c ^ ((((k >> 1) & 1) << 1) | (((k >> 3) & 1) << 2)); }

// Two floats to bf16 (RNE) in one v_cvt_pk_bf16_f32, lo in the low half.
typedef float qg_f2 __attribute__((ext_vector_type(2)));
typedef __bf16 qg_b2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t qg_pack(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((qg_f2){lo, hi}, qg_b2));
}

// One thread's share of a step's packed weights.
//   int4: packed rows 2 pp, 2 pp + 1 at columns 4 cq .. +3 (w0, w1), the 4
//         bf16 scales (s) and 4 zero points (z) of those columns.
//   int8: 16 bytes of k row kr at columns 16 cc .. +15 (v).
struct QgW {
  uint32_t w0, w1, z;
  u32x2 s;
  u32x4 v;
};

template <bool INT4>
__global__ __launch_bounds__(256) void qgemm_kernel(QgArgs a) {
  constexpr int P = kQgAhead;
  __shared__ __attribute__((aligned(16))) unsigned char bbuf[2][kQgBuf];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int N = a.N, K = a.K, M = a.M;
  const int tiles_n = N / 64;
  const uint32_t L = xcd_logical_id(blockIdx.x, gridDim.x);
  const int tm = (int)L / tiles_n, tn = (int)L - tm * tiles_n;
  const int m0 = tm * 256, n0 = tn * 64;
  const int KT = K / 64;

  // ---- weight loads (steps past the end reload the last one).  Every
  //      address is a wave-uniform per-step base plus a per-lane 32-bit byte
  //      offset, so the per-step work is scalar. ----
  const int pp = tid >> 4, cq = tid & 15;  // int4
  const int kr = tid >> 2, cc = tid & 3;   // int8
  const uint32_t woff = INT4 ? (uint32_t)(2 * pp * N + n0 + 4 * cq) : (uint32_t)(kr * N + n0 + 16 * cc);
  const uint32_t soff = (uint32_t)(2 * (n0 + 4 * cq)), zoff = (uint32_t)(n0 + 4 * cq);
  auto load_w = [&](int st, QgW& r) {
    st = st < KT ? st : KT - 1;
    if (INT4) {
      const uint32_t o = (uint32_t)st * (uint32_t)(32 * N) + woff;
      r.w0 = *reinterpret_cast<const uint32_t*>(a.w + o);
      r.w1 = *reinterpret_cast<const uint32_t*>(a.w + (o + (uint32_t)N));
      r.s = *reinterpret_cast<const u32x2*>(static_cast<const uint8_t*>(a.s) + ((uint32_t)st * (uint32_t)(2 * N) + soff));
      r.z = *reinterpret_cast<const uint32_t*>(a.z + ((uint32_t)st * (uint32_t)N + zoff));
    } else {
      r.v = *reinterpret_cast<const u32x4*>(a.w + ((uint32_t)st * (uint32_t)(64 * N) + woff));
    }
  };

  // ---- x fragments: tile i, half hh: row m0 + 64 wave + 16 i + lane%16,
  //      k = 64 t + 32 hh + 8 (lane/16) .. +7 ----
  uint32_t xoff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = std::min(m0 + 64 * wave + 16 * i + (lane & 15), M - 1);
    xoff[i] = (uint32_t)(2 * (r * K + 8 * (lane >> 4)));
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
    unsigned char* dst = bbuf[t & 1];
    if (INT4) {
      float s[4], s16[4], zs[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const uint32_t sb = (c < 2 ? r.s.x : r.s.y) >> (16 * (c & 1));
        s[c] = bf16_to_f32(sb & 0xffffu);
        s16[c] = s[c] * 0.0625f;
        zs[c] = (float)((r.z >> (8 * c)) & 0xffu) * s[c];
      }
      // Rows k = 4 pp + {0, 1, 2, 3}: low / high nibbles of packed rows 2 pp
      // and 2 pp + 1.  High nibbles are converted as 16 q and scaled by s/16.
      uint32_t lo[2] = {r.w0 & 0x0f0f0f0fu, r.w1 & 0x0f0f0f0fu};
      uint32_t hi[2] = {r.w0 & 0xf0f0f0f0u, r.w1 & 0xf0f0f0f0u};
      // Keep the masked words as they are, so each byte converts with one
      // v_cvt_f32_ubyteN instead of a bit-field extract and a convert.
      asm volatile("" : "+v"(lo[0]), "+v"(lo[1]), "+v"(hi[0]), "+v"(hi[1]));
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const uint32_t src = (kk & 1) ? hi[kk >> 1] : lo[kk >> 1];
        float v[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const float q = (float)((src >> (8 * c)) & 0xffu);
          v[c] = __builtin_fmaf(q, (kk & 1) ? s16[c] : s[c], -zs[c]);
        }
        const int k = 4 * pp + kk;
        *reinterpret_cast<u32x2*>(dst + 128 * k + 16 * qg_swz(k, cq >> 1) + 8 * (cq & 1)) =
            u32x2{qg_pack(v[0], v[1]), qg_pack(v[2], v[3])};
      }
    } else {
      uint32_t o[8];
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const uint32_t b = r.v[d] ^ 0x80808080u;  // w + 128 as u8
        float f[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) f[e] = (float)((b >> (8 * e)) & 0xffu) - 128.0f;
        o[2 * d] = qg_pack(f[0], f[1]);
        o[2 * d + 1] = qg_pack(f[2], f[3]);
      }
      *reinterpret_cast<u32x4*>(dst + 128 * kr + 16 * qg_swz(kr, 2 * cc)) = u32x4{o[0], o[1], o[2], o[3]};
      *reinterpret_cast<u32x4*>(dst + 128 * kr + 16 * qg_swz(kr, 2 * cc + 1)) = u32x4{o[4], o[5], o[6], o[7]};
    }
  };

  // ---- B fragment offsets: tile j; the k half h of 32-row block hh adds
  //      the uniform 128 (32 hh + 4 h).  The swizzle term depends only on
  //      bits of the lane's k row 8g + r that 32 hh + 4 h does not change. ----
  int boff[4];
  {
    const int g = lane >> 4, r = (lane & 15) >> 2, q = lane & 3;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int k = 8 * g + r, col = 16 * j + 4 * q;
      boff[j] = 128 * k + 16 * qg_swz(k, col >> 3) + 2 * (col & 7);
    }
  }

  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto mma = [&](int t, const u32x4 (&xa)[8]) {
    const unsigned char* b = bbuf[t & 1];
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      u32x4 bf[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const qg_s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((qg_lds_s16x4_ptr)(b + boff[j] + 4096 * hh));
        const qg_s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((qg_lds_s16x4_ptr)(b + boff[j] + 4096 * hh + 512));
        const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
        bf[j] = u32x4{l2.x, l2.y, h2.x, h2.y};
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma16x16x32(bf[j], xa[4 * hh + i], acc[i][j]);
    }
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

  // ---- epilogue: lane owns row m, columns n .. n + 3 of each tile ----
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = m0 + 64 * wave + 16 * i + (lane & 15);
    if (m >= M) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
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

}  // namespace mk

namespace mkq {

bool qgemm_supported(int64_t M, int64_t K, int64_t N) {
  // Per-lane offsets are 32-bit: the weight matrix and x stay under 2 GiB.
  return M >= 1 && K >= 64 && K % 64 == 0 && N >= 64 && N % 64 == 0 && K * N < ((int64_t)1 << 31) &&
         M * K * 2 < ((int64_t)1 << 31);
}

hipError_t qgemm_launch(bool int4, const void* x, const void* w, const void* s, const void* z, void* y, int64_t M,
                        int64_t K, int64_t N, const void* aux, int epi, hipStream_t stream) {
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
  const dim3 grid((unsigned)(((M + 255) / 256) * (N / 64)));
  if (int4)
    hipLaunchKernelGGL(mk::qgemm_kernel<true>, grid, dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL(mk::qgemm_kernel<false>, grid, dim3(256), 0, stream, a);
  return hipGetLastError();
}

}  // namespace mkq
