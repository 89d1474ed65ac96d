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
//     order, with its 64-k group sums.
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

// Sum of the 8 bf16 values of one staged fragment, in slot order.
__device__ __forceinline__ float frag_sum(const u32x4& v) {
  float s = 0.f;
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    s += bf16_to_f32(w[i] & 0xFFFFu);
    s += bf16_to_f32(w[i] >> 16);
  }
  return s;
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

__device__ __forceinline__ uint32_t load_w4(const uint8_t* p, bool ok) {
  return ok ? *reinterpret_cast<const uint32_t*>(p) : 0u;
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
  const int ncol = n0 + 4 * c;
  const bool colok = ncol < a.N;
  const int ngroups = a.kwave >> 6;
  const size_t N = (size_t)a.N;

  unsigned char* wsm = smem + wv * a.wave_lds;
  u32x4* xl = reinterpret_cast<u32x4*>(wsm);
  float* xs = reinterpret_cast<float*>(smem + NW * a.wave_lds) + wv * ngroups * kQRows;

  // W rows of this lane: kp = kbeg/2 + 32*g + 16*h + 4*j + r (group g, step h).
  const uint8_t* wbase = a.w + (size_t)(kbeg / 2 + 4 * j) * N + ncol;
  const size_t sbase = (size_t)(kbeg >> 6) * N + ncol;
  const uint16_t* sptr = reinterpret_cast<const uint16_t*>(a.s);

  uint32_t rn[kQPF][8];
  u32x2 sn[kQPF];
  uint32_t zn[kQPF];
  auto load_group = [&](int g, uint32_t (&r)[8], u32x2& sv, uint32_t& zv) {
    const uint8_t* p = wbase + (size_t)(32 * g) * N;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int q = 0; q < 4; ++q) r[4 * h + q] = load_w4(p + (size_t)(16 * h + q) * N, colok);
    const size_t so = sbase + (size_t)g * N;
    sv = colok ? *reinterpret_cast<const u32x2*>(sptr + so) : u32x2{0u, 0u};
    zv = colok ? *reinterpret_cast<const uint32_t*>(a.z + so) : 0u;
  };
#pragma unroll
  for (int p = 0; p < kQPF; ++p)
    if (p < ngroups) load_group(p, rn[p], sn[p], zn[p]);

  stage_x<true>(a, xl, lane, m0, mrows, kbeg);
  for (int t = lane; t < ngroups * kQRows; t += kWave) {
    const int g = t >> 4, m = t & 15;
    float s = 0.f;
#pragma unroll
    for (int cc = 0; cc < 8; ++cc) {
      const int kc = 8 * g + cc;
      s += frag_sum(xl[((kc >> 2) * 4 + (kc & 3)) * 16 + m]);
    }
    xs[g * kQRows + m] = s;
  }
  __syncthreads();

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

      f32x4 acc[4];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const u32x4 A = xl[((2 * g + h) * 4 + j) * 16 + c];
        uint32_t t[4];
        transpose4x4(rc[4 * h + 0], rc[4 * h + 1], rc[4 * h + 2], rc[4 * h + 3], t[0], t[1], t[2],
                     t[3]);
#pragma unroll
        for (int w = 0; w < 4; ++w)
          acc[w] = mfma16x16x32(A, unpack_int4(t[w]), h == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : acc[w]);
      }
      const f32x4 xv = *reinterpret_cast<const f32x4*>(xs + g * kQRows + 4 * j);
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const uint32_t sw = (w < 2) ? sv.x : sv.y;
        const float sf = bf16_to_f32((w & 1) ? (sw >> 16) : (sw & 0xFFFFu));
        const float zf = (float)((zv >> (8 * w)) & 0xFFu);
        const float sz = sf * (128.f + zf);
        y[w] = sf * acc[w] + y[w];
        y[w] = y[w] - sz * xv;
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
  const int ncol = n0 + 4 * c;
  const bool colok = ncol < a.N;
  const int nsteps = a.kwave >> 5;
  const size_t N = (size_t)a.N;

  unsigned char* wsm = smem + wv * a.wave_lds;
  u32x4* xl = reinterpret_cast<u32x4*>(wsm);
  float* xs = reinterpret_cast<float*>(smem + NW * a.wave_lds) + wv * kQRows;

  // W rows of this lane: k = kbeg + 32*step + 8*j + r.
  const uint8_t* wbase = a.w + (size_t)(kbeg + 8 * j) * N + ncol;

  uint32_t rn[kQPF][8];
  auto load_step = [&](int st, uint32_t (&r)[8]) {
    const uint8_t* p = wbase + (size_t)(32 * st) * N;
#pragma unroll
    for (int q = 0; q < 8; ++q) r[q] = load_w4(p + (size_t)q * N, colok);
  };
#pragma unroll
  for (int p = 0; p < kQPF; ++p)
    if (p < nsteps) load_step(p, rn[p]);

  stage_x<false>(a, xl, lane, m0, mrows, kbeg);
  if (lane < kQRows) {
    float s = 0.f;
    for (int kc = 0; kc < (a.kwave >> 3); ++kc) s += frag_sum(xl[((kc >> 2) * 4 + (kc & 3)) * 16 + lane]);
    xs[lane] = s;
  }
  __syncthreads();

  f32x4 y[4];
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
    }
  }
  // Remove the +128 offset: y -= 128 * sum_k x over this wave's K range.
  const f32x4 xv = *reinterpret_cast<const f32x4*>(xs + 4 * j);
#pragma unroll
  for (int w = 0; w < 4; ++w) y[w] = y[w] - 128.f * xv;
  spill_y(wsm, y, c, j);
  reduce_and_store<NW, true>(a, smem, ksi, rb, m0, mrows, n0);
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
  const int xs_floats = (fmt == MK_QFMT_INT4_G64 ? (p->kwave / 64) : 1) * mk::kQRows;
  p->lds_bytes = (size_t)nw * p->wave_lds + (size_t)nw * xs_floats * 4;
  return p->lds_bytes <= kMaxLds;
}

// Pick waves per workgroup (nw) and split-K (ks).  K stays whole inside a
// workgroup whenever x fits in LDS and the grid already covers ~192+ CUs;
// otherwise the smallest split that does.  Every wave gets a whole number of
// 64-k groups.  MK_QMM_KS / MK_QMM_NW force a choice (tuning sweeps).
bool plan_q(int fmt, int64_t M, int64_t K, int64_t N, QPlan* p) {
  p->ntiles = (int)((N + mk::kQCols - 1) / mk::kQCols);
  p->rowblocks = (int)((M + mk::kQRows - 1) / mk::kQRows);
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
  switch (p.nw) {
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
