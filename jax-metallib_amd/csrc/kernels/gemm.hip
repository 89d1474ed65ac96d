// dot_general GEMM for gfx950: C[b] = A[b] @ B[b], row-major A [M,K] and
// B [K,N] (the canonical form the executor reduces dot_general to; reference
// HandleDotGeneral, ops/binary_ops.mm:644-1100, rank-2 NN path :1011-1019,
// and the generated tiled kernels runtime/metal_kernels.mm:2477-2761).
//
// bf16 x bf16 -> f32 accumulation -> bf16 or f32 output
//   (preferred_element_type = f32 returns f32, binary_ops.mm:775-782)
// f32  x f32  -> f32 (v_mfma_f32_16x16x4_f32, full f32 products)
//
// Design:
//   * Block tile BM x BN x 64 (bf16) with WM x WN waves; every wave owns a
//     (BM/WM) x (BN/WN) sub-tile of 16x16 MFMA tiles held in accumulators.
//   * Global -> registers -> LDS double buffering, one barrier per k-tile:
//     the next k-tile's global loads are in flight while the MFMAs consume
//     the current one.
//   * A is staged as-is ([m][k], k contiguous).  B arrives n-contiguous, but
//     the MFMA wants k runs per lane, so each thread transposes an 8x8 block
//     of B in registers (v_perm_b32 on 16-bit halves) while staging; LDS then
//     holds B as [n][k].  Rows are padded to 144 B so the 16-byte fragment
//     reads of 16 consecutive rows hit distinct LDS banks.
//   * The MFMA is issued as B-fragment x A-fragment, which yields C^T tiles:
//     each lane then owns 4 consecutive columns of one row, stored as one
//     8-byte (bf16) or 16-byte (f32) write.
//   * Workgroup -> tile mapping is XCD-aware: runs of consecutive logical
//     ids stay on one XCD and cover a 4-row band of tiles, so the A panels and
//     B panels they share stay in that XCD's L2.
#include "common.h"
#include "epilogue.h"

namespace mk {

struct GemmArgs {
  const void* a;
  const void* b;
  void* c;
  int M, N, K;
  int64_t sa, sb, sc;  // batch strides in elements
  int out_f32;         // bf16 kernel: 1 -> f32 output, 0 -> bf16 output
  int epi;             // bf16 output: MK_EPI_NONE / MK_EPI_ADD / MK_EPI_SWIGLU with aux
  const uint16_t* aux; // bf16, same layout and batch stride as C
};

// Four bf16 outputs of C row-major at offset off, with the GEMM's epilogue.
__device__ __forceinline__ void store_bf16x4(const GemmArgs& p, uint16_t* C, const uint16_t* X, size_t off,
                                             const f32x4& acc) {
  epi_store_bf16x4(C, X, p.epi, off, acc);
}

// Map a logical workgroup id to a (tile row, tile col) with bands of GM tile
// rows, so consecutive ids sweep a GM-tall column block.
__device__ __forceinline__ void tile_coords(uint32_t L, int tiles_m, int tiles_n, int& tm, int& tn) {
  constexpr int GM = 4;
  if (tiles_m % GM == 0) {
    const int band = (int)L / (GM * tiles_n);
    const int r = (int)L - band * GM * tiles_n;
    tm = band * GM + r % GM;
    tn = r / GM;
  } else {
    tm = (int)L / tiles_n;
    tn = (int)L - tm * tiles_n;
  }
}

template <int BM, int BN, int WM, int WN>
__global__ __launch_bounds__(WM * WN * 64) void gemm_bf16_kernel(GemmArgs p) {
  constexpr int BK = 64;
  constexpr int LDK = BK + 8;  // padded row length (bf16 elements)
  constexpr int NT = WM * WN * 64;
  constexpr int TM = BM / WM / 16;
  constexpr int TN = BN / WN / 16;
  constexpr int ACH = BM * BK / 8 / NT;             // A 16-byte chunks per thread
  constexpr int BTOT = (BK / 8) * (BN / 8);         // B 8x8 blocks per tile
  constexpr int BBL = (BTOT + NT - 1) / NT;         // B blocks per thread
  static_assert(ACH * NT * 8 == BM * BK, "A staging must divide evenly");

  extern __shared__ __align__(16) unsigned char smem[];
  uint16_t* As = reinterpret_cast<uint16_t*>(smem);  // [2][BM][LDK]
  uint16_t* Bs = As + 2 * BM * LDK;                   // [2][BN][LDK]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int tiles_m = (p.M + BM - 1) / BM, tiles_n = (p.N + BN - 1) / BN;
  int tm, tn;
  tile_coords(xcd_logical_id(blockIdx.x, gridDim.x), tiles_m, tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const uint16_t* A = static_cast<const uint16_t*>(p.a) + (size_t)blockIdx.z * p.sa;
  const uint16_t* B = static_cast<const uint16_t*>(p.b) + (size_t)blockIdx.z * p.sb;
  const int M = p.M, N = p.N, K = p.K;

  u32x4 ra[ACH];
  u32x4 rb[BBL][8];

  auto load_tile = [&](int k0) {
#pragma unroll
    for (int i = 0; i < ACH; ++i) {
      const int q = tid + i * NT;
      const int row = q / (BK / 8), kc = q % (BK / 8);
      const int gm = m0 + row, gk = k0 + 8 * kc;
      ra[i] = (gm < M && gk < K) ? *reinterpret_cast<const u32x4*>(A + (size_t)gm * K + gk)
                                 : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int i = 0; i < BBL; ++i) {
      const int q = tid + i * NT;
      const int kb = q / (BN / 8), nb = q % (BN / 8);
      const int gn = n0 + 8 * nb;
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        const int gk = k0 + 8 * kb + r;
        rb[i][r] = (q < BTOT && gn < N && gk < K) ? *reinterpret_cast<const u32x4*>(B + (size_t)gk * N + gn)
                                      : u32x4{0u, 0u, 0u, 0u};
      }
    }
  };

  auto store_tile = [&](int buf) {
    uint16_t* as = As + buf * BM * LDK;
    uint16_t* bs = Bs + buf * BN * LDK;
#pragma unroll
    for (int i = 0; i < ACH; ++i) {
      const int q = tid + i * NT;
      const int row = q / (BK / 8), kc = q % (BK / 8);
      *reinterpret_cast<u32x4*>(as + row * LDK + 8 * kc) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < BBL; ++i) {
      const int q = tid + i * NT;
      if (q >= BTOT) break;
      const int kb = q / (BN / 8), nb = q % (BN / 8);
      // Transpose the 8 (k) x 8 (n) block: column c gets halfword c of rows 0..7.
      const uint32_t* w = reinterpret_cast<const uint32_t*>(&rb[i][0]);
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const uint32_t sel = (c & 1) ? 0x07060302u : 0x05040100u;
        const int d = c >> 1;
        u32x4 o;
        o.x = perm(w[1 * 4 + d], w[0 * 4 + d], sel);
        o.y = perm(w[3 * 4 + d], w[2 * 4 + d], sel);
        o.z = perm(w[5 * 4 + d], w[4 * 4 + d], sel);
        o.w = perm(w[7 * 4 + d], w[6 * 4 + d], sel);
        *reinterpret_cast<u32x4*>(bs + (8 * nb + c) * LDK + 8 * kb) = o;
      }
    }
  };

  f32x4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int KT = (K + BK - 1) / BK;
  load_tile(0);
  store_tile(0);
  __syncthreads();

  const int arow = wm * TM * 16 + (lane & 15);
  const int brow = wn * TN * 16 + (lane & 15);
  const int kofs = 8 * (lane >> 4);

  for (int kt = 0; kt < KT; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < KT) load_tile((kt + 1) * BK);
    const uint16_t* as = As + buf * BM * LDK;
    const uint16_t* bs = Bs + buf * BN * LDK;
#pragma unroll
    for (int ks = 0; ks < BK / 32; ++ks) {
      u32x4 af[TM], bf[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i)
        af[i] = *reinterpret_cast<const u32x4*>(as + (arow + 16 * i) * LDK + 32 * ks + kofs);
#pragma unroll
      for (int j = 0; j < TN; ++j)
        bf[j] = *reinterpret_cast<const u32x4*>(bs + (brow + 16 * j) * LDK + 32 * ks + kofs);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = mfma16x16x32(bf[j], af[i], acc[i][j]);
    }
    if (kt + 1 < KT) store_tile(buf ^ 1);
    __syncthreads();
  }

  // Epilogue: lane owns row m, columns n..n+3 of each 16x16 tile.
  const int mrow = m0 + wm * TM * 16 + (lane & 15);
  const int ncol = n0 + wn * TN * 16 + 4 * (lane >> 4);
  if (p.out_f32) {
    float* C = static_cast<float*>(p.c) + (size_t)blockIdx.z * p.sc;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int m = mrow + 16 * i;
      if (m >= M) continue;
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int n = ncol + 16 * j;
        if (n < N) *reinterpret_cast<f32x4*>(C + (size_t)m * N + n) = acc[i][j];
      }
    }
  } else {
    uint16_t* C = static_cast<uint16_t*>(p.c) + (size_t)blockIdx.z * p.sc;
    const uint16_t* X = p.aux + (p.epi != MK_EPI_NONE ? (size_t)blockIdx.z * p.sc : 0);
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int m = mrow + 16 * i;
      if (m >= M) continue;
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int n = ncol + 16 * j;
        if (n < N) store_bf16x4(p, C, X, (size_t)m * N + n, acc[i][j]);
      }
    }
  }
}

// f32 GEMM: v_mfma_f32_16x16x4_f32.  Within each 32-k chunk a lane of k
// block j (= lane / 16) feeds k = 8j + s to the s-th MFMA, for both operands,
// so a fragment is 8 consecutive floats of one row (two 16-byte LDS reads).
template <int BM, int BN, int WM, int WN>
__global__ __launch_bounds__(WM * WN * 64) void gemm_f32_kernel(GemmArgs p) {
  constexpr int BK = 32;
  constexpr int LDK = BK + 4;  // padded row length (floats): 144 B
  constexpr int NT = WM * WN * 64;
  constexpr int TM = BM / WM / 16;
  constexpr int TN = BN / WN / 16;
  constexpr int ACH = BM * BK / 4 / NT;          // A 16-byte chunks per thread
  constexpr int BTOT = (BK / 4) * (BN / 4);      // B 4x4 blocks per tile
  constexpr int BBL = (BTOT + NT - 1) / NT;      // B blocks per thread
  static_assert(ACH * NT * 4 == BM * BK, "A staging must divide evenly");

  extern __shared__ __align__(16) unsigned char smem[];
  float* As = reinterpret_cast<float*>(smem);  // [2][BM][LDK]
  float* Bs = As + 2 * BM * LDK;               // [2][BN][LDK]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int tiles_m = (p.M + BM - 1) / BM, tiles_n = (p.N + BN - 1) / BN;
  int tm, tn;
  tile_coords(xcd_logical_id(blockIdx.x, gridDim.x), tiles_m, tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const float* A = static_cast<const float*>(p.a) + (size_t)blockIdx.z * p.sa;
  const float* B = static_cast<const float*>(p.b) + (size_t)blockIdx.z * p.sb;
  const int M = p.M, N = p.N, K = p.K;

  f32x4 ra[ACH];
  f32x4 rb[BBL][4];

  auto load_tile = [&](int k0) {
#pragma unroll
    for (int i = 0; i < ACH; ++i) {
      const int q = tid + i * NT;
      const int row = q / (BK / 4), kc = q % (BK / 4);
      const int gm = m0 + row, gk = k0 + 4 * kc;
      ra[i] = (gm < M && gk < K) ? *reinterpret_cast<const f32x4*>(A + (size_t)gm * K + gk)
                                 : f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int i = 0; i < BBL; ++i) {
      const int q = tid + i * NT;
      const int kb = q / (BN / 4), nb = q % (BN / 4);
      const int gn = n0 + 4 * nb;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int gk = k0 + 4 * kb + r;
        rb[i][r] = (q < BTOT && gn < N && gk < K) ? *reinterpret_cast<const f32x4*>(B + (size_t)gk * N + gn)
                                      : f32x4{0.f, 0.f, 0.f, 0.f};
      }
    }
  };

  auto store_tile = [&](int buf) {
    float* as = As + buf * BM * LDK;
    float* bs = Bs + buf * BN * LDK;
#pragma unroll
    for (int i = 0; i < ACH; ++i) {
      const int q = tid + i * NT;
      const int row = q / (BK / 4), kc = q % (BK / 4);
      *reinterpret_cast<f32x4*>(as + row * LDK + 4 * kc) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < BBL; ++i) {
      const int q = tid + i * NT;
      if (q >= BTOT) break;
      const int kb = q / (BN / 4), nb = q % (BN / 4);
      *reinterpret_cast<f32x4*>(bs + (4 * nb + 0) * LDK + 4 * kb) =
          f32x4{rb[i][0].x, rb[i][1].x, rb[i][2].x, rb[i][3].x};
      *reinterpret_cast<f32x4*>(bs + (4 * nb + 1) * LDK + 4 * kb) =
          f32x4{rb[i][0].y, rb[i][1].y, rb[i][2].y, rb[i][3].y};
      *reinterpret_cast<f32x4*>(bs + (4 * nb + 2) * LDK + 4 * kb) =
          f32x4{rb[i][0].z, rb[i][1].z, rb[i][2].z, rb[i][3].z};
      *reinterpret_cast<f32x4*>(bs + (4 * nb + 3) * LDK + 4 * kb) =
          f32x4{rb[i][0].w, rb[i][1].w, rb[i][2].w, rb[i][3].w};
    }
  };

  f32x4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int KT = (K + BK - 1) / BK;
  load_tile(0);
  store_tile(0);
  __syncthreads();

  const int arow = wm * TM * 16 + (lane & 15);
  const int brow = wn * TN * 16 + (lane & 15);
  const int kofs = 8 * (lane >> 4);

  for (int kt = 0; kt < KT; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < KT) load_tile((kt + 1) * BK);
    const float* as = As + buf * BM * LDK;
    const float* bs = Bs + buf * BN * LDK;
    f32x4 af[TM][2], bf[TN][2];
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      af[i][0] = *reinterpret_cast<const f32x4*>(as + (arow + 16 * i) * LDK + kofs);
      af[i][1] = *reinterpret_cast<const f32x4*>(as + (arow + 16 * i) * LDK + kofs + 4);
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      bf[j][0] = *reinterpret_cast<const f32x4*>(bs + (brow + 16 * j) * LDK + kofs);
      bf[j][1] = *reinterpret_cast<const f32x4*>(bs + (brow + 16 * j) * LDK + kofs + 4);
    }
#pragma unroll
    for (int s = 0; s < 8; ++s) {
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(bf[j][s >> 2][s & 3], af[i][s >> 2][s & 3],
                                                          acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < KT) store_tile(buf ^ 1);
    __syncthreads();
  }

  float* C = static_cast<float*>(p.c) + (size_t)blockIdx.z * p.sc;
  const int mrow = m0 + wm * TM * 16 + (lane & 15);
  const int ncol = n0 + wn * TN * 16 + 4 * (lane >> 4);
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int m = mrow + 16 * i;
    if (m >= M) continue;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int n = ncol + 16 * j;
      if (n < N) *reinterpret_cast<f32x4*>(C + (size_t)m * N + n) = acc[i][j];
    }
  }
}


// ---------------------------------------------------------------------------
// Large-tile bf16 GEMM (M % 256 == 0, N % 256 == 0, K % 64 == 0).
//
// 256 x 256 x 64 workgroup tile; WM x WN waves (2 x 4: each wave a 128 x 64
// tile of 8 x 4 16x16x32 MFMA accumulators; 2 x 2: 128 x 128, 8 x 8).  Both operands are
// staged in LDS in their natural layouts (A [m][k], B [k][n]) through
// registers with one barrier per k-tile (double buffer, 128 KB).  The B
// fragments come straight out of the [k][n] layout with gfx950's transposing
// LDS read, ds_read_b64_tr_b16: within each 16-lane group, lanes 4r + q name
// the 8 bytes of row r, columns 4q..4q+3, and lane j receives column j of
// the 4 x 16 block -- four consecutive k of one n, i.e. half of an MFMA
// fragment.  No register transposes remain.
//
// LDS swizzles (16-byte chunks): A row r, chunk c lives at chunk
// c ^ ((r >> 1) & 7), so the 16 rows of one fragment read cover all 64
// banks; B row k, chunk c lives at c ^ (k & 3 | ((k >> 3) & 3) << 2), so the
// 16 rows one transposing read touches land in 16 different 16-byte slots.
// ---------------------------------------------------------------------------
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4* lds_s16x4_ptr;

__device__ __forceinline__ int swz_a(int row, int c) { return c ^ ((row >> 1) & 7); }
__device__ __forceinline__ int swz_b(int k, int c) { return c ^ ((k & 3) | (((k >> 3) & 3) << 2)); }

__device__ __forceinline__ u32x2 lds_tr16(const uint16_t* p) {
  const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_ptr)(p));
  return __builtin_bit_cast(u32x2, v);
}

template <int WM_, int WN_>
__global__ __launch_bounds__(WM_ * WN_ * 64) void gemm_bf16_256_kernel(GemmArgs p) {
  constexpr int BM = 256, BN = 256, BK = 64, NT = WM_ * WN_ * 64;
  constexpr int TM = BM / WM_ / 16, TN = BN / WN_ / 16;  // per-wave MFMA tiles
  constexpr int CH = BM * BK / 8 / NT;                   // 16-byte chunks per thread (A and B each)
  extern __shared__ __align__(16) unsigned char smem[];
  uint16_t* As = reinterpret_cast<uint16_t*>(smem);  // [2][BM * BK]
  uint16_t* Bs = As + 2 * BM * BK;                    // [2][BK * BN]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN_, wn = wave % WN_;
  const int tiles_m = p.M / BM, tiles_n = p.N / BN;
  int tm, tn;
  tile_coords(xcd_logical_id(blockIdx.x, gridDim.x), tiles_m, tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const uint16_t* A = static_cast<const uint16_t*>(p.a) + (size_t)blockIdx.z * p.sa + (size_t)m0 * p.K;
  const uint16_t* B = static_cast<const uint16_t*>(p.b) + (size_t)blockIdx.z * p.sb + n0;
  const int K = p.K, N = p.N;

  // Staging: CH A chunks (row q/8, chunk q%8) and CH B chunks (row q/32,
  // chunk q%32) per thread, q = tid + NT * i, moved in two halves so only
  // CH/2 + CH/2 chunks sit in registers at a time: half h of the next tile is
  // loaded before 32-k step h and stored to the free buffer after it.
  constexpr int HC = CH / 2;
  static_assert(HC * 2 == CH, "staging splits in halves");
  u32x4 ra[HC], rb[HC];
  auto load_half = [&](int k0, int h) {
#pragma unroll
    for (int i = 0; i < HC; ++i) {
      const int q = tid + NT * (h * HC + i);
      ra[i] = *reinterpret_cast<const u32x4*>(A + (size_t)(q >> 3) * K + k0 + 8 * (q & 7));
      rb[i] = *reinterpret_cast<const u32x4*>(B + (size_t)(k0 + (q >> 5)) * N + 8 * (q & 31));
    }
  };
  auto store_half = [&](int buf, int h) {
    uint16_t* as = As + buf * BM * BK;
    uint16_t* bs = Bs + buf * BK * BN;
#pragma unroll
    for (int i = 0; i < HC; ++i) {
      const int q = tid + NT * (h * HC + i);
      const int ar = q >> 3, ac = q & 7, br = q >> 5, bc = q & 31;
      *reinterpret_cast<u32x4*>(as + ar * BK + 8 * swz_a(ar, ac)) = ra[i];
      *reinterpret_cast<u32x4*>(bs + br * BN + 8 * swz_b(br, bc)) = rb[i];
    }
  };

  f32x4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int KT = K / BK;
  load_half(0, 0);
  store_half(0, 0);
  load_half(0, 1);
  store_half(0, 1);
  __syncthreads();

  // Per-lane fragment coordinates.
  const int arow0 = wm * (16 * TM) + (lane & 15);   // + 16 * i
  const int akb = lane >> 4;                          // k block (8 k) in a 32-k step
  const int g = lane >> 4, r = (lane & 15) >> 2, q = lane & 3;
  const int bcol0 = wn * (16 * TN) + 4 * q;          // + 16 * j

  for (int kt = 0; kt < KT; ++kt) {
    const int buf = kt & 1;
    const bool more = kt + 1 < KT;
    const uint16_t* as = As + buf * BM * BK;
    const uint16_t* bs = Bs + buf * BK * BN;
#pragma unroll
    for (int ks = 0; ks < BK / 32; ++ks) {
      if (more) load_half((kt + 1) * BK, ks);
      // All B fragments of the step, then one A fragment per row of tiles
      // (keeps only TN + 1 fragments live).
      u32x4 bf[TN];
      const int k1 = 32 * ks + 8 * g + r;
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int col = bcol0 + 16 * j;
        const u32x2 lo = lds_tr16(bs + k1 * BN + 8 * swz_b(k1, col >> 3) + (col & 7));
        const u32x2 hi = lds_tr16(bs + (k1 + 4) * BN + 8 * swz_b(k1 + 4, col >> 3) + (col & 7));
        bf[j] = u32x4{lo.x, lo.y, hi.x, hi.y};
      }
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int row = arow0 + 16 * i;
        const u32x4 af = *reinterpret_cast<const u32x4*>(as + row * BK + 8 * swz_a(row, 4 * ks + akb));
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = mfma16x16x32(bf[j], af, acc[i][j]);
      }
      if (more) store_half(buf ^ 1, ks);
    }
    __syncthreads();
  }

  // Epilogue (C^T tiles): lane owns row m, columns n..n+3 of each tile.
  const int mrow = m0 + wm * (16 * TM) + (lane & 15);
  const int ncol = n0 + wn * (16 * TN) + 4 * (lane >> 4);
  if (p.out_f32) {
    float* C = static_cast<float*>(p.c) + (size_t)blockIdx.z * p.sc;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
        *reinterpret_cast<f32x4*>(C + (size_t)(mrow + 16 * i) * N + ncol + 16 * j) = acc[i][j];
  } else {
    uint16_t* C = static_cast<uint16_t*>(p.c) + (size_t)blockIdx.z * p.sc;
    const uint16_t* X = p.aux + (p.epi != MK_EPI_NONE ? (size_t)blockIdx.z * p.sc : 0);
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) store_bf16x4(p, C, X, (size_t)(mrow + 16 * i) * N + ncol + 16 * j, acc[i][j]);
  }
}


// ---------------------------------------------------------------------------
// 256 x 256 tile fed by LDS DMA.
//
// A 4-stage ring of 32-k stages (A 256 x 32 | B 32 x 256 bf16, 32 KB each,
// 128 KB of LDS) is filled by global_load_lds three stages ahead, so the
// MFMAs of stage k overlap the HBM latency of stages k+1..k+3 and no staging
// registers are needed.  Each stage takes 4 DMA instructions per wave and
// one barrier (raw s_barrier: every thread first waits for its own DMAs of
// the stage, so no fence drains the ring).  The DMAs are issued from inline
// asm with explicit waits, so the compiler -- which then sees no pending
// LDS writes -- schedules the fragment reads against the MFMAs itself.
// LDS layouts (swizzles applied by choosing each DMA lane's source chunk):
//   A row r (64 B): 16-byte chunk c at position c ^ (r / 2 % 4) (ten chunk
//     swizzles were measured with SQ_LDS_BANK_CONFLICT on this fragment read,
//     row = lane % 16 and chunk = lane / 16; only this one had no conflicts,
//     the former c ^ (r / 4 % 4) doubled the cycles of every A read);
//   B k row (512 B): chunk c at c ^ (2 (k % 4) + 8 (k / 8 % 2)),
// which make the A ds_read_b128 and the B ds_read_b64_tr_b16 fragment reads
// bank-conflict-free.  Waves 2 x 4, each 128 x 64 (8 x 4 MFMA 16x16x32
// tiles per 32 k).
// ---------------------------------------------------------------------------
#ifndef MK_GEMM_STAGES
#define MK_GEMM_STAGES 4
#endif
constexpr int kGemmStages = MK_GEMM_STAGES;
constexpr int kPipeStages = 5;  // 5 x 32 KB: all of the 160 KB LDS
constexpr int kEpiStageRow = 272;                   // bf16 per staged output row (256 + 16 pad)
constexpr int kEpiStageBytes = 256 * kEpiStageRow * 2;  // 139,264 B: the staged 256x256 tile
constexpr int kGemmStageBytes = 32 * 1024;

__device__ __forceinline__ int swz_b2(int k, int c) { return c ^ ((2 * (k & 3)) | (((k >> 3) & 1) << 3)); }


// BT: B arrives as B^T [N, K] (k contiguous).  Its stage then has A's layout
// (256 n rows of 64 B, the same swizzle) and each B fragment is one
// ds_read_b128 instead of two transposing reads; the registers hold the same
// values, so the results are the same bits as with B [K, N].
template <int WN_, bool PIPE, bool BT = false>  // waves 2 x WN_; each 128 x (256 / WN_)
__global__ __launch_bounds__(2 * WN_ * 64) void gemm_bf16_256dma_kernel(GemmArgs p) {
  constexpr int BM = 256, BN = 256, BK = 32, TM = 8, TN = 256 / WN_ / 16;
  constexpr int NW = 2 * WN_, DI = 16 / NW;  // waves; DMA instructions per wave for A (and B)
  constexpr int ABYTES = BM * BK * 2;  // 16 KB
  extern __shared__ __align__(16) unsigned char smem[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN_, wn = wave % WN_;
  const int tiles_m = p.M / BM, tiles_n = p.N / BN;
  int tm, tn;
  tile_coords(xcd_logical_id(blockIdx.x, gridDim.x), tiles_m, tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const uint16_t* A = static_cast<const uint16_t*>(p.a) + (size_t)blockIdx.z * p.sa + (size_t)m0 * p.K;
  const uint16_t* B = static_cast<const uint16_t*>(p.b) + (size_t)blockIdx.z * p.sb + (BT ? (size_t)n0 * p.K : n0);
  const int K = p.K, N = p.N;
  // Elements between consecutive stages of one B DMA source.
  const size_t bstep = BT ? (size_t)BK : (size_t)BK * N;

  // DMA sources.  A instruction i (rows 16i..16i+15): lane L fills row
  // 16i + L/4, position L%4.  B instruction i (k rows 2i, 2i+1): lane L
  // fills k row 2i + L/32, position L%32.  Wave w issues i = DI w .. DI w + DI - 1
  // of each.
  const uint16_t* asrc[DI];
  const uint16_t* bsrc[DI];
#pragma unroll
  for (int u = 0; u < DI; ++u) {
    const int i = DI * wave + u;
    const int row = 16 * i + (lane >> 2), pa = lane & 3;
    asrc[u] = A + (size_t)row * K + 8 * (pa ^ ((row >> 1) & 3));
    if constexpr (BT) {
      bsrc[u] = B + (size_t)row * K + 8 * (pa ^ ((row >> 1) & 3));
    } else {
      const int kr = 2 * i + (lane >> 5), pb = lane & 31;
      bsrc[u] = B + (size_t)kr * N + 8 * swz_b2(kr, pb);
    }
  }
  const uint32_t sbase = lds_addr(smem);
  auto issue = [&](int kt) {
    const uint32_t st = sbase + (uint32_t)((kt % kGemmStages) * kGemmStageBytes);
#pragma unroll
    for (int u = 0; u < DI; ++u) dma16_asm(asrc[u] + kt * BK, st + (uint32_t)((DI * wave + u) * 1024));
#pragma unroll
    for (int u = 0; u < DI; ++u)
      dma16_asm(bsrc[u] + (size_t)kt * bstep, st + (uint32_t)(ABYTES + (DI * wave + u) * 1024));
  };

  // Fragment offsets within a stage.  A tile i of this wave: row
  // wm*128 + 16i + (lane & 15), 16-byte chunk lane >> 4.  B tile j, low/high
  // 4 k: tr16 lane 4r + q of 16-lane group g reads k row 8g + r (+4), columns
  // wn*64 + 16j + 4q .. +3.
  const int arow = wm * 128 + (lane & 15);
  const int aoff = arow * 64 + 16 * ((lane >> 4) ^ ((arow >> 1) & 3));
  int boff[2 * TN];
  if constexpr (BT) {
    // B^T tile j: n row wn*64 + 16j + (lane & 15), chunk lane >> 4 (A's read).
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int nrow = wn * (16 * TN) + 16 * j + (lane & 15);
      boff[j] = ABYTES + nrow * 64 + 16 * ((lane >> 4) ^ ((nrow >> 1) & 3));
      boff[TN + j] = 0;
    }
  } else {
    const int g = lane >> 4, r = (lane & 15) >> 2, q = lane & 3;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int col = wn * (16 * TN) + 16 * j + 4 * q;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int k1 = 8 * g + r + 4 * h;
        boff[2 * j + h] = ABYTES + k1 * (BN * 2) + 16 * swz_b2(k1, col >> 3) + 2 * (col & 7);
      }
    }
  }

  f32x4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Epilogue operand: loaded before the K loop so its latency hides behind
  // the whole loop (64 VGPRs; the epilogue itself then only computes).  The
  // 4-wave variant, with twice the tiles per wave, reads it at the end.
  const int mrow = m0 + wm * (16 * TM) + (lane & 15);
  const int ncol = n0 + wn * (16 * TN) + 4 * (lane >> 4);
  constexpr bool kPreAux = WN_ == 4 && !PIPE;
  u32x2 auxv[kPreAux ? TM : 1][kPreAux ? TN : 1];
  if (kPreAux && (p.epi == MK_EPI_ADD || p.epi == MK_EPI_SWIGLU)) {
    const uint16_t* X = p.aux + (size_t)blockIdx.z * p.sc;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
        auxv[kPreAux ? i : 0][kPreAux ? j : 0] =
            *reinterpret_cast<const u32x2*>(X + (size_t)(mrow + 16 * i) * N + ncol + 16 * j);
  }

  const int KT = K / BK;
  if constexpr (PIPE) {
    // Fragment pipelining: the fragments of stage kt+1 are read from LDS
    // while the MFMAs of stage kt (fragments already in registers) run, so
    // LDS latency overlaps the matrix pipe instead of following it.  A
    // stage's slot is free once its fragments are in registers, so a ring
    // of kPipeStages slots keeps kPipeStages - 1 stages of DMA in flight.
    // Measured on 4096^3 (skip-work variants of this loop): the L2 -> LDS
    // feed alone takes ~70 us and the MFMA + fragment loop alone ~94 us, so
    // the kernel is bound by how well the two overlap (~126 us).
    auto read_b = [&](const unsigned char* st, u32x4* bf) {
      if constexpr (BT) {
#pragma unroll
        for (int j = 0; j < TN; ++j) bf[j] = *reinterpret_cast<const u32x4*>(st + boff[j]);
        return;
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_ptr)(st + boff[2 * j]));
        const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_ptr)(st + boff[2 * j + 1]));
        const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
        bf[j] = u32x4{l2.x, l2.y, h2.x, h2.y};
      }
    };
    // Ring of S stages; stage s lives in slot s % S.  Iteration kt issues
    // stage kt + S (if it exists) into the slot stage kt has just left.
    constexpr int S = kPipeStages;
    auto issue_a = [&](int ks, int slot, int u) {
      dma16_asm(asrc[u] + ks * BK, sbase + (uint32_t)(slot * kGemmStageBytes + (DI * wave + u) * 1024));
    };
    auto issue_b = [&](int ks, int slot, int u) {
      dma16_asm(bsrc[u] + (size_t)ks * bstep,
                sbase + (uint32_t)(slot * kGemmStageBytes + ABYTES + (DI * wave + u) * 1024));
    };
    // The host only picks this kernel when KT >= 2 S.
    for (int s = 0; s < S; ++s) {
#pragma unroll
      for (int u = 0; u < DI; ++u) issue_a(s, s, u);
#pragma unroll
      for (int u = 0; u < DI; ++u) issue_b(s, s, u);
    }
    vm_wait(2 * DI * (S - 1));
    asm volatile("s_barrier" ::: "memory");
    // Fragments: A in one set (fragment i of stage kt+1 is read into the
    // registers of fragment i of stage kt right after its last MFMA), B in
    // two sets alternated by a 2x unrolled loop.
    u32x4 bf0[TN], bf1[TN], af[TM];
    read_b(smem, bf0);
#pragma unroll
    for (int i = 0; i < TM; ++i) af[i] = *reinterpret_cast<const u32x4*>(smem + aoff + 1024 * i);
    int slot_cur = 0;  // kt % S
    auto step = [&](auto with_dma, int kt, u32x4* bfc, u32x4* bfn) {
      constexpr bool kDma = decltype(with_dma)::value;
      __builtin_amdgcn_sched_barrier(0);
      // Own DMAs of stage kt+1 landed and own fragment reads of stage kt
      // complete; after the barrier every wave's are, so stage kt+1 is
      // visible and stage kt's slot is free.  lgkmcnt(0) and the barrier
      // are builtins so the compiler knows the reads have completed and
      // adds no wait of its own later.  DMA stages in flight after stage
      // kt+1: kt+2 .. min(kt+S-1, KT-1), i.e. S-2 while iteration kt still
      // issues one; in the last iterations the wait is for all of them.
      if constexpr (kDma) vm_wait(2 * DI * (S - 2));
      else vm_wait(0);
      __builtin_amdgcn_s_waitcnt(0xC07F);
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
      const int ks = kt + S;
      const int slot_nx = slot_cur + 1 == S ? 0 : slot_cur + 1;
      // On the last stage this reads a stale slot; the values are unused.
      const unsigned char* nx = smem + slot_nx * kGemmStageBytes;
      read_b(nx, bfn);
      // The DMAs of the new stage are spread over the MFMA groups.
#pragma unroll
      for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = mfma16x16x32(bfc[j], af[i], acc[i][j]);
        af[i] = *reinterpret_cast<const u32x4*>(nx + aoff + 1024 * i);
        if constexpr (kDma) {
          if (i < DI) issue_a(ks, slot_cur, i);
          else if (i < 2 * DI) issue_b(ks, slot_cur, i - DI);
        }
        // Keep this order: the compiler would otherwise cluster the reads
        // and DMAs and move MFMAs across the barrier.
        __builtin_amdgcn_sched_barrier(0);
      }
      slot_cur = slot_nx;
    };
    using DmaOn = std::integral_constant<bool, true>;
    using DmaOff = std::integral_constant<bool, false>;
    // Pairs of iterations that both issue a stage; kt stays even, so the
    // B fragment sets alternate at compile time.
    int kt = 0;
    for (; kt + 1 + S < KT; kt += 2) {
      step(DmaOn{}, kt, bf0, bf1);
      step(DmaOn{}, kt + 1, bf1, bf0);
    }
    // S or S+1 iterations remain; the first of S+1 still issues a stage.
    if (kt + S < KT) {
      step(DmaOn{}, kt, bf0, bf1);
      ++kt;
#pragma unroll
      for (int j = 0; j < TN; ++j) bf0[j] = bf1[j];
    }
#pragma unroll
    for (int t = 0; t < S; ++t) step(DmaOff{}, kt + t, (t & 1) ? bf1 : bf0, (t & 1) ? bf0 : bf1);
  } else {
  const int pre = KT < kGemmStages - 1 ? KT : kGemmStages - 1;
  for (int kt = 0; kt < pre; ++kt) issue(kt);
  for (int kt = 0; kt < KT; ++kt) {
    // This thread's DMAs of stage kt have landed (later stages may not).
    {
      const int ahead = KT - 1 - kt < kGemmStages - 2 ? KT - 1 - kt : kGemmStages - 2;  // later stages in flight
      vm_wait(2 * DI * ahead);
    }
    // Everyone's have; everyone is done reading stage kt-1's slot.
    asm volatile("s_barrier" ::: "memory");
    if (kt + kGemmStages - 1 < KT) issue(kt + kGemmStages - 1);
    const unsigned char* st = smem + (kt % kGemmStages) * kGemmStageBytes;
    u32x4 bf[TN];
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      if constexpr (BT) {
        bf[j] = *reinterpret_cast<const u32x4*>(st + boff[j]);
        continue;
      }
      const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_ptr)(st + boff[2 * j]));
      const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_ptr)(st + boff[2 * j + 1]));
      const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
      bf[j] = u32x4{l2.x, l2.y, h2.x, h2.y};
    }
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const u32x4 af = *reinterpret_cast<const u32x4*>(st + aoff + 1024 * i);
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] = mfma16x16x32(bf[j], af, acc[i][j]);
    }
  }
  }

  // bf16 output through LDS (8-wave kernels; the ring kernel keeps its
  // preloaded ADD / SWIGLU operand in registers and stores those directly).
  // Stored from the registers, each lane writes 4 columns of a row (8
  // bytes), so a wave's store touches 16 rows in 32-byte pieces and the
  // end-of-kernel burst of such requests cost ~8 us at 4096^3.  Staged as
  // bf16 (the rounding every path applies first), the tile is read back 16
  // bytes per lane along rows, and the epilogue operand is read the same way.
  if constexpr (WN_ == 4) {
    if (!p.out_f32 && (PIPE || p.epi == MK_EPI_NONE || p.epi == MK_EPI_SWIGLU_PAIRS)) {
      constexpr int SROW = kEpiStageRow;  // staged row stride (544 B: consecutive rows 8 banks apart)
      uint16_t* st = reinterpret_cast<uint16_t*>(smem);
      __syncthreads();  // every wave is done with the ring
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          *reinterpret_cast<u32x2*>(st + (wm * (16 * TM) + 16 * i + (lane & 15)) * SROW + wn * (16 * TN) + 16 * j +
                                    4 * (lane >> 4)) =
              u32x2{pack_bf16x2(acc[i][j].x, acc[i][j].y), pack_bf16x2(acc[i][j].z, acc[i][j].w)};
      __syncthreads();
      auto f4 = [](uint32_t lo, uint32_t hi) {
        return f32x4{bf16_to_f32(lo & 0xffffu), bf16_to_f32(lo >> 16), bf16_to_f32(hi & 0xffffu),
                     bf16_to_f32(hi >> 16)};
      };
      uint16_t* C = static_cast<uint16_t*>(p.c) + (size_t)blockIdx.z * p.sc;
      if (p.epi == MK_EPI_SWIGLU_PAIRS) {
        // Output column o of the tile: gate at staged column 32 (o / 16) +
        // o % 16, up 16 further.  16 lanes cover a 128-column output row.
        const int N2 = N / 2;
#pragma unroll 2
        for (int r = 0; r < BM / 32; ++r) {
          const int row = 32 * r + (tid >> 4), o = 8 * (tid & 15);
          const uint16_t* sp = st + row * SROW + 32 * (o >> 4) + (o & 15);
          const u32x4 g = *reinterpret_cast<const u32x4*>(sp);
          const u32x4 u = *reinterpret_cast<const u32x4*>(sp + 16);
          const size_t off = (size_t)(m0 + row) * N2 + n0 / 2 + o;
          epi_store_swiglu_pair(C, off, f4(g.x, g.y), f4(u.x, u.y));
          epi_store_swiglu_pair(C, off + 4, f4(g.z, g.w), f4(u.z, u.w));
        }
      } else {
        const uint16_t* X = p.aux + (size_t)blockIdx.z * p.sc;
#pragma unroll 2
        for (int r = 0; r < BM / 16; ++r) {
          const int row = 16 * r + (tid >> 5), c8 = 8 * (tid & 31);
          const u32x4 v = *reinterpret_cast<const u32x4*>(st + row * SROW + c8);
          const size_t off = (size_t)(m0 + row) * N + n0 + c8;
          if (p.epi == MK_EPI_NONE) {
            *reinterpret_cast<u32x4*>(C + off) = v;
          } else {
            const u32x4 w = *reinterpret_cast<const u32x4*>(X + off);
            epi_store_bf16x4_v(C, u32x2{w.x, w.y}, p.epi, off, f4(v.x, v.y));
            epi_store_bf16x4_v(C, u32x2{w.z, w.w}, p.epi, off + 4, f4(v.z, v.w));
          }
        }
      }
      return;
    }
  }

  // Epilogue (C^T tiles): lane owns row m, columns n..n+3 of each tile.
  if (p.epi == MK_EPI_SWIGLU_PAIRS) {
    // Blocks j (gate) and j+1 (up), j even, hold the same output columns.
    uint16_t* C = static_cast<uint16_t*>(p.c) + (size_t)blockIdx.z * p.sc;
    const int N2 = N / 2, ncol2 = ncol / 2 + 2 * (lane >> 4);  // = n0/2 + wn*8*TN + 4*(lane>>4)
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int q = 0; q < TN / 2; ++q)
        epi_store_swiglu_pair(C, (size_t)(mrow + 16 * i) * N2 + ncol2 + 16 * q, acc[i][2 * q], acc[i][2 * q + 1]);
  } else if (p.out_f32) {
    float* C = static_cast<float*>(p.c) + (size_t)blockIdx.z * p.sc;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
        *reinterpret_cast<f32x4*>(C + (size_t)(mrow + 16 * i) * N + ncol + 16 * j) = acc[i][j];
  } else {
    uint16_t* C = static_cast<uint16_t*>(p.c) + (size_t)blockIdx.z * p.sc;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const size_t off = (size_t)(mrow + 16 * i) * N + ncol + 16 * j;
        if constexpr (kPreAux)
          epi_store_bf16x4_v(C, auxv[i][j], p.epi, off, acc[i][j]);
        else
          epi_store_bf16x4(C, p.aux + (size_t)blockIdx.z * p.sc, p.epi, off, acc[i][j]);
      }
  }
}

// ---------------------------------------------------------------------------
// Short-K kernel (K <= 256, e.g. the batched [2048,128] x [128,2048] product):
// output-store bound, the 256 x 256 kernel runs one workgroup per CU and
// serialises its loads, its 128 KB of MFMA work and its 128 KB of stores.
// Here a 128 x 128 tile keeps all of K in LDS (16 KB per 32 k: A [128][32]
// then B [32][128], the same chunk swizzles as above), so at K = 128 a
// workgroup takes 64 KB and two run on a CU: one's stores drain while the
// other loads and multiplies.  Four waves of 64 x 64 (4 x 4 MFMA tiles); all
// DMAs are issued up front and each 32-k stage is multiplied once it has
// landed.  The bf16 tile is then staged in LDS over A / B (rows of 272 B) and
// written out in 256-byte row pieces, with the ADD / SWIGLU epilogue applied
// on the way.  Each k runs in the same order in the same MFMA as in the 256
// x 256 kernels, so the f32 accumulators, and the bf16 results, are the
// same bits.
// ---------------------------------------------------------------------------
constexpr int kShortStageBytes = 16 * 1024;
constexpr int kShortEpiRow = 136;  // bf16 per staged row (128 + 8 pad: consecutive rows 4 banks apart)
constexpr int kShortEpiBytes = 128 * kShortEpiRow * 2;

__host__ __device__ constexpr int short_lds_bytes(int kt) {
  return kt * kShortStageBytes > kShortEpiBytes ? kt * kShortStageBytes : kShortEpiBytes;
}

template <int KT>
__global__ __launch_bounds__(256) void gemm_bf16_shortk_kernel(GemmArgs p) {
  constexpr int BM = 128, BN = 128, BK = 32, TM = 4, TN = 4;
  constexpr int ABYTES = BM * BK * 2;  // 8 KB
  extern __shared__ __align__(16) unsigned char smem[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int tiles_m = p.M / BM, tiles_n = p.N / BN;
  int tm, tn;
  tile_coords(xcd_logical_id(blockIdx.x, gridDim.x), tiles_m, tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int K = p.K, N = p.N;
  const uint16_t* A = static_cast<const uint16_t*>(p.a) + (size_t)blockIdx.z * p.sa + (size_t)m0 * K;
  const uint16_t* B = static_cast<const uint16_t*>(p.b) + (size_t)blockIdx.z * p.sb + n0;
  const uint32_t sbase = lds_addr(smem);

  // DMA, per 32-k stage, 8 A and 8 B instructions of 1 KB, two of each per
  // wave.  A instruction i: lane L fills row 16i + L/4, 16-byte chunk L%4.
  // B instruction i: lane L fills k row 4i + L/16, chunk L%16.
  {
    const uint16_t* asrc[2];
    const uint16_t* bsrc[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int i = 2 * wave + u;
      const int row = 16 * i + (lane >> 2), pa = lane & 3;
      asrc[u] = A + (size_t)row * K + 8 * (pa ^ ((row >> 1) & 3));
      const int kr = 4 * i + (lane >> 4), pb = lane & 15;
      bsrc[u] = B + (size_t)kr * N + 8 * swz_b2(kr, pb);
    }
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
      const uint32_t st = sbase + (uint32_t)(kt * kShortStageBytes);
#pragma unroll
      for (int u = 0; u < 2; ++u) dma16_asm(asrc[u] + kt * BK, st + (uint32_t)((2 * wave + u) * 1024));
#pragma unroll
      for (int u = 0; u < 2; ++u)
        dma16_asm(bsrc[u] + (size_t)kt * BK * N, st + (uint32_t)(ABYTES + (2 * wave + u) * 1024));
    }
  }

  // Fragment offsets within a stage (as in the 256 x 256 kernel, for 128-row
  // A stages and 256-byte B rows).
  const int arow = wm * 64 + (lane & 15);
  const int aoff = arow * 64 + 16 * ((lane >> 4) ^ ((arow >> 1) & 3));
  int boff[2 * TN];
  {
    const int g = lane >> 4, r = (lane & 15) >> 2, q = lane & 3;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int col = wn * 64 + 16 * j + 4 * q;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int k1 = 8 * g + r + 4 * h;
        boff[2 * j + h] = ABYTES + k1 * (BN * 2) + 16 * swz_b2(k1, col >> 3) + 2 * (col & 7);
      }
    }
  }

  f32x4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int kt = 0; kt < KT; ++kt) {
    // This wave's DMAs of stages 0..kt have landed (4 per stage, in order).
    vm_wait(4 * (KT - 1 - kt));
    asm volatile("s_barrier" ::: "memory");
    const unsigned char* st = smem + kt * kShortStageBytes;
    u32x4 bf[TN];
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_ptr)(st + boff[2 * j]));
      const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_ptr)(st + boff[2 * j + 1]));
      const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
      bf[j] = u32x4{l2.x, l2.y, h2.x, h2.y};
    }
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const u32x4 af = *reinterpret_cast<const u32x4*>(st + aoff + 1024 * i);
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] = mfma16x16x32(bf[j], af, acc[i][j]);
    }
  }

  // Stage the bf16 tile over the operands (lane: row lane & 15 of its 16-row
  // block, columns 4 (lane >> 4) .. +3 of its 16-column block), then write
  // rows out 16 bytes per lane.
  uint16_t* stg = reinterpret_cast<uint16_t*>(smem);
  __syncthreads();
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
      *reinterpret_cast<u32x2*>(stg + (wm * 64 + 16 * i + (lane & 15)) * kShortEpiRow + wn * 64 + 16 * j +
                                4 * (lane >> 4)) =
          u32x2{pack_bf16x2(acc[i][j].x, acc[i][j].y), pack_bf16x2(acc[i][j].z, acc[i][j].w)};
  __syncthreads();
  uint16_t* C = static_cast<uint16_t*>(p.c) + (size_t)blockIdx.z * p.sc;
  const uint16_t* X = p.aux ? p.aux + (size_t)blockIdx.z * p.sc : nullptr;
  auto f4 = [](uint32_t lo, uint32_t hi) {
    return f32x4{bf16_to_f32(lo & 0xffffu), bf16_to_f32(lo >> 16), bf16_to_f32(hi & 0xffffu), bf16_to_f32(hi >> 16)};
  };
#pragma unroll 4
  for (int r = 0; r < BM / 16; ++r) {
    const int row = 16 * r + (tid >> 4), c8 = 8 * (tid & 15);
    const u32x4 v = *reinterpret_cast<const u32x4*>(stg + row * kShortEpiRow + c8);
    const size_t off = (size_t)(m0 + row) * N + n0 + c8;
    if (p.epi == MK_EPI_NONE) {
      *reinterpret_cast<u32x4*>(C + off) = v;
    } else {
      const u32x4 w = *reinterpret_cast<const u32x4*>(X + off);
      epi_store_bf16x4_v(C, u32x2{w.x, w.y}, p.epi, off, f4(v.x, v.y));
      epi_store_bf16x4_v(C, u32x2{w.z, w.w}, p.epi, off + 4, f4(v.z, v.w));
    }
  }
}

// ---------------------------------------------------------------------------
// Persistent short-K kernel (K <= 128): 256 x 256 tiles as in the kernel
// above (2 x 4 waves of 128 x 64, the same stage layout, swizzles and MFMA
// order, so the same bits), one workgroup per CU walking tiles t, t + grid,
// ....  All of K fits the ring (KT stages of 32 KB), so as soon as a tile's
// MFMAs are done the next tile's DMAs are issued, and the current tile is
// stored while they are in flight: loads, MFMAs and the 128 KB of stores of
// consecutive tiles overlap instead of following each other.  The stores go
// through a 2 KB LDS buffer per wave (16 rows x 128 B, 16-byte chunks XOR
// row % 8): each 16 x 64 block of the wave's accumulators is written 8 bytes
// per lane and read back as full 128-byte row pieces, with no workgroup
// barrier, so the ring is never touched by the epilogue.
// ---------------------------------------------------------------------------
constexpr int kPersistWaveStage = 2048;

__host__ __device__ constexpr int persist_lds_bytes(int kt) { return kt * kGemmStageBytes + 8 * kPersistWaveStage; }

template <int KT>
__global__ __launch_bounds__(512) void gemm_bf16_persist_kernel(GemmArgs p, int batch) {
  constexpr int BM = 256, BN = 256, BK = 32, TM = 8, TN = 4, DI = 2;
  constexpr int ABYTES = BM * BK * 2;  // 16 KB
  extern __shared__ __align__(16) unsigned char smem[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 2, wn = wave & 3;
  const int tiles_m = p.M / BM, tiles_n = p.N / BN, per_batch = tiles_m * tiles_n;
  const int total = per_batch * batch;
  const int K = p.K, N = p.N;
  const uint32_t sbase = lds_addr(smem);
  unsigned char* wstage = smem + KT * kGemmStageBytes + wave * kPersistWaveStage;

  auto coords = [&](int t, int& z, int& m0, int& n0) {
    z = t / per_batch;
    int tm, tn;
    tile_coords((uint32_t)(t - z * per_batch), tiles_m, tiles_n, tm, tn);
    m0 = tm * BM;
    n0 = tn * BN;
  };
  // DMA of all KT stages of tile t (as the ring kernel: A instruction i fills
  // rows 16i..16i+15, B instruction i k rows 2i, 2i+1; two of each per wave).
  auto issue = [&](int t) {
    int z, m0, n0;
    coords(t, z, m0, n0);
    const uint16_t* A = static_cast<const uint16_t*>(p.a) + (size_t)z * p.sa + (size_t)m0 * K;
    const uint16_t* B = static_cast<const uint16_t*>(p.b) + (size_t)z * p.sb + n0;
#pragma unroll
    for (int u = 0; u < DI; ++u) {
      const int i = DI * wave + u;
      const int row = 16 * i + (lane >> 2), pa = lane & 3;
      const uint16_t* as = A + (size_t)row * K + 8 * (pa ^ ((row >> 1) & 3));
      const int kr = 2 * i + (lane >> 5), pb = lane & 31;
      const uint16_t* bs = B + (size_t)kr * N + 8 * swz_b2(kr, pb);
#pragma unroll
      for (int kt = 0; kt < KT; ++kt) {
        const uint32_t st = sbase + (uint32_t)(kt * kGemmStageBytes);
        dma16_asm(as + kt * BK, st + (uint32_t)(i * 1024));
        dma16_asm(bs + (size_t)kt * BK * N, st + (uint32_t)(ABYTES + i * 1024));
      }
    }
  };

  const int arow = wm * 128 + (lane & 15);
  const int aoff = arow * 64 + 16 * ((lane >> 4) ^ ((arow >> 1) & 3));
  int boff[2 * TN];
  {
    const int g = lane >> 4, r = (lane & 15) >> 2, q = lane & 3;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int col = wn * 64 + 16 * j + 4 * q;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int k1 = 8 * g + r + 4 * h;
        boff[2 * j + h] = ABYTES + k1 * (BN * 2) + 16 * swz_b2(k1, col >> 3) + 2 * (col & 7);
      }
    }
  }
  // Wave staging: element (row, col) of a 16 x 64 block at row * 128 +
  // 16 * ((col / 8) ^ (row % 8)) + 2 * (col % 8).
  const int sr = lane & 15, sg = lane >> 4;
  const int rrow = lane >> 3, rchunk = lane & 7;
  auto f4 = [](uint32_t lo, uint32_t hi) {
    return f32x4{bf16_to_f32(lo & 0xffffu), bf16_to_f32(lo >> 16), bf16_to_f32(hi & 0xffffu), bf16_to_f32(hi >> 16)};
  };

  int t = blockIdx.x;
  if (t < total) issue(t);
  for (; t < total; t += gridDim.x) {
    // Tile t's operands have landed (and the previous tile's stores are done).
    vm_wait(0);
    asm volatile("s_barrier" ::: "memory");
    f32x4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
      const unsigned char* st = smem + kt * kGemmStageBytes;
      u32x4 bf[TN];
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_ptr)(st + boff[2 * j]));
        const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_ptr)(st + boff[2 * j + 1]));
        const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
        bf[j] = u32x4{l2.x, l2.y, h2.x, h2.y};
      }
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const u32x4 af = *reinterpret_cast<const u32x4*>(st + aoff + 1024 * i);
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = mfma16x16x32(bf[j], af, acc[i][j]);
      }
    }
    // Every wave's fragment reads of this tile are done: the ring is free.
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    if (t + (int)gridDim.x < total) issue(t + gridDim.x);

    int z, m0, n0;
    coords(t, z, m0, n0);
    uint16_t* C = static_cast<uint16_t*>(p.c) + (size_t)z * p.sc;
    const uint16_t* X = p.aux ? p.aux + (size_t)z * p.sc : nullptr;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int col = 16 * j + 4 * sg;
        *reinterpret_cast<u32x2*>(wstage + sr * 128 + 16 * ((col >> 3) ^ (sr & 7)) + 2 * (col & 7)) =
            u32x2{pack_bf16x2(acc[i][j].x, acc[i][j].y), pack_bf16x2(acc[i][j].z, acc[i][j].w)};
      }
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int row = rrow + 8 * h;
        const u32x4 v = *reinterpret_cast<const u32x4*>(wstage + row * 128 + 16 * (rchunk ^ (row & 7)));
        const size_t off = (size_t)(m0 + wm * 128 + 16 * i + row) * N + n0 + wn * 64 + 8 * rchunk;
        if (p.epi == MK_EPI_NONE) {
          *reinterpret_cast<u32x4*>(C + off) = v;
        } else {
          const u32x4 w = *reinterpret_cast<const u32x4*>(X + off);
          epi_store_bf16x4_v(C, u32x2{w.x, w.y}, p.epi, off, f4(v.x, v.y));
          epi_store_bf16x4_v(C, u32x2{w.z, w.w}, p.epi, off + 4, f4(v.z, v.w));
        }
      }
    }
  }
}

}  // namespace mk

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
#include "../capi_internal.h"

#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <vector>

namespace {

hipError_t lds_opt_in(const void* fn, size_t bytes) {
  if (bytes <= 64 * 1024) return hipSuccess;
  return hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
}

template <int BM, int BN, int WM, int WN>
hipError_t launch_bf16(const mk::GemmArgs& a, int batch, hipStream_t st) {
  constexpr size_t lds = (size_t)2 * (BM + BN) * (64 + 8) * 2;
  const void* fn = (const void*)mk::gemm_bf16_kernel<BM, BN, WM, WN>;
  hipError_t e = lds_opt_in(fn, lds);
  if (e != hipSuccess) return e;
  const int tiles = ((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
  hipLaunchKernelGGL((mk::gemm_bf16_kernel<BM, BN, WM, WN>), dim3(tiles, 1, batch),
                     dim3(WM * WN * 64), lds, st, a);
  return hipGetLastError();
}

template <int BM, int BN, int WM, int WN>
hipError_t launch_f32(const mk::GemmArgs& a, int batch, hipStream_t st) {
  constexpr size_t lds = (size_t)2 * (BM + BN) * (32 + 4) * 4;
  const void* fn = (const void*)mk::gemm_f32_kernel<BM, BN, WM, WN>;
  hipError_t e = lds_opt_in(fn, lds);
  if (e != hipSuccess) return e;
  const int tiles = ((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
  hipLaunchKernelGGL((mk::gemm_f32_kernel<BM, BN, WM, WN>), dim3(tiles, 1, batch),
                     dim3(WM * WN * 64), lds, st, a);
  return hipGetLastError();
}

int check_gemm(const char* fn, const void* a, const void* b, void* c, int64_t batch, int64_t M,
               int64_t N, int64_t K) {
  if (!a || !b || !c) return mkc::fail(MK_EINVAL, "%s: null pointer argument", fn);
  if (batch <= 0 || M <= 0 || N <= 0 || K <= 0)
    return mkc::fail(MK_EINVAL, "%s: batch, M, N, K must be positive (got %lld, %lld, %lld, %lld)",
                     fn, (long long)batch, (long long)M, (long long)N, (long long)K);
  if (K % 8 != 0 || N % 8 != 0)
    return mkc::fail(MK_EUNSUPPORTED, "%s: needs K %% 8 == 0 and N %% 8 == 0 (got K=%lld, N=%lld)",
                     fn, (long long)K, (long long)N);
  // Every kernel's grid (64-row tiles at the smallest, times the batch for
  // the persistent kernel's tile count) stays below 2^31 workgroups.
  if (M > (1 << 24) || N > (1 << 24) || K > (1 << 24) || batch > 65535 || M * K > ((int64_t)1 << 40) ||
      ((M + 63) / 64) * ((N + 63) / 64) * batch > (int64_t)INT32_MAX)
    return mkc::fail(MK_EINVAL, "%s: shape too large", fn);
  return MK_OK;
}

// Compute units of the current device (queried once per device).
int device_cus() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int v = cache[dev].load(std::memory_order_relaxed);
  if (v > 0) return v;
  if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
  cache[dev].store(v, std::memory_order_relaxed);
  return v;
}

int env_int_gemm(const char* name, int dflt) {
  const char* v = getenv(name);
  return v ? atoi(v) : dflt;
}

int env_tile() {
  const char* v = getenv("MK_GEMM_TILE");
  return v ? atoi(v) : 0;
}

}  // namespace

namespace {

// bt: b is B^T [N, K] (only the DMA-fed 256 x 256 kernel takes it).
// Routes: the kernel choices of the [K, N] bf16 product (MK_GEMM_ROUTE_*).
// Every route computes each output's k in the same order in the same MFMA,
// so all of them give the same bits; they differ only in speed.
bool route_fits(int route, int64_t M, int64_t N, int64_t K, int epi, int out_f32) {
  const bool a256 = M % 256 == 0 && N % 256 == 0;
  const bool simple_epi = epi == MK_EPI_NONE || epi == MK_EPI_ADD || epi == MK_EPI_SWIGLU;
  switch (route) {
    case MK_GEMM_ROUTE_RING:
      return a256 && K % 32 == 0;
    case MK_GEMM_ROUTE_PIPE:
      return a256 && K % 32 == 0 && K >= 2 * 32 * mk::kPipeStages;
    case MK_GEMM_ROUTE_PERSIST:
      return a256 && K % 32 == 0 && K <= 128 && !out_f32 && simple_epi;
    case MK_GEMM_ROUTE_SHORT:
      return M % 128 == 0 && N % 128 == 0 && K % 32 == 0 && K <= 256 && !out_f32 && simple_epi;
    case MK_GEMM_ROUTE_REG256:
      return a256 && K % 64 == 0 && simple_epi;
    case MK_GEMM_ROUTE_GENERIC256:
    case MK_GEMM_ROUTE_GENERIC128:
      return simple_epi;
    default:
      return false;
  }
}

// The built-in choice (what MK_GEMM_* environment knobs steer), from
// timings with operands rotated past the 256 MB Infinity Cache (one box,
// us):
//   - K >= 512 on 256-multiples: the pipelined kernel (fragment prefetch,
//     5-stage ring) at any tile count: 2048^3 51.1 against 54.2 (128-tile
//     kernel) / 58.6 (ring); 1024^3 28.4 / 28.6 / 31.8; 16 x 1024^3 42.9 /
//     77.3 / 45.2; 8192^2 x 1024 151.6 / 288.2 / 153.4; 256 x 14336 x 4096
//     102.1 / 103.5 / 106.7 (8 x 512^2 x 4096: 106.4 / 103.7 / 114.0).  It
//     runs at a lower clock (GRBM_GUI_ACTIVE per ns ~2.1 against
//     ~2.35 GHz), which slows the kernels around it; in the decoder (K
//     2048 and 8192) it still gains end to end: QKV and paired gate/up 2 %
//     (5.00 vs 5.09 ms), the output and down projections another 2.5 %
//     (4.82 vs 4.95 ms).  MK_GEMM_PIPE_K moves the threshold, MK_GEMM_PIPE=0
//     keeps the ring kernel.
//   - K <= 256 with fewer 256 x 256 tiles than CUs: the 128 x 128 kernel
//     with all of K in LDS: 2048^2 x 256 7.9 against 12.1 (128-tile
//     kernel); 1024^2 x 256 5.7 / 10.5; 4 x 1024^2 x 128 6.1 / 9.1 (9.9
//     persistent).
//   - K <= 128 with a tile per CU or more: the persistent kernel (the next
//     tile's loads under the current tile's stores): 16 x 2048^2 x 128 48.5
//     against 54.2 (ring) / 58.6 (128 x 128 all-K-in-LDS).
//     MK_GEMM_PERSIST=0 turns it off.
//   - MK_GEMM_SHORTK sets the largest K of the 128 x 128 all-K-in-LDS
//     kernel (default 256 on 256-multiples, 128 on other 128-multiples;
//     0: never).
int default_route(int64_t batch, int64_t M, int64_t N, int64_t K, int epi, int out_f32) {
  const char* dma_env = getenv("MK_GEMM_DMA");
  const bool dma = !(dma_env && dma_env[0] == '0');
  const bool simple_epi = epi == MK_EPI_NONE || epi == MK_EPI_ADD || epi == MK_EPI_SWIGLU;
  const int64_t big_tiles = ((M + 255) / 256) * ((N + 255) / 256) * batch;
  const int env_t = env_tile();
  int tile = env_t;
  if (tile == 0) tile = big_tiles >= 128 ? 256 : 128;
  if (epi == MK_EPI_SWIGLU_PAIRS) tile = 256;
  const bool a256 = M % 256 == 0 && N % 256 == 0 && K % 32 == 0;
  const char* sk = getenv("MK_GEMM_SHORTK");
  const int64_t shortk_max = std::min<int64_t>(sk ? atoll(sk) : (a256 ? 256 : 128), 256);
  const char* pe = getenv("MK_GEMM_PERSIST");
  const bool persist_on = !(pe && pe[0] == '0') && dma;
  const int cus = device_cus();
  if (a256 && env_t == 0 && persist_on && big_tiles >= cus && route_fits(MK_GEMM_ROUTE_PERSIST, M, N, K, epi, out_f32))
    return MK_GEMM_ROUTE_PERSIST;
  if (K <= shortk_max && (!a256 || big_tiles < cus || !persist_on) && env_t == 0 &&
      route_fits(MK_GEMM_ROUTE_SHORT, M, N, K, epi, out_f32))
    return MK_GEMM_ROUTE_SHORT;
  const char* pv = getenv("MK_GEMM_PIPE");
  const char* pk = getenv("MK_GEMM_PIPE_K");
  const int64_t pipe_k = pk ? atoll(pk) : 512;
  const bool pipe = !(pv && atoi(pv) == 0) && K >= pipe_k && route_fits(MK_GEMM_ROUTE_PIPE, M, N, K, epi, out_f32);
  if (dma && a256 && (tile == 256 || (pipe && env_t == 0)))
    return pipe ? MK_GEMM_ROUTE_PIPE : MK_GEMM_ROUTE_RING;
  if (!simple_epi) return MK_GEMM_ROUTE_RING;  // paired SwiGLU: checked aligned by the caller
  if (tile == 256 && route_fits(MK_GEMM_ROUTE_REG256, M, N, K, epi, out_f32)) return MK_GEMM_ROUTE_REG256;
  return tile == 256 ? MK_GEMM_ROUTE_GENERIC256 : MK_GEMM_ROUTE_GENERIC128;
}

hipError_t launch_route(int route, const mk::GemmArgs& p, int64_t batch, hipStream_t st) {
  hipError_t e = hipErrorInvalidValue;
  const int64_t M = p.M, N = p.N, K = p.K;
  const char* w = getenv("MK_GEMM_WAVES");
  const bool four_waves = w && atoi(w) == 4;
  switch (route) {
    case MK_GEMM_ROUTE_PERSIST: {
      const int64_t total = (M / 256) * (N / 256) * batch;
      const dim3 grid((unsigned)std::min<int64_t>(total, device_cus()));
      switch (K / 32) {
#define MK_PERSIST_CASE(KT)                                                                              \
  case KT:                                                                                               \
    e = lds_opt_in((const void*)mk::gemm_bf16_persist_kernel<KT>, (size_t)mk::persist_lds_bytes(KT));   \
    if (e == hipSuccess)                                                                                 \
      hipLaunchKernelGGL((mk::gemm_bf16_persist_kernel<KT>), grid, dim3(512), mk::persist_lds_bytes(KT), st, p, \
                         (int)batch);                                                                    \
    break;
        MK_PERSIST_CASE(1) MK_PERSIST_CASE(2) MK_PERSIST_CASE(3) MK_PERSIST_CASE(4)
#undef MK_PERSIST_CASE
        default: break;
      }
      break;
    }
    case MK_GEMM_ROUTE_SHORT: {
      const dim3 grid((unsigned)((M / 128) * (N / 128)), 1, (unsigned)batch);
      switch (K / 32) {
#define MK_SHORTK_CASE(KT)                                                                           \
  case KT:                                                                                           \
    e = lds_opt_in((const void*)mk::gemm_bf16_shortk_kernel<KT>, (size_t)mk::short_lds_bytes(KT));  \
    if (e == hipSuccess)                                                                             \
      hipLaunchKernelGGL((mk::gemm_bf16_shortk_kernel<KT>), grid, dim3(256), mk::short_lds_bytes(KT), st, p); \
    break;
        MK_SHORTK_CASE(1) MK_SHORTK_CASE(2) MK_SHORTK_CASE(3) MK_SHORTK_CASE(4)
        MK_SHORTK_CASE(5) MK_SHORTK_CASE(6) MK_SHORTK_CASE(7) MK_SHORTK_CASE(8)
#undef MK_SHORTK_CASE
        default: break;
      }
      break;
    }
    case MK_GEMM_ROUTE_RING:
    case MK_GEMM_ROUTE_PIPE: {
      constexpr size_t lds = (size_t)mk::kGemmStages * mk::kGemmStageBytes;
      const dim3 grid((unsigned)((M / 256) * (N / 256)), 1, (unsigned)batch);
      if (four_waves) {
        e = lds_opt_in((const void*)mk::gemm_bf16_256dma_kernel<2, false>, lds);
        if (e == hipSuccess) hipLaunchKernelGGL((mk::gemm_bf16_256dma_kernel<2, false>), grid, dim3(256), lds, st, p);
      } else if (route == MK_GEMM_ROUTE_PIPE) {
        constexpr size_t lds_p = (size_t)mk::kPipeStages * mk::kGemmStageBytes;
        e = lds_opt_in((const void*)mk::gemm_bf16_256dma_kernel<4, true>, lds_p);
        if (e == hipSuccess) hipLaunchKernelGGL((mk::gemm_bf16_256dma_kernel<4, true>), grid, dim3(512), lds_p, st, p);
      } else {
        // The ring takes 128 KB; the staged epilogue tile needs 136 KB (one
        // workgroup per CU either way).
        constexpr size_t lds4 = lds > (size_t)mk::kEpiStageBytes ? lds : (size_t)mk::kEpiStageBytes;
        e = lds_opt_in((const void*)mk::gemm_bf16_256dma_kernel<4, false>, lds4);
        if (e == hipSuccess) hipLaunchKernelGGL((mk::gemm_bf16_256dma_kernel<4, false>), grid, dim3(512), lds4, st, p);
      }
      break;
    }
    case MK_GEMM_ROUTE_REG256: {
      constexpr size_t lds = (size_t)2 * (256 * 64 + 64 * 256) * 2;
      const dim3 grid((unsigned)((M / 256) * (N / 256)), 1, (unsigned)batch);
      if (four_waves) {
        e = lds_opt_in((const void*)mk::gemm_bf16_256_kernel<2, 2>, lds);
        if (e == hipSuccess) hipLaunchKernelGGL((mk::gemm_bf16_256_kernel<2, 2>), grid, dim3(256), lds, st, p);
      } else {
        e = lds_opt_in((const void*)mk::gemm_bf16_256_kernel<2, 4>, lds);
        if (e == hipSuccess) hipLaunchKernelGGL((mk::gemm_bf16_256_kernel<2, 4>), grid, dim3(512), lds, st, p);
      }
      break;
    }
    case MK_GEMM_ROUTE_GENERIC256:
      return launch_bf16<256, 256, 2, 2>(p, (int)batch, st);
    case MK_GEMM_ROUTE_GENERIC128:
      return launch_bf16<128, 128, 2, 2>(p, (int)batch, st);
    default:
      return hipErrorInvalidValue;
  }
  if (e == hipSuccess) e = hipGetLastError();
  return e;
}

int run_gemm_bf16(const char* fn, const void* a, const void* b, void* c, const void* aux, int epi, int64_t batch,
                  int64_t M, int64_t N, int64_t K, int out_f32, void* stream, bool bt = false,
                  int route = MK_GEMM_ROUTE_DEFAULT) {
  mkc::clear_error();
  int rc = check_gemm(fn, a, b, c, batch, M, N, K);
  if (rc != MK_OK) return rc;
  if (epi != MK_EPI_NONE && epi != MK_EPI_ADD && epi != MK_EPI_SWIGLU && epi != MK_EPI_SWIGLU_PAIRS)
    return mkc::fail(MK_EINVAL, "%s: unknown epilogue %d", fn, epi);
  if (epi != MK_EPI_NONE && (out_f32 || (!aux && epi != MK_EPI_SWIGLU_PAIRS)))
    return mkc::fail(MK_EINVAL, "%s: an epilogue needs a bf16 output and an aux operand", fn);
  const char* dma_env = getenv("MK_GEMM_DMA");
  const bool dma = !(dma_env && dma_env[0] == '0');
  if (bt && !(M % 256 == 0 && N % 256 == 0 && K % 32 == 0))
    return mkc::fail(MK_EUNSUPPORTED, "%s: needs M %% 256 == 0, N %% 256 == 0, K %% 32 == 0 "
                     "(got M=%lld, N=%lld, K=%lld)", fn, (long long)M, (long long)N, (long long)K);
  if (epi == MK_EPI_SWIGLU_PAIRS && !(dma && M % 256 == 0 && N % 256 == 0 && K % 32 == 0))
    return mkc::fail(MK_EUNSUPPORTED, "%s: paired SwiGLU needs M %% 256 == 0, N %% 256 == 0, K %% 32 == 0 "
                     "(got M=%lld, N=%lld, K=%lld)", fn, (long long)M, (long long)N, (long long)K);
  mk::GemmArgs p;
  p.a = a; p.b = b; p.c = c;
  p.M = (int)M; p.N = (int)N; p.K = (int)K;
  p.sa = M * K; p.sb = K * N; p.sc = epi == MK_EPI_SWIGLU_PAIRS ? M * (N / 2) : M * N;
  p.out_f32 = out_f32 ? 1 : 0;
  p.epi = epi;
  p.aux = static_cast<const uint16_t*>(aux);
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipError_t e;
  if (bt) {
    const dim3 grid((unsigned)((M / 256) * (N / 256)), 1, (unsigned)batch);
    const char* pv = getenv("MK_GEMM_PIPE");
    const char* pk = getenv("MK_GEMM_PIPE_K");
    const int64_t pipe_k = pk ? atoll(pk) : 2048;
    if (!(pv && atoi(pv) == 0) && K >= pipe_k && K >= 2 * 32 * mk::kPipeStages) {
      constexpr size_t lds_p = (size_t)mk::kPipeStages * mk::kGemmStageBytes;
      e = lds_opt_in((const void*)mk::gemm_bf16_256dma_kernel<4, true, true>, lds_p);
      if (e == hipSuccess)
        hipLaunchKernelGGL((mk::gemm_bf16_256dma_kernel<4, true, true>), grid, dim3(512), lds_p, st, p);
    } else {
      constexpr size_t lds = (size_t)mk::kGemmStages * mk::kGemmStageBytes;
      constexpr size_t lds4 = lds > (size_t)mk::kEpiStageBytes ? lds : (size_t)mk::kEpiStageBytes;
      e = lds_opt_in((const void*)mk::gemm_bf16_256dma_kernel<4, false, true>, lds4);
      if (e == hipSuccess)
        hipLaunchKernelGGL((mk::gemm_bf16_256dma_kernel<4, false, true>), grid, dim3(512), lds4, st, p);
    }
    if (e == hipSuccess) e = hipGetLastError();
  } else {
    if (route == MK_GEMM_ROUTE_DEFAULT) route = default_route(batch, M, N, K, epi, out_f32);
    else if (!route_fits(route, M, N, K, epi, out_f32))
      return mkc::fail(MK_EUNSUPPORTED, "%s: route %d does not take this product (M=%lld, N=%lld, K=%lld, "
                       "epilogue %d, f32 output %d)", fn, route, (long long)M, (long long)N, (long long)K, epi,
                       out_f32);
    e = launch_route(route, p, batch, st);
  }
  if (e != hipSuccess) return mkc::fail(MK_ELAUNCH, "%s: launch failed: %s", fn, hipGetErrorString(e));
  return MK_OK;
}

}  // namespace

extern "C" int mk_gemm_bf16(const void* a, const void* b, void* c, int64_t batch, int64_t M,
                            int64_t N, int64_t K, int out_f32, void* stream) {
  return run_gemm_bf16("mk_gemm_bf16", a, b, c, nullptr, MK_EPI_NONE, batch, M, N, K, out_f32, stream);
}

extern "C" int mk_gemm_bf16_epilogue(const void* a, const void* b, void* c, const void* aux, int epilogue,
                                     int64_t batch, int64_t M, int64_t N, int64_t K, void* stream) {
  return run_gemm_bf16("mk_gemm_bf16_epilogue", a, b, c, aux, epilogue, batch, M, N, K, 0, stream);
}

extern "C" int mk_gemm_bf16_nt(const void* a, const void* bt, void* c, const void* aux, int epilogue,
                               int64_t batch, int64_t M, int64_t N, int64_t K, void* stream) {
  return run_gemm_bf16("mk_gemm_bf16_nt", a, bt, c, aux, epilogue, batch, M, N, K, 0, stream, true);
}


extern "C" int mk_gemm_bf16_route(const void* a, const void* b, void* c, const void* aux, int epilogue,
                                  int64_t batch, int64_t M, int64_t N, int64_t K, int out_f32, int route,
                                  void* stream) {
  if (route < MK_GEMM_ROUTE_DEFAULT || route >= MK_GEMM_ROUTE_COUNT)
    return mkc::fail(MK_EINVAL, "mk_gemm_bf16_route: unknown route %d", route);
  return run_gemm_bf16("mk_gemm_bf16_route", a, b, c, aux, epilogue, batch, M, N, K, out_f32, stream, false, route);
}

extern "C" int mk_gemm_bf16_route_fits(int route, int64_t M, int64_t N, int64_t K, int epilogue, int out_f32) {
  return route_fits(route, M, N, K, epilogue, out_f32) ? 1 : 0;
}

// ---------------------------------------------------------------------------
// Measured route choice.  A product is keyed by the device (architecture
// name and CU count) and its shape, epilogue class and output type; the
// table holds the fastest route measured for it and that time.
// ---------------------------------------------------------------------------
namespace {

struct TuneEntry {
  int route;
  float us;
};
std::mutex g_tune_mu;
std::map<std::string, TuneEntry> g_tune;

// "gfx950 256" of the current device, cached per device.
std::string device_tag() {
  static std::mutex mu;
  static std::map<int, std::string> tags;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return "none 0";
  std::lock_guard<std::mutex> g(mu);
  auto it = tags.find(dev);
  if (it != tags.end()) return it->second;
  hipDeviceProp_t prop;
  std::string tag = "none 0";
  if (hipGetDeviceProperties(&prop, dev) == hipSuccess) {
    std::string arch = prop.gcnArchName;
    arch = arch.substr(0, arch.find(':'));
    tag = arch + " " + std::to_string(prop.multiProcessorCount);
  }
  tags[dev] = tag;
  return tag;
}

// ADD and SWIGLU cost the same (one aux read per output); the paired form
// writes half the output.
int epi_class(int epi) { return epi == MK_EPI_NONE ? 0 : epi == MK_EPI_SWIGLU_PAIRS ? 2 : 1; }

std::string tune_key(const std::string& tag, int64_t batch, int64_t M, int64_t N, int64_t K, int ecls, int out_f32) {
  char buf[160];
  snprintf(buf, sizeof buf, "%s %lld %lld %lld %lld %d %d", tag.c_str(), (long long)batch, (long long)M,
           (long long)N, (long long)K, ecls, out_f32 ? 1 : 0);
  return buf;
}

// The table file's first line: the format version and this library's build
// stamp.  A table measured against another build of these kernels is refused,
// so a rebuilt library re-measures instead of following stale choices.
const std::string& tune_header() {
  static const std::string h = [] {
    std::string s = "mk-gemm-autotune 1 build ";
    for (const char* p = __DATE__ " " __TIME__; *p; ++p)  // "Dec  2 2026 10:11:12" -> "Dec_2_2026_10:11:12"
      if (*p != ' ') s += *p;
      else if (s.back() != '_') s += '_';
    return s;
  }();
  return h;
}

}  // namespace

extern "C" int mk_gemm_bf16_autotune(const void* a, const void* b, void* c, const void* aux, int epilogue,
                                     int64_t batch, int64_t M, int64_t N, int64_t K, int out_f32, void* stream,
                                     int* route_out, float* us_out) {
  const char* fn = "mk_gemm_bf16_autotune";
  mkc::clear_error();
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone)
    return mkc::fail(MK_EINVAL, "%s: cannot time launches under stream capture", fn);
  const int warm = std::max(0, env_int_gemm("MK_GEMM_AUTOTUNE_WARMUP", 2));
  const int iters = std::max(1, env_int_gemm("MK_GEMM_AUTOTUNE_ITERS", 5));
  if (aux && aux == c)
    return mkc::fail(MK_EINVAL, "%s: aux may not be c here (every timed launch rewrites c)", fn);
  hipEvent_t ev[2] = {nullptr, nullptr};
  if (hipEventCreate(&ev[0]) != hipSuccess || hipEventCreate(&ev[1]) != hipSuccess) {
    if (ev[0]) (void)hipEventDestroy(ev[0]);
    return mkc::fail(MK_ELAUNCH, "%s: event creation failed", fn);
  }
  int best = MK_GEMM_ROUTE_DEFAULT;
  float best_us = 0.f;
  int rc = MK_OK;
  for (int r = 1; r < MK_GEMM_ROUTE_COUNT && rc == MK_OK; ++r) {
    if (!route_fits(r, M, N, K, epilogue, out_f32)) continue;
    std::vector<float> t;
    for (int i = 0; i < warm + iters && rc == MK_OK; ++i) {
      if (i >= warm && hipEventRecord(ev[0], st) != hipSuccess) rc = mkc::fail(MK_ELAUNCH, "%s: event record", fn);
      if (rc == MK_OK) rc = run_gemm_bf16(fn, a, b, c, aux, epilogue, batch, M, N, K, out_f32, stream, false, r);
      if (rc == MK_OK && i >= warm) {
        float ms = 0.f;
        if (hipEventRecord(ev[1], st) != hipSuccess || hipEventSynchronize(ev[1]) != hipSuccess ||
            hipEventElapsedTime(&ms, ev[0], ev[1]) != hipSuccess)
          rc = mkc::fail(MK_ELAUNCH, "%s: event timing failed", fn);
        t.push_back(ms * 1e3f);
      }
    }
    if (rc != MK_OK) break;
    std::sort(t.begin(), t.end());
    const float med = t[t.size() / 2];
    if (best == MK_GEMM_ROUTE_DEFAULT || med < best_us) {
      best = r;
      best_us = med;
    }
  }
  (void)hipEventDestroy(ev[0]);
  (void)hipEventDestroy(ev[1]);
  if (rc != MK_OK) return rc;
  if (best == MK_GEMM_ROUTE_DEFAULT)
    return mkc::fail(MK_EUNSUPPORTED, "%s: no route takes this product", fn);
  // Leave c holding the chosen route's result (every route gives the same
  // bits; this keeps the contract independent of that).
  rc = run_gemm_bf16(fn, a, b, c, aux, epilogue, batch, M, N, K, out_f32, stream, false, best);
  if (rc != MK_OK) return rc;
  {
    std::lock_guard<std::mutex> g(g_tune_mu);
    g_tune[tune_key(device_tag(), batch, M, N, K, epi_class(epilogue), out_f32)] = TuneEntry{best, best_us};
  }
  if (route_out) *route_out = best;
  if (us_out) *us_out = best_us;
  return MK_OK;
}

extern "C" int mk_gemm_tuned_route(int64_t batch, int64_t M, int64_t N, int64_t K, int epilogue, int out_f32) {
  const std::string key = tune_key(device_tag(), batch, M, N, K, epi_class(epilogue), out_f32);
  std::lock_guard<std::mutex> g(g_tune_mu);
  auto it = g_tune.find(key);
  return it == g_tune.end() ? MK_GEMM_ROUTE_DEFAULT : it->second.route;
}

extern "C" int mk_gemm_autotune_save(const char* path) {
  mkc::clear_error();
  if (!path) return -mkc::fail(MK_EINVAL, "mk_gemm_autotune_save: null path");
  const std::string tmp = std::string(path) + ".tmp" + std::to_string((long long)getpid());
  FILE* f = fopen(tmp.c_str(), "w");
  if (!f) return -mkc::fail(MK_EINVAL, "mk_gemm_autotune_save: cannot write %s", tmp.c_str());
  int n = 0;
  {
    std::lock_guard<std::mutex> g(g_tune_mu);
    fprintf(f, "%s\n", tune_header().c_str());
    for (const auto& [k, v] : g_tune) {
      fprintf(f, "%s %d %.3f\n", k.c_str(), v.route, v.us);
      ++n;
    }
  }
  const bool ok = fflush(f) == 0 && fclose(f) == 0;
  if (!ok || rename(tmp.c_str(), path) != 0) {
    remove(tmp.c_str());
    return -mkc::fail(MK_EINVAL, "mk_gemm_autotune_save: cannot write %s", path);
  }
  return n;
}

// Merges the entries of a file written by mk_gemm_autotune_save (entries of
// other devices included; they are only looked up on such a device).
// Returns the number read, or -MK_EINVAL for a missing or malformed file.
extern "C" int mk_gemm_autotune_load(const char* path) {
  mkc::clear_error();
  if (!path) return -mkc::fail(MK_EINVAL, "mk_gemm_autotune_load: null path");
  FILE* f = fopen(path, "r");
  if (!f) return -mkc::fail(MK_EINVAL, "mk_gemm_autotune_load: cannot read %s", path);
  char line[256];
  const std::string& hdr = tune_header();
  if (!fgets(line, sizeof line, f) || strncmp(line, hdr.c_str(), hdr.size()) != 0 ||
      (line[hdr.size()] != '\n' && line[hdr.size()] != '\0')) {
    fclose(f);
    return -mkc::fail(MK_EINVAL, "mk_gemm_autotune_load: %s is not a route table of this build (header \"%s\")",
                      path, hdr.c_str());
  }
  std::vector<std::pair<std::string, TuneEntry>> got;
  int lineno = 1;
  while (fgets(line, sizeof line, f)) {
    ++lineno;
    char arch[64];
    int cus = 0, ecls = 0, of = 0, route = 0;
    long long b = 0, m = 0, n = 0, k = 0;
    float us = 0.f;
    char extra = 0;
    if (line[0] == '\n') continue;
    if (sscanf(line, "%63s %d %lld %lld %lld %lld %d %d %d %f %c", arch, &cus, &b, &m, &n, &k, &ecls, &of, &route,
               &us, &extra) != 10 || cus <= 0 || b <= 0 || m <= 0 || n <= 0 || k <= 0 || ecls < 0 || ecls > 2 ||
        (of != 0 && of != 1) || route <= MK_GEMM_ROUTE_DEFAULT || route >= MK_GEMM_ROUTE_COUNT || !(us >= 0.f)) {
      fclose(f);
      return -mkc::fail(MK_EINVAL, "mk_gemm_autotune_load: %s line %d is malformed", path, lineno);
    }
    got.emplace_back(tune_key(std::string(arch) + " " + std::to_string(cus), b, m, n, k, ecls, of),
                     TuneEntry{route, us});
  }
  fclose(f);
  std::lock_guard<std::mutex> g(g_tune_mu);
  for (auto& [key, v] : got) g_tune[key] = v;
  return (int)got.size();
}

extern "C" const char* mk_gemm_autotune_header(void) { return tune_header().c_str(); }

extern "C" void mk_gemm_autotune_clear(void) {
  std::lock_guard<std::mutex> g(g_tune_mu);
  g_tune.clear();
}

extern "C" int mk_gemm_f32(const void* a, const void* b, void* c, int64_t batch, int64_t M,
                           int64_t N, int64_t K, void* stream) {
  mkc::clear_error();
  int rc = check_gemm("mk_gemm_f32", a, b, c, batch, M, N, K);
  if (rc != MK_OK) return rc;
  mk::GemmArgs p;
  p.a = a; p.b = b; p.c = c;
  p.M = (int)M; p.N = (int)N; p.K = (int)K;
  p.sa = M * K; p.sb = K * N; p.sc = M * N;
  p.out_f32 = 1;
  p.epi = MK_EPI_NONE;
  p.aux = nullptr;
  // 128 x 128 tiles once they fill the chip (2048^3: 170 us against 183 us
  // with 64 x 64); below about 192 of them 64 x 64 tiles, four times as many
  // workgroups (1024^3: 35 us against 86 us).  Same k order, same bits.
  // MK_GEMM_F32_TILE=64 / 128 overrides.
  const int64_t t128 = ((M + 127) / 128) * ((N + 127) / 128) * batch;
  const char* ft = getenv("MK_GEMM_F32_TILE");
  const int tile = ft ? atoi(ft) : (t128 < 192 ? 64 : 128);
  hipError_t e = tile == 64 ? launch_f32<64, 64, 2, 2>(p, (int)batch, static_cast<hipStream_t>(stream))
                            : launch_f32<128, 128, 2, 2>(p, (int)batch, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return mkc::fail(MK_ELAUNCH, "mk_gemm_f32: launch failed: %s", hipGetErrorString(e));
  return MK_OK;
}
