// The pieces of the workload's Llama-style decoder layer that are not
// GEMMs, row reductions or plain elementwise chains, for gfx950:
//
//   * mk_rope_qkv_split_bf16: the fused QKV projection output [B*S, 3*H*D]
//     (column blocks q | k | v, each H heads of D, the reference layer's
//     reshape (B, T, 3, H, Dh), benchmarks/vs_cpu.py:603-610) split into
//     per-head q [B*H, S, D], k transposed kT [B*H, D, S] and v [B*H, S, D],
//     with rotary position embedding applied to q and k on the way
//     (rotate-half form: x[i] * cos - x[i + D/2] * sin, x[i + D/2] * cos +
//     x[i] * sin; cos/sin tables [S, D/2] in f32 from the caller).  kT is
//     what the batched NN GEMM needs for the scores q @ k^T.
//   * mk_softmax_causal_bf16: scores [B*H, S, S] -> probabilities, row i of
//     each S x S block keeping columns j <= i: p = exp(scale*s - m) / sum
//     (m, sum over j <= i) in f32, zeros above the diagonal.  Columns past
//     the diagonal are never read.
//   * mk_merge_heads_bf16: attention output [B*H, S, D] -> [B*S, H*D] (the
//     reference layer's transpose (0, 2, 1, 3) + reshape, vs_cpu.py:615).
//
// jax.jit lowers these parts to generic StableHLO (slices, concatenates,
// multiplies for the rotation; iota / compare / select for the mask;
// transposes), which the reference runs as MPSGraph ops; here each is one
// pass over memory with 16-byte accesses.
#include "common.h"

#include <math.h>

namespace mk {

typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4_t* lds_s16x4_t;

constexpr int kRopeTok = 64;  // tokens per workgroup of the split kernel
constexpr int kHeadDim = 128;

struct RopeArgs {
  const uint16_t* qkv;
  const float* cosb;
  const float* sinb;
  uint16_t* q;
  uint16_t* kT;
  uint16_t* v;
  int B, S, H;
  int k_rows;  // 1: k as [B*H, S, D] (for the attention kernel); 0: kT [B*H, D, S]
};

__device__ __forceinline__ void unpack8(const u32x4& w, float (&f)[8]) {
  const uint32_t a[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = bf16_to_f32(a[i] & 0xffffu);
    f[2 * i + 1] = bf16_to_f32(a[i] >> 16);
  }
}

__device__ __forceinline__ u32x4 pack8(const float (&f)[8]) {
  return u32x4{pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]), pack_bf16x2(f[4], f[5]), pack_bf16x2(f[6], f[7])};
}

// Workgroup: one (batch b, head h) and 64 consecutive tokens.  Thread t
// handles token s0 + t/4 and the 16-dimension slices 16 c .. +15 and
// 64 + 16 c .. +15 (c = t % 4), which are rotation partners.
__global__ __launch_bounds__(256) void rope_qkv_split_kernel(RopeArgs a) {
  constexpr int D = kHeadDim, HALF = D / 2;
  __shared__ __attribute__((aligned(16))) uint16_t kt[D][kRopeTok + 8];  // k of the tile, transposed (row pad 16 B)
  const int tid = threadIdx.x;
  const int tiles = a.S / kRopeTok;
  const int bh = blockIdx.x / tiles, s0 = (blockIdx.x - bh * tiles) * kRopeTok;
  const int b = bh / a.H, h = bh - b * a.H;
  const int tok = tid >> 2, c = tid & 3;
  const int s = s0 + tok;
  const int64_t row = (int64_t)(b * a.S + s) * (3 * a.H * D);
  const float* cs = a.cosb + (int64_t)s * HALF + 16 * c;
  const float* sn = a.sinb + (int64_t)s * HALF + 16 * c;
  float cv[16], sv[16];
#pragma unroll
  for (int i = 0; i < 16; i += 4) {
    const f32x4 c4 = *reinterpret_cast<const f32x4*>(cs + i);
    const f32x4 s4 = *reinterpret_cast<const f32x4*>(sn + i);
    cv[i] = c4.x; cv[i + 1] = c4.y; cv[i + 2] = c4.z; cv[i + 3] = c4.w;
    sv[i] = s4.x; sv[i + 1] = s4.y; sv[i + 2] = s4.z; sv[i + 3] = s4.w;
  }
  const int64_t out_row = ((int64_t)bh * a.S + s) * D;
#pragma unroll
  for (int part = 0; part < 3; ++part) {  // q, k, v
    const uint16_t* src = a.qkv + row + (int64_t)part * a.H * D + h * D;
    float lo[16], hi[16];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      float f[8];
      unpack8(*reinterpret_cast<const u32x4*>(src + 16 * c + 8 * u), f);
#pragma unroll
      for (int e = 0; e < 8; ++e) lo[8 * u + e] = f[e];
      unpack8(*reinterpret_cast<const u32x4*>(src + HALF + 16 * c + 8 * u), f);
#pragma unroll
      for (int e = 0; e < 8; ++e) hi[8 * u + e] = f[e];
    }
    if (part < 2) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float x0 = lo[i], x1 = hi[i];
        lo[i] = x0 * cv[i] - x1 * sv[i];
        hi[i] = x1 * cv[i] + x0 * sv[i];
      }
    }
    if (part == 1 && !a.k_rows) {
      // k: through LDS so kT rows (one dimension, 64 tokens) store whole.
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        kt[16 * c + i][tok] = (uint16_t)f32_to_bf16(lo[i]);
        kt[HALF + 16 * c + i][tok] = (uint16_t)f32_to_bf16(hi[i]);
      }
    } else {
      uint16_t* dst = (part == 0 ? a.q : part == 1 ? a.kT : a.v) + out_row;
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        float f[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) f[e] = lo[8 * u + e];
        *reinterpret_cast<u32x4*>(dst + 16 * c + 8 * u) = pack8(f);
#pragma unroll
        for (int e = 0; e < 8; ++e) f[e] = hi[8 * u + e];
        *reinterpret_cast<u32x4*>(dst + HALF + 16 * c + 8 * u) = pack8(f);
      }
    }
  }
  if (a.k_rows) return;  // uniform across the workgroup
  __syncthreads();
  // kT [bh][d][s0 .. s0 + 63]: 128 rows of 128 B; thread t writes row t/2,
  // half t%2 (32 tokens = 4 x 16 B).
  {
    const int d = tid >> 1, half = tid & 1;
    uint16_t* dst = a.kT + ((int64_t)bh * D + d) * a.S + s0 + 32 * half;
#pragma unroll
    for (int u = 0; u < 4; ++u)
      *reinterpret_cast<u32x4*>(dst + 8 * u) = *reinterpret_cast<const u32x4*>(&kt[d][32 * half + 8 * u]);
  }
}

struct CausalArgs {
  const uint16_t* s;
  uint16_t* p;
  int64_t rows;
  int S;
  float scale;
};

__device__ __forceinline__ float c_wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ float c_wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// One workgroup (256 threads) per row; VPT vectors of 8 columns per thread.
// Vectors entirely above the diagonal are neither read nor exponentiated,
// only zero-filled.
template <int VPT>
__global__ __launch_bounds__(256) void softmax_causal_kernel(CausalArgs a) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const int i = (int)(row % a.S);  // position in the sequence: columns 0..i kept
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const uint16_t* src = a.s + row * a.S;
  uint16_t* dst = a.p + row * a.S;
  float v[VPT][8];
  float m = -INFINITY;
#pragma unroll
  for (int q = 0; q < VPT; ++q) {
    const int c0 = (q * 256 + tid) * 8;
    if (c0 < a.S && c0 <= i) {
      unpack8(*reinterpret_cast<const u32x4*>(src + c0), v[q]);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        v[q][e] = c0 + e <= i ? v[q][e] * a.scale : -INFINITY;
        m = fmaxf(m, v[q][e]);
      }
    }
  }
  m = c_wave_max(m);
  if (lane == 0) red[wv] = m;
  __syncthreads();
  m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  float sum = 0.f;
#pragma unroll
  for (int q = 0; q < VPT; ++q) {
    const int c0 = (q * 256 + tid) * 8;
    if (c0 < a.S && c0 <= i) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float ex = c0 + e <= i ? __expf(v[q][e] - m) : 0.f;
        v[q][e] = ex;
        sum += ex;
      }
    }
  }
  sum = c_wave_sum(sum);
  if (lane == 0) red[wv] = sum;
  __syncthreads();
  sum = red[0] + red[1] + red[2] + red[3];
  const float r = 1.0f / sum;
#pragma unroll
  for (int q = 0; q < VPT; ++q) {
    const int c0 = (q * 256 + tid) * 8;
    if (c0 >= a.S) continue;
    if (c0 <= i) {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[q][e] *= r;
      *reinterpret_cast<u32x4*>(dst + c0) = pack8(v[q]);
    } else {
      *reinterpret_cast<u32x4*>(dst + c0) = u32x4{0u, 0u, 0u, 0u};
    }
  }
}

// ---------------------------------------------------------------------------
// Causal attention in one pass (flash-attention style): per (b, h) and
// 8 x 16 RB query rows, loop over 64-key tiles up to the diagonal; scores, the
// online softmax and P @ V stay on chip, and the output goes straight to the
// merged [B*S, H*D] layout.  8 waves, each 16 RB query rows (RB row blocks of
// 16); v_mfma_f32_16x16x32_bf16 throughout.  Every K and V fragment read
// from LDS feeds RB MFMAs, so RB = 2 (S % 256 == 0) halves the LDS reads per
// MFMA of RB = 1.
//   S = Q K^T: first operand K rows (lane: key 16t + l%16, 8 consecutive d
//     from an XOR-swizzled LDS tile), second Q rows (registers, loaded from
//     global memory once) -> lane holds row i = l%16 of its block and keys
//     4(l/16) .. +3 of each 16-key block.
//   P @ V: second operand P straight from those registers (bf16); its 8
//     k-slots per lane are keys {4g .. 4g+3} and {16 + 4g .. 16 + 4g + 3} of
//     a 32-key block (g = l/16), and the V fragment is read with
//     ds_read_b64_tr_b16 from exactly those rows, so no shuffle is needed.
// Scores are scaled into log2 units; exp2 is the hardware v_exp_f32.
// ---------------------------------------------------------------------------
constexpr int kFaKV = 64;  // keys per tile

struct AttnArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* out;
  int B, H, S;
  float scale_log2;  // softmax scale times log2(e)
};

// V tile row swizzle (16-byte chunk position = chunk ^ fa_vswz(row)): the 64
// lanes of one transposing read touch every bank exactly twice.
__device__ __forceinline__ int fa_vswz(int r) { return (2 * (r & 3)) | (8 * ((r >> 2) & 1)); }

__device__ __forceinline__ float fa_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// K / V tiles reach LDS by DMA (global_load_lds): a ring of kFaRing stages
// (one K tile and one V tile, 32 KB) issued kFaRing - 1 tiles ahead, so each
// tile's load latency hides behind the previous tiles' MFMAs; 128 KB in all.
// The XOR swizzles are applied by choosing each DMA lane's source chunk.
constexpr int kFaRing = 4;
constexpr int kFaStage = 2 * kFaKV * kHeadDim * 2;  // 32 KB
constexpr int kFaLds = kFaRing * kFaStage;          // 128 KB

template <int RB>
__global__ __launch_bounds__(512) void attention_causal_kernel(AttnArgs a) {
  constexpr int D = kHeadDim, ROWB = D * 2;  // 256-byte rows
  constexpr int R = kFaRing, QW = 16 * RB, QT = 8 * QW;  // rows per wave / per workgroup
  extern __shared__ __attribute__((aligned(16))) unsigned char fa_smem[];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g = lane >> 4, l16 = lane & 15;
  const int BH = a.B * a.H;
  const int bh = (int)(blockIdx.x % BH);
  const int qt = a.S / QT - 1 - (int)(blockIdx.x / BH);  // longest rows first
  const int q0 = qt * QT, i0 = q0 + QW * w;
  const uint16_t* Qg = a.q + (int64_t)bh * a.S * D;
  const uint16_t* Kg = a.k + (int64_t)bh * a.S * D;
  const uint16_t* Vg = a.v + (int64_t)bh * a.S * D;
  const uint32_t sbase = lds_addr(fa_smem);

  // This wave's Q fragments: block rb, d chunk 4s + g of row i0 + 16 rb + l16.
  u32x4 qf[RB][4];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int s = 0; s < 4; ++s)
      qf[rb][s] = *reinterpret_cast<const u32x4*>(Qg + (int64_t)(i0 + 16 * rb + l16) * D + 8 * (4 * s + g));

  // DMA instruction I = 2w + u (u = 0, 1) of a tile covers rows 4I .. 4I+3
  // of K and of V: lane L fills row 4I + L/16, chunk position L%16, from
  // the source chunk the swizzle puts there (K: c ^ (row % 16), V:
  // c ^ fa_vswz(row)).
  const uint16_t* ksrc[2];
  const uint16_t* vsrc[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int row = 4 * (2 * w + u) + (lane >> 4), p = lane & 15;
    ksrc[u] = Kg + (int64_t)row * D + 8 * (p ^ (row & 15));
    vsrc[u] = Vg + (int64_t)row * D + 8 * (p ^ fa_vswz(row));
  }
  auto issue = [&](int t, int slot) {
    const uint32_t st = sbase + (uint32_t)(slot * kFaStage);
#pragma unroll
    for (int u = 0; u < 2; ++u) dma16_asm(ksrc[u] + (int64_t)t * kFaKV * D, st + (uint32_t)((2 * w + u) * 1024));
#pragma unroll
    for (int u = 0; u < 2; ++u)
      dma16_asm(vsrc[u] + (int64_t)t * kFaKV * D, st + (uint32_t)(kFaKV * ROWB + (2 * w + u) * 1024));
  };
  const int ntiles = (q0 + QT) / kFaKV;  // >= 2
  const int pre = ntiles < R - 1 ? ntiles : R - 1;
  for (int t = 0; t < pre; ++t) issue(t, t);

  f32x4 o[RB][8];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int n = 0; n < 8; ++n) o[rb][n] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m[RB], lsum[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    m[rb] = -INFINITY;
    lsum[rb] = 0.f;
  }

  // V fragment byte offsets (tile-relative): d tile n, 32-key block u, low /
  // high 4 keys.  Lane (g, r = (l%16)/4, q = l%4) reads row 32u + 4g + r
  // (+16), columns 16n + 4q .. +3.
  const int vr_r = (lane & 15) >> 2, vr_q = lane & 3;

  for (int t = 0; t < ntiles; ++t) {
    const int slot = t % R;
    // Own DMAs of tile t landed; the tiles issued after it may still be in
    // flight (R - 2 of them while the ring is full, fewer at the end, where
    // the wait is for all).  After the barrier every wave's have landed and
    // every wave is done with tile t-1's slot.
    if (t + R - 1 <= ntiles) vm_wait(4 * (R - 2));
    else vm_wait(0);
    asm volatile("s_barrier" ::: "memory");
    if (t + R - 1 < ntiles) issue(t + R - 1, (t + R - 1) % R);
    const int kv0 = t * kFaKV;
    // Some key of the tile is visible to this wave's rows.  kv0 - i0 is a
    // multiple of 16 RB, so then kv0 <= i0: every row of every block sees
    // at least key kv0, and no row max below is -inf.
    if (kv0 <= i0 + QW - 1) {
      const unsigned char* Ks = fa_smem + slot * kFaStage;
      const unsigned char* Vs = Ks + kFaKV * ROWB;
      f32x4 sacc[RB][4];
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) sacc[rb][tt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) {
          const int j = 16 * tt + l16;
          const u32x4 kf = *reinterpret_cast<const u32x4*>(Ks + j * ROWB + 16 * ((4 * s + g) ^ (j & 15)));
#pragma unroll
          for (int rb = 0; rb < RB; ++rb) sacc[rb][tt] = mfma16x16x32(kf, qf[rb][s], sacc[rb][tt]);
        }
      // Only a tile that crosses the diagonal of this wave's rows is masked
      // (a wave-uniform branch).
      if (kv0 + kFaKV - 1 > i0) {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
          const int i = i0 + 16 * rb + l16;
#pragma unroll
          for (int tt = 0; tt < 4; ++tt)
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (kv0 + 16 * tt + 4 * g + e > i) sacc[rb][tt][e] = -INFINITY;
        }
      }
      u32x4 pf[RB][2];
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        // The scale (log2 units) is positive, so the row max of the scaled
        // scores is the scaled max of the raw ones (rounding is monotonic),
        // and each probability takes one fma before its exp2.
        float mt = -INFINITY;
#pragma unroll
        for (int tt = 0; tt < 4; ++tt)
#pragma unroll
          for (int e = 0; e < 4; ++e) mt = fmaxf(mt, sacc[rb][tt][e]);
        mt = fmaxf(mt, __shfl_xor(mt, 16, 64));
        mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
        const float mn = fmaxf(m[rb], mt * a.scale_log2);
        const float alpha = fa_exp2(m[rb] - mn);
        // alpha is exactly 1 for a row whose max held; when that is every
        // row of the block the rescale is skipped.
        const bool rescale = !__all(mn == m[rb]);
        m[rb] = mn;
        float ps = 0.f;
#pragma unroll
        for (int tt = 0; tt < 4; ++tt)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float p = fa_exp2(__builtin_fmaf(sacc[rb][tt][e], a.scale_log2, -mn));
            sacc[rb][tt][e] = p;
            ps += p;
          }
        lsum[rb] = lsum[rb] * alpha + ps;
        if (rescale) {
#pragma unroll
          for (int n = 0; n < 8; ++n) o[rb][n] *= alpha;
        }
#pragma unroll
        for (int u = 0; u < 2; ++u)
          pf[rb][u] = u32x4{pack_bf16x2(sacc[rb][2 * u][0], sacc[rb][2 * u][1]),
                            pack_bf16x2(sacc[rb][2 * u][2], sacc[rb][2 * u][3]),
                            pack_bf16x2(sacc[rb][2 * u + 1][0], sacc[rb][2 * u + 1][1]),
                            pack_bf16x2(sacc[rb][2 * u + 1][2], sacc[rb][2 * u + 1][3])};
      }
#pragma unroll
      for (int n = 0; n < 8; ++n)
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int c = 2 * n + (vr_q >> 1), hb = 8 * (vr_q & 1);
          const int r0 = 32 * u + 4 * g + vr_r, r1 = r0 + 16;
          const s16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (lds_s16x4_t)(Vs + r0 * ROWB + 16 * (c ^ fa_vswz(r0)) + hb));
          const s16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (lds_s16x4_t)(Vs + r1 * ROWB + 16 * (c ^ fa_vswz(r1)) + hb));
          const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
          const u32x4 vf = u32x4{l2.x, l2.y, h2.x, h2.y};
#pragma unroll
          for (int rb = 0; rb < RB; ++rb) o[rb][n] = mfma16x16x32(vf, pf[rb][u], o[rb][n]);
        }
    }
    // This wave's reads of the slot are complete before the next barrier
    // lets another wave's DMA refill it.
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  }

  const int b = bh / a.H, h = bh - b * a.H;
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    float l = lsum[rb];
    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
    const float inv = 1.0f / l;
    uint16_t* out = a.out + ((int64_t)b * a.S + i0 + 16 * rb + l16) * (a.H * D) + h * D + 4 * g;
#pragma unroll
    for (int n = 0; n < 8; ++n)
      *reinterpret_cast<u32x2*>(out + 16 * n) = u32x2{pack_bf16x2(o[rb][n].x * inv, o[rb][n].y * inv),
                                                      pack_bf16x2(o[rb][n].z * inv, o[rb][n].w * inv)};
  }
}

struct MergeArgs {
  const uint16_t* o;
  uint16_t* out;
  int B, H, S;
};

// out[b*S + s][h*D + d] = o[(b*H + h)*S + s][d]; one 16-byte chunk per thread.
__global__ __launch_bounds__(256) void merge_heads_kernel(MergeArgs a) {
  constexpr int D = kHeadDim, CH = D / 8;
  const int64_t total = (int64_t)a.B * a.H * a.S * CH;
  for (int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x; t < total; t += (int64_t)gridDim.x * 256) {
    const int ch = (int)(t % CH);
    const int64_t r = t / CH;  // (b*H + h)*S + s
    const int s = (int)(r % a.S);
    const int64_t bh = r / a.S;
    const int h = (int)(bh % a.H), b = (int)(bh / a.H);
    const u32x4 w = *reinterpret_cast<const u32x4*>(a.o + r * D + 8 * ch);
    *reinterpret_cast<u32x4*>(a.out + ((int64_t)b * a.S + s) * a.H * D + h * D + 8 * ch) = w;
  }
}

}  // namespace mk

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
#include "../capi_internal.h"

#include <algorithm>
#include <cmath>
#include <cstdlib>

extern "C" int mk_rope_qkv_split_bf16(const void* qkv, const float* cos_table, const float* sin_table, void* q,
                                      void* k, void* v, int64_t B, int64_t S, int64_t H, int64_t D, int k_rows,
                                      void* stream) {
  mkc::clear_error();
  const char* fn = "mk_rope_qkv_split_bf16";
  if (!qkv || !cos_table || !sin_table || !q || !k || !v) return mkc::fail(MK_EINVAL, "%s: null pointer", fn);
  if (B <= 0 || S <= 0 || H <= 0 || D <= 0) return mkc::fail(MK_EINVAL, "%s: sizes must be positive", fn);
  if (D != mk::kHeadDim) return mkc::fail(MK_EUNSUPPORTED, "%s: head dim %lld (only 128)", fn, (long long)D);
  if (S % mk::kRopeTok != 0)
    return mkc::fail(MK_EUNSUPPORTED, "%s: sequence length %lld not a multiple of 64", fn, (long long)S);
  if (B * H * (S / mk::kRopeTok) > (1 << 30) || B * S * 3 * H * D > ((int64_t)1 << 40))
    return mkc::fail(MK_EINVAL, "%s: shape too large", fn);
  mk::RopeArgs a;
  a.qkv = static_cast<const uint16_t*>(qkv);
  a.cosb = cos_table;
  a.sinb = sin_table;
  a.q = static_cast<uint16_t*>(q);
  a.kT = static_cast<uint16_t*>(k);
  a.k_rows = k_rows ? 1 : 0;
  a.v = static_cast<uint16_t*>(v);
  a.B = (int)B;
  a.S = (int)S;
  a.H = (int)H;
  hipLaunchKernelGGL(mk::rope_qkv_split_kernel, dim3((unsigned)(B * H * (S / mk::kRopeTok))), dim3(256), 0,
                     static_cast<hipStream_t>(stream), a);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return mkc::fail(MK_ELAUNCH, "%s: launch failed: %s", fn, hipGetErrorString(e));
  return MK_OK;
}

extern "C" int mk_softmax_causal_bf16(const void* scores, void* probs, int64_t batches, int64_t S, float scale,
                                      void* stream) {
  mkc::clear_error();
  const char* fn = "mk_softmax_causal_bf16";
  if (!scores || !probs) return mkc::fail(MK_EINVAL, "%s: null pointer", fn);
  if (batches <= 0 || S <= 0) return mkc::fail(MK_EINVAL, "%s: sizes must be positive", fn);
  if (S % 8 != 0 || S > 8192)
    return mkc::fail(MK_EUNSUPPORTED, "%s: sequence length %lld (need S %% 8 == 0, S <= 8192)", fn,
                     (long long)S);
  if (batches * S > (int64_t)1 << 31) return mkc::fail(MK_EINVAL, "%s: shape too large", fn);
  mk::CausalArgs a;
  a.s = static_cast<const uint16_t*>(scores);
  a.p = static_cast<uint16_t*>(probs);
  a.rows = batches * S;
  a.S = (int)S;
  a.scale = scale;
  const dim3 grid((unsigned)(batches * S));
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int vpt = (int)((S + 2047) / 2048);
  switch (vpt) {
    case 1: hipLaunchKernelGGL(mk::softmax_causal_kernel<1>, grid, dim3(256), 0, st, a); break;
    case 2: hipLaunchKernelGGL(mk::softmax_causal_kernel<2>, grid, dim3(256), 0, st, a); break;
    default: hipLaunchKernelGGL(mk::softmax_causal_kernel<4>, grid, dim3(256), 0, st, a); break;
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return mkc::fail(MK_ELAUNCH, "%s: launch failed: %s", fn, hipGetErrorString(e));
  return MK_OK;
}

extern "C" int mk_merge_heads_bf16(const void* o, void* out, int64_t B, int64_t H, int64_t S, int64_t D,
                                   void* stream) {
  mkc::clear_error();
  const char* fn = "mk_merge_heads_bf16";
  if (!o || !out) return mkc::fail(MK_EINVAL, "%s: null pointer", fn);
  if (B <= 0 || S <= 0 || H <= 0 || D <= 0) return mkc::fail(MK_EINVAL, "%s: sizes must be positive", fn);
  if (D != mk::kHeadDim) return mkc::fail(MK_EUNSUPPORTED, "%s: head dim %lld (only 128)", fn, (long long)D);
  if (B * H * S > (int64_t)1 << 31) return mkc::fail(MK_EINVAL, "%s: shape too large", fn);
  mk::MergeArgs a;
  a.o = static_cast<const uint16_t*>(o);
  a.out = static_cast<uint16_t*>(out);
  a.B = (int)B;
  a.H = (int)H;
  a.S = (int)S;
  const int64_t chunks = B * H * S * (D / 8);
  const int blocks = (int)std::min<int64_t>((chunks + 255) / 256, 16384);
  hipLaunchKernelGGL(mk::merge_heads_kernel, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream), a);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return mkc::fail(MK_ELAUNCH, "%s: launch failed: %s", fn, hipGetErrorString(e));
  return MK_OK;
}

extern "C" int mk_attention_causal_bf16(const void* q, const void* k, const void* v, void* out, int64_t B,
                                        int64_t H, int64_t S, int64_t D, float scale, void* stream) {
  mkc::clear_error();
  const char* fn = "mk_attention_causal_bf16";
  if (!q || !k || !v || !out) return mkc::fail(MK_EINVAL, "%s: null pointer", fn);
  if (B <= 0 || S <= 0 || H <= 0 || D <= 0) return mkc::fail(MK_EINVAL, "%s: sizes must be positive", fn);
  if (D != mk::kHeadDim) return mkc::fail(MK_EUNSUPPORTED, "%s: head dim %lld (only 128)", fn, (long long)D);
  if (S % 128 != 0)
    return mkc::fail(MK_EUNSUPPORTED, "%s: sequence length %lld not a multiple of 128", fn, (long long)S);
  if (B * H * (S / 128) > (1 << 30) || B * H * S * D > ((int64_t)1 << 40))
    return mkc::fail(MK_EINVAL, "%s: shape too large", fn);
  mk::AttnArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.k = static_cast<const uint16_t*>(k);
  a.v = static_cast<const uint16_t*>(v);
  a.out = static_cast<uint16_t*>(out);
  a.B = (int)B;
  a.H = (int)H;
  a.S = (int)S;
  if (!(scale > 0.f) || !std::isfinite(scale))
    return mkc::fail(MK_EINVAL, "%s: scale must be positive and finite (got %g)", fn, (double)scale);
  a.scale_log2 = scale * 1.4426950408889634f;
  // 32 query rows per wave when S allows (256 per workgroup), else 16.
  // MK_ATTN_RB=1 keeps 16; the results are the same bits either way.
  const char* rbv = getenv("MK_ATTN_RB");
  const bool rb2 = S % 256 == 0 && !(rbv && atoi(rbv) == 1);
  const void* kfn = rb2 ? (const void*)mk::attention_causal_kernel<2> : (const void*)mk::attention_causal_kernel<1>;
  hipError_t e = hipFuncSetAttribute(kfn, hipFuncAttributeMaxDynamicSharedMemorySize, mk::kFaLds);
  if (e != hipSuccess) return mkc::fail(MK_ELAUNCH, "%s: LDS opt-in failed: %s", fn, hipGetErrorString(e));
  const dim3 grid((unsigned)(B * H * (S / (rb2 ? 256 : 128))));
  if (rb2)
    hipLaunchKernelGGL(mk::attention_causal_kernel<2>, grid, dim3(512), mk::kFaLds, static_cast<hipStream_t>(stream), a);
  else
    hipLaunchKernelGGL(mk::attention_causal_kernel<1>, grid, dim3(512), mk::kFaLds, static_cast<hipStream_t>(stream), a);
  e = hipGetLastError();
  if (e != hipSuccess) return mkc::fail(MK_ELAUNCH, "%s: launch failed: %s", fn, hipGetErrorString(e));
  return MK_OK;
}
