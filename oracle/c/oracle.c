/*
 * C restatement of the hot-path arithmetic -- TEST INFRASTRUCTURE ONLY.
 *
 * Used by tests/ as a second checker and by bench.py's cpu_baseline leg as the
 * timed CPU port ("kind": "port").  The plugin never links or calls this file.
 * It follows the same definitions as oracle/quant.py and oracle/gemm.py:
 *
 *   int4 g64:  Y = X @ ((W - z) * s), W packed two nibbles per byte along K
 *              (low nibble = even k, reference quantized.py:189-190), the
 *              dequantized weight rounded to bf16 as XLA:CPU rounds the bf16
 *              multiply (reference ops/registry.h:273-287), f32 accumulation.
 *   int8 pc:   Y = s[n] * sum_k X[m,k] W[k,n]  (f32 accumulation).
 *   bf16 GEMM: C = A @ B with f32 accumulation (reference
 *              ops/binary_ops.mm:775-782: bf16 x bf16 -> f32 preferred type).
 *   argmax:    first NaN, else first maximum, -0 == +0
 *              (reference ops/reduction_ops.mm:1478-1536).
 *
 * Built by oracle/build_oracle.sh into oracle/lib/liboracle_c.so.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#include <stdlib.h>
#include <omp.h>

static inline float bf16_to_f32(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static inline float round_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) {
        u |= 0x00400000u;
    } else {
        u += 0x7fffu + ((u >> 16) & 1u);
    }
    u &= 0xffff0000u;
    memcpy(&f, &u, 4);
    return f;
}

int orc_threads(int n) {
    if (n > 0) omp_set_num_threads(n);
    return omp_get_max_threads();
}

/* Y[M,N] (f32) = X[M,K] (bf16) @ ((W - z) * s), columns n in [n0, n1). */
void orc_int4_g64_matmul(const uint16_t* x, const uint8_t* w, const uint16_t* s,
                         const uint8_t* z, int64_t M, int64_t K, int64_t N,
                         int64_t n0, int64_t n1, float* y) {
    const int64_t NT = 64;
    #pragma omp parallel for schedule(dynamic, 1)
    for (int64_t nb = n0; nb < n1; nb += NT) {
        int64_t ne = nb + NT < n1 ? nb + NT : n1;
        int64_t nw = ne - nb;
        float acc[64 * 64];
        float wrow[64];
        for (int64_t i = 0; i < M * NT && i < 64 * 64; ++i) acc[i] = 0.f;
        for (int64_t m0 = 0; m0 < M; m0 += 64) {
            int64_t mw = M - m0 < 64 ? M - m0 : 64;
            memset(acc, 0, sizeof(acc));
            for (int64_t k = 0; k < K; ++k) {
                const uint8_t* wr = w + (k >> 1) * N;
                const int64_t g = k >> 6;
                const int shift = (int)(k & 1) * 4;
                for (int64_t j = 0; j < nw; ++j) {
                    int64_t n = nb + j;
                    int q = (wr[n] >> shift) & 0xF;
                    float d = (float)(q - (int)z[g * N + n]) * bf16_to_f32(s[g * N + n]);
                    wrow[j] = round_to_bf16(d);
                }
                for (int64_t mi = 0; mi < mw; ++mi) {
                    float xv = bf16_to_f32(x[(m0 + mi) * K + k]);
                    float* a = acc + mi * 64;
                    for (int64_t j = 0; j < nw; ++j) a[j] += xv * wrow[j];
                }
            }
            for (int64_t mi = 0; mi < mw; ++mi)
                for (int64_t j = 0; j < nw; ++j) y[(m0 + mi) * N + nb + j] = acc[mi * 64 + j];
        }
    }
}

/* Y[M,N] (f32) = s[n] * sum_k X[m,k] W[k,n], columns n in [n0, n1). */
void orc_int8_pc_matmul(const uint16_t* x, const int8_t* w, const float* s,
                        int64_t M, int64_t K, int64_t N, int64_t n0, int64_t n1, float* y) {
    const int64_t NT = 64;
    #pragma omp parallel for schedule(dynamic, 1)
    for (int64_t nb = n0; nb < n1; nb += NT) {
        int64_t ne = nb + NT < n1 ? nb + NT : n1;
        int64_t nw = ne - nb;
        float acc[64 * 64];
        for (int64_t m0 = 0; m0 < M; m0 += 64) {
            int64_t mw = M - m0 < 64 ? M - m0 : 64;
            memset(acc, 0, sizeof(acc));
            for (int64_t k = 0; k < K; ++k) {
                const int8_t* wr = w + k * N + nb;
                for (int64_t mi = 0; mi < mw; ++mi) {
                    float xv = bf16_to_f32(x[(m0 + mi) * K + k]);
                    float* a = acc + mi * 64;
                    for (int64_t j = 0; j < nw; ++j) a[j] += xv * (float)wr[j];
                }
            }
            for (int64_t mi = 0; mi < mw; ++mi)
                for (int64_t j = 0; j < nw; ++j)
                    y[(m0 + mi) * N + nb + j] = acc[mi * 64 + j] * s[nb + j];
        }
    }
}

/* C[M,N] (f32) = A[M,K] (bf16) @ B[K,N] (bf16), rows m in [m0, m1). */
void orc_gemm_bf16(const uint16_t* a, const uint16_t* b, int64_t M, int64_t K, int64_t N,
                   int64_t m0, int64_t m1, float* c) {
    (void)M;
    #pragma omp parallel for schedule(dynamic, 1)
    for (int64_t m = m0; m < m1; ++m) {
        float* cr = c + m * N;
        for (int64_t n = 0; n < N; ++n) cr[n] = 0.f;
        for (int64_t k = 0; k < K; ++k) {
            float av = bf16_to_f32(a[m * K + k]);
            const uint16_t* br = b + k * N;
            for (int64_t n = 0; n < N; ++n) cr[n] += av * bf16_to_f32(br[n]);
        }
    }
}

/* First NaN, else first max (-0 == +0), per row of a row-major f32 matrix. */
void orc_argmax_f32(const float* x, int64_t rows, int64_t cols, int32_t* out) {
    #pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        const float* p = x + r * cols;
        int64_t best = 0;
        float bv = p[0];
        if (bv != bv) { out[r] = 0; continue; }
        int found_nan = 0;
        for (int64_t i = 1; i < cols; ++i) {
            float v = p[i];
            if (v != v) { best = i; found_nan = 1; break; }
            if (v > bv) { bv = v; best = i; }
        }
        (void)found_nan;
        out[r] = (int32_t)best;
    }
}
