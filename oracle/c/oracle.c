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
 *   f32 GEMM:  C = A @ B in f32, k ascending (the reference's f32 dot,
 *              ops/binary_ops.mm:775-782, at f32 throughout).
 *   argmax:    first NaN, else first maximum, -0 == +0
 *              (reference ops/reduction_ops.mm:1478-1536).
 *   softmax:   exp(x - max) / sum over the last axis; a NaN or infinite row
 *              maximum gives a NaN row (reference
 *              core/mps_executable.mm:1922-2089, tests/test_native_softmax.py:26-35);
 *              bf16 with XLA:CPU's rounding points d = r(x - m), e = r(exp d),
 *              s = r(sum_f32 e), y = r(e / s) (as oracle/rowops.py restates
 *              runtime/metal_kernels.mm:1742-1819).
 *   rmsnorm:   x * 1/sqrt(mean(x^2) + eps) * g in f32 (bf16: one rounding
 *              of the output), the workload's definition.
 *   chain6:    a = x*1.5, b = a+0.5, c = exp b, d = log1p c, e = max(d, x),
 *              y = x > 0 ? e : b, each float result rounded to the program's
 *              type (bf16 per op as XLA:CPU does, ops/registry.h:273-287).
 *   plumbing:  y[i] = sum_j tanh(sum_k a[i,k] b[k,j]) in f32 (the workload's
 *              jax.jit(tanh(A @ B).sum(axis=1)) case).
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

/* C[M,N] (f32) = A[M,K] (f32) @ B[K,N] (f32), rows m in [m0, m1). */
void orc_gemm_f32(const float* a, const float* b, int64_t M, int64_t K, int64_t N,
                  int64_t m0, int64_t m1, float* c) {
    (void)M;
    #pragma omp parallel for schedule(dynamic, 1)
    for (int64_t m = m0; m < m1; ++m) {
        float* cr = c + m * N;
        for (int64_t n = 0; n < N; ++n) cr[n] = 0.f;
        for (int64_t k = 0; k < K; ++k) {
            const float av = a[m * K + k];
            const float* br = b + k * N;
            for (int64_t n = 0; n < N; ++n) cr[n] += av * br[n];
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

static inline uint16_t f32_to_bf16_bits(float f) {
    float r = round_to_bf16(f);
    uint32_t u;
    memcpy(&u, &r, 4);
    return (uint16_t)(u >> 16);
}

/* First NaN, else first max (-0 == +0), per row of a row-major bf16 matrix. */
void orc_argmax_bf16(const uint16_t* x, int64_t rows, int64_t cols, int32_t* out) {
    #pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        const uint16_t* p = x + r * cols;
        int64_t best = 0;
        float bv = bf16_to_f32(p[0]);
        if (bv != bv) { out[r] = 0; continue; }
        for (int64_t i = 1; i < cols; ++i) {
            float v = bf16_to_f32(p[i]);
            if (v != v) { best = i; break; }
            if (v > bv) { bv = v; best = i; }
        }
        out[r] = (int32_t)best;
    }
}

static inline float row_max_f32(const float* p, int64_t cols) {
    float m = -INFINITY;
    for (int64_t i = 0; i < cols; ++i) {
        float v = p[i];
        if (v != v) return v;
        if (v > m) m = v;
    }
    return m;
}

/* Softmax of rows [r0, r1) of a row-major f32 matrix (f32 arithmetic). */
void orc_softmax_f32(const float* x, int64_t cols, int64_t r0, int64_t r1, float* y) {
    #pragma omp parallel for schedule(static)
    for (int64_t r = r0; r < r1; ++r) {
        const float* p = x + r * cols;
        float* o = y + r * cols;
        float m = row_max_f32(p, cols);
        float sum = 0.f;
        for (int64_t i = 0; i < cols; ++i) {
            float e = expf(p[i] - m);
            o[i] = e;
            sum += e;
        }
        float inv = 1.f / sum;
        for (int64_t i = 0; i < cols; ++i) o[i] = o[i] * inv;
        if (m != m || isinf(m))
            for (int64_t i = 0; i < cols; ++i) o[i] = NAN;
    }
}

/* bf16 softmax with XLA:CPU's rounding points, rows [r0, r1) -> bf16 bits. */
void orc_softmax_bf16(const uint16_t* x, int64_t cols, int64_t r0, int64_t r1, uint16_t* y) {
    #pragma omp parallel for schedule(static)
    for (int64_t r = r0; r < r1; ++r) {
        const uint16_t* p = x + r * cols;
        uint16_t* o = y + r * cols;
        float m = -INFINITY;
        int nan = 0;
        for (int64_t i = 0; i < cols; ++i) {
            float v = bf16_to_f32(p[i]);
            if (v != v) nan = 1;
            if (v > m) m = v;
        }
        if (nan || isinf(m)) {
            for (int64_t i = 0; i < cols; ++i) o[i] = 0x7fc0u;
            continue;
        }
        float sum = 0.f;
        for (int64_t i = 0; i < cols; ++i) {
            float d = round_to_bf16(bf16_to_f32(p[i]) - m);
            sum += round_to_bf16(expf(d));
        }
        float s = round_to_bf16(sum);
        for (int64_t i = 0; i < cols; ++i) {
            float e = round_to_bf16(expf(round_to_bf16(bf16_to_f32(p[i]) - m)));
            o[i] = f32_to_bf16_bits(e / s);
        }
    }
}

/* RMSNorm of rows [r0, r1): y = x * 1/sqrt(mean(x^2) + eps) * g (f32). */
void orc_rmsnorm_f32(const float* x, const float* g, int64_t cols, float eps, int64_t r0, int64_t r1,
                     float* y) {
    #pragma omp parallel for schedule(static)
    for (int64_t r = r0; r < r1; ++r) {
        const float* p = x + r * cols;
        float* o = y + r * cols;
        double ss = 0.0;
        for (int64_t i = 0; i < cols; ++i) ss += (double)p[i] * p[i];
        float inv = 1.f / sqrtf((float)(ss / (double)cols) + eps);
        for (int64_t i = 0; i < cols; ++i) o[i] = p[i] * inv * g[i];
    }
}

/* bf16 RMSNorm of rows [r0, r1): f32 arithmetic, the output rounded once. */
void orc_rmsnorm_bf16(const uint16_t* x, const uint16_t* g, int64_t cols, float eps, int64_t r0, int64_t r1,
                      uint16_t* y) {
    #pragma omp parallel for schedule(static)
    for (int64_t r = r0; r < r1; ++r) {
        const uint16_t* p = x + r * cols;
        uint16_t* o = y + r * cols;
        double ss = 0.0;
        for (int64_t i = 0; i < cols; ++i) {
            double v = bf16_to_f32(p[i]);
            ss += v * v;
        }
        float inv = 1.f / sqrtf((float)(ss / (double)cols) + eps);
        for (int64_t i = 0; i < cols; ++i) o[i] = f32_to_bf16_bits(bf16_to_f32(p[i]) * inv * bf16_to_f32(g[i]));
    }
}

/* stablehlo.maximum: NaN propagates, -0 < +0. */
static inline float shlo_max(float a, float b) {
    if (a != a) return a;
    if (b != b) return b;
    if (a == 0.f && b == 0.f) return signbit(a) ? b : a;
    return a > b ? a : b;
}

/* The 6-op chain over n elements (f32 results rounded to f32). */
void orc_chain6_f32(const float* x, int64_t n, float* y) {
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        float v = x[i];
        float a = v * 1.5f, b = a + 0.5f, c = expf(b), d = log1pf(c), e = shlo_max(d, v);
        y[i] = v > 0.f ? e : b;
    }
}

/* The 6-op chain on bf16 (every float result rounded to bf16) -> bf16 bits. */
void orc_chain6_bf16(const uint16_t* x, int64_t n, uint16_t* y) {
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        float v = bf16_to_f32(x[i]);
        float a = round_to_bf16(v * 1.5f);
        float b = round_to_bf16(a + 0.5f);
        float c = round_to_bf16(expf(b));
        float d = round_to_bf16(log1pf(c));
        float e = shlo_max(d, v);
        y[i] = f32_to_bf16_bits(v > 0.f ? e : b);
    }
}

/* y[i] = sum_j tanh(sum_k a[i,k] b[k,j]) for rows [r0, r1) of f32 a [n, n], b [n, n]. */
void orc_plumbing_f32(const float* a, const float* b, int64_t n, int64_t r0, int64_t r1, float* y) {
    #pragma omp parallel for schedule(dynamic, 1)
    for (int64_t i = r0; i < r1; ++i) {
        float* row = (float*)malloc((size_t)n * sizeof(float));
        for (int64_t j = 0; j < n; ++j) row[j] = 0.f;
        for (int64_t k = 0; k < n; ++k) {
            float av = a[i * n + k];
            const float* br = b + k * n;
            for (int64_t j = 0; j < n; ++j) row[j] += av * br[j];
        }
        float s = 0.f;
        for (int64_t j = 0; j < n; ++j) s += tanhf(row[j]);
        y[i] = s;
        free(row);
    }
}
