/*
 * mk_kernels.h -- C-ABI of the MI355X (gfx950) hot-path kernels.
 *
 * This is the internal operator boundary of the plugin: the executor calls
 * these entry points where the reference calls a NativeOpHandler
 * (src/pjrt_plugin/ops/registry.h:87-88, a function taking the device, the
 * command buffer, the op and its input buffers) or encodes an MPSGraph
 * segment (src/pjrt_plugin/core/mps_executable.mm:7328-7388).
 *
 * Conventions (all entry points):
 *   - pointers are device pointers (hipMalloc'd), row-major, densely packed;
 *   - bf16 tensors are 16-bit bit patterns (uint16_t storage);
 *   - `stream` is a hipStream_t (0 = the null stream); every call is
 *     asynchronous on it and allocates nothing;
 *   - shapes are validated on the host before any launch; the return value is
 *     MK_OK or an MK_E* code, and mk_last_error() describes the failure.
 *     Nothing is launched when a call fails validation.
 */
#ifndef MK_KERNELS_H_
#define MK_KERNELS_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  MK_OK = 0,
  MK_EINVAL = 1,        /* bad pointer, shape or size */
  MK_EUNSUPPORTED = 2,  /* valid request this build does not implement */
  MK_EWORKSPACE = 3,    /* workspace missing or too small */
  MK_ELAUNCH = 4        /* the HIP launch itself failed */
};

/* Message for the last failing call on this thread ("" when none). */
const char* mk_last_error(void);

/* Library version string. */
const char* mk_version(void);

/* ------------------------------------------------------------------------
 * Quantized matmul, any M: HBM bound at decode shapes (M <= 16), MFMA bound
 * from a few hundred rows.
 *
 * Replaces the reference's affine quantized GEMM
 * (src/jax_plugins/silicon/quantized.py:1077-1152, kernels :760-958), which
 * reads W [N, K] as uint32 words of eight nibbles and runs outside jax.jit,
 * with the workload's jit-level format:
 *
 *   int4 g64:  x bf16 [M, K]; w_packed uint8 [K/2, N], two nibbles per byte
 *              along K, low nibble = even k (reference nibble order,
 *              quantized.py:189-190); scale bf16 [K/64, N]; zero uint8
 *              [K/64, N] holding 0..15.  y = x @ ((w - zero) * scale), bf16
 *              [M, N], f32 accumulation.
 *   int8 pc:   x bf16 [M, K]; w int8 [K, N]; scale f32 [N].
 *              y = x @ (w * scale), bf16 [M, N], f32 accumulation.
 *
 * Both need K % 64 == 0 and N % 8 == 0.  `workspace` receives split-K
 * partial sums when a call splits K across workgroups, and for many rows
 * (M >= 768, or M >= 256 when N % 64 != 0) the bf16-dequantised W [K, N]
 * that the bf16 GEMM then multiplies; mk_qmatmul_workspace_bytes gives the
 * size, 0 when none is needed (then workspace may be NULL).  Its first 64 KB hold per-tile arrival counters:
 * zero-fill a workspace once before its first use; every completed call
 * leaves the counters at zero again.  Calls that share a workspace must be
 * ordered (same stream).
 * ---------------------------------------------------------------------- */
enum { MK_QFMT_INT4_G64 = 0, MK_QFMT_INT8_PC = 1 };

int64_t mk_qmatmul_workspace_bytes(int fmt, int64_t M, int64_t K, int64_t N);

/* 1 when a *_matmul_epilogue_bf16 call of this shape with this epilogue
 * runs, 0 when it would return an error: MK_EPI_SWIGLU_PAIRS takes the
 * dequantise-then-GEMM route only (many rows, M % 256 == 0, N % 256 == 0).
 * Host-only; no reference counterpart (callers use it to choose between
 * the paired and the two-product form). */
int mk_qmatmul_epilogue_supported(int fmt, int64_t M, int64_t K, int64_t N, int epilogue);

int mk_int4g64_matmul_bf16(const void* x, const void* w_packed, const void* scale,
                           const void* zero, void* y, int64_t M, int64_t K, int64_t N,
                           void* workspace, int64_t workspace_bytes, void* stream);

int mk_int8pc_matmul_bf16(const void* x, const void* w, const void* scale, void* y,
                          int64_t M, int64_t K, int64_t N, void* workspace,
                          int64_t workspace_bytes, void* stream);

/* The same with an epilogue against aux (bf16 [M, N]), as for
 * mk_gemm_bf16_epilogue (MK_EPI_ADD / MK_EPI_SWIGLU, declared below), fused
 * into the final bf16 store of whichever kernel runs; aux may equal y.
 * Bit-identical to the plain call followed by the elementwise program. */
int mk_int4g64_matmul_epilogue_bf16(const void* x, const void* w_packed, const void* scale,
                                    const void* zero, void* y, const void* aux, int epilogue, int64_t M,
                                    int64_t K, int64_t N, void* workspace, int64_t workspace_bytes,
                                    void* stream);

int mk_int8pc_matmul_epilogue_bf16(const void* x, const void* w, const void* scale, void* y,
                                   const void* aux, int epilogue, int64_t M, int64_t K, int64_t N,
                                   void* workspace, int64_t workspace_bytes, void* stream);

/* y = silu(x @ Wg) * (x @ Wu), bf16 [M, N], from two separate quantized
 * weights of the same format and shape (int4: packed / scale / zero of each;
 * int8: weight / scale of each), the SwiGLU of the reference's transformer
 * benchmark (benchmarks/vs_cpu.py:603-626) as jax.jit lowers it.  No single
 * reference handler does this: the reference runs the two products and the
 * elementwise ops separately; the result here is bit-identical to that
 * sequence (the two *_matmul_bf16 calls, then the SwiGLU elementwise
 * program).  Both weights are dequantised into one interleaved bf16 buffer
 * in the workspace and multiplied by one GEMM.  Many-row shapes only: the
 * workspace size is 0 or more when the shape runs (M % 256 == 0,
 * N % 128 == 0, K % 64 == 0, M on the dequantise-then-GEMM route), -1 when
 * it does not (then the call returns MK_EUNSUPPORTED). */
int64_t mk_qmatmul_swiglu_pair_workspace_bytes(int fmt, int64_t M, int64_t K, int64_t N);

int mk_int4g64_matmul_swiglu_pair_bf16(const void* x, const void* wg_packed, const void* g_scale,
                                       const void* g_zero, const void* wu_packed, const void* u_scale,
                                       const void* u_zero, void* y, int64_t M, int64_t K, int64_t N,
                                       void* workspace, int64_t workspace_bytes, void* stream);

int mk_int8pc_matmul_swiglu_pair_bf16(const void* x, const void* wg, const void* g_scale, const void* wu,
                                      const void* u_scale, void* y, int64_t M, int64_t K, int64_t N,
                                      void* workspace, int64_t workspace_bytes, void* stream);

/* mk_int4g64_matmul_bf16 without a workspace argument, for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  No counterpart in the reference.
 * The workspace is a file-scope device array of 8 MiB per GPU, held until the
 * process ends.  The many-row kernel (128 <= M < 768) runs here without its
 * K split when the split's partials would not fit (at K = 4096, N = 14336:
 * same results to the bf16 tolerance, not bit for bit); shapes whose plan
 * still needs more than 8 MiB (the dequantise-then-GEMM route, for example
 * M >= 768 at K = 4096, N = 14336) return MK_EWORKSPACE before any launch.
 * The first call on a device sets the array up (its address, and its
 * counters cleared by a kernel on `stream`).  The call allocates nothing and
 * otherwise gives bit-identical results to mk_int4g64_matmul_bf16.  Every
 * call on one GPU shares the array: calls that overlap in time on one GPU
 * (unordered streams) race. */
int mk_int4g64_matmul_bf16_noalloc(const void* x, const void* w_packed, const void* scale,
                                   const void* zero, void* y, int64_t M, int64_t K, int64_t N,
                                   void* stream);

/* ------------------------------------------------------------------------
 * dot_general GEMM (canonical batched NN form).
 *
 * Replaces the reference's dot_general lowering (HandleDotGeneral,
 * src/pjrt_plugin/ops/binary_ops.mm:644-1100; rank-2 NN path :1011-1019;
 * native tiled kernels runtime/metal_kernels.mm:2477-2761 selected by
 * ClassifyDotGeneralNN, core/mps_executable.mm:2706-2891).  The executor
 * reduces dot_general (batch dims, contracting dims, transposes) to
 *   C[b] = A[b] @ B[b],  A [batch, M, K], B [batch, K, N], C [batch, M, N],
 * all row-major and densely packed.
 *
 * mk_gemm_bf16: bf16 inputs, f32 accumulation; C is bf16 (out_f32 = 0) or
 *   f32 (out_f32 = 1, dot_general with preferred_element_type = f32,
 *   binary_ops.mm:775-782).
 * mk_gemm_f32:  f32 inputs and output, f32 products and accumulation.
 * Both need K % 8 == 0 and N % 8 == 0 (else MK_EUNSUPPORTED).
 * ---------------------------------------------------------------------- */
int mk_gemm_bf16(const void* a, const void* b, void* c, int64_t batch, int64_t M, int64_t N,
                 int64_t K, int out_f32, void* stream);

int mk_gemm_f32(const void* a, const void* b, void* c, int64_t batch, int64_t M, int64_t N,
                int64_t K, void* stream);

/* mk_gemm_bf16_epilogue: mk_gemm_bf16 with bf16 output and an elementwise
 * epilogue against aux (bf16, the layout of C), fused into the GEMM's store:
 *   MK_EPI_ADD:    c = r(r(acc) + aux)                       (residual add)
 *   MK_EPI_SWIGLU: c = r(r(aux * r(logistic(aux))) * r(acc)) (silu(aux) * acc)
 * r() is bf16 rounding; the results equal, bit for bit, mk_gemm_bf16
 * followed by the bf16 elementwise program (MK_EW_ADD, or MK_EW_LOGISTIC +
 * MK_EW_MUL + MK_EW_MUL) -- the reference runs these as separate MPSGraph
 * ops (ops/binary_ops.mm).  aux may equal c (in-place residual). */
enum { MK_EPI_NONE = 0, MK_EPI_ADD = 1, MK_EPI_SWIGLU = 2, MK_EPI_SWIGLU_PAIRS = 3 };
/* MK_EPI_SWIGLU_PAIRS: the gate and up projections as one product.  B's N
 * columns interleave 16-column blocks of the gate and up weights (gate
 * block q at columns 32q..32q+15, up block q at 32q+16..32q+31); C is
 * bf16 [batch, M, N/2] with
 *   C[m, 16q + c] = r(r(g * r(logistic(g))) * r(u)),
 *   g = r(acc[m, 32q + c]),  u = r(acc[m, 32q + 16 + c]),
 * bit-identical to two plain GEMMs and the MK_EPI_SWIGLU formula.  aux is
 * unused (may be null).  Needs the 256x256 kernel's shapes: M % 256 == 0,
 * N % 256 == 0, K % 32 == 0 (else MK_EUNSUPPORTED). */

int mk_gemm_bf16_epilogue(const void* a, const void* b, void* c, const void* aux, int epilogue,
                          int64_t batch, int64_t M, int64_t N, int64_t K, void* stream);

/* mk_gemm_bf16_nt: mk_gemm_bf16_epilogue with B given transposed, bt bf16
 * [batch, N, K] (k contiguous): C = A @ bt^T, the dot_general whose rhs
 * contracts its last dimension (x @ W.T, q @ k^T), which the reference
 * lowers with a transpose inside HandleDotGeneral
 * (src/pjrt_plugin/ops/binary_ops.mm:644-1100).  Epilogues as above.
 * Results equal, bit for bit, mk_gemm_bf16_epilogue on the transposed copy
 * of bt: the fragments reach the matrix cores with the same values in the
 * same k order.  Needs M % 256 == 0, N % 256 == 0, K % 32 == 0 (else
 * MK_EUNSUPPORTED). */
int mk_gemm_bf16_nt(const void* a, const void* bt, void* c, const void* aux, int epilogue, int64_t batch,
                    int64_t M, int64_t N, int64_t K, void* stream);

/* Routes of the bf16 product (B [K, N]): the kernels mk_gemm_bf16 and
 * mk_gemm_bf16_epilogue choose between by shape.  Every route computes
 * each output's k in the same order in the same MFMA, so all give the same
 * bits; they differ only in speed.
 *   RING        256 x 256 tiles, 4-stage LDS DMA ring   (M, N % 256, K % 32)
 *   PIPE        the same with fragment prefetch, 5 stages (and K >= 320)
 *   PERSIST     256 x 256, one workgroup per CU over the tiles
 *               (K <= 128, bf16 output, no paired epilogue)
 *   SHORT       128 x 128 with all of K in LDS (M, N % 128, K % 32,
 *               K <= 256, bf16 output, no paired epilogue)
 *   REG256      256 x 256, register-staged operands (M, N % 256, K % 64)
 *   GENERIC256, GENERIC128  any shape (no paired epilogue)
 * The reference picks between its GEMM variants the same way, by timing
 * them at the first plan build and keeping the fastest per device and
 * shape (AutotuneGemm, src/pjrt_plugin/core/mps_executable.mm:3433-3725;
 * its persistent cache :3270-3420). */
enum {
  MK_GEMM_ROUTE_DEFAULT = 0,
  MK_GEMM_ROUTE_RING = 1,
  MK_GEMM_ROUTE_PIPE = 2,
  MK_GEMM_ROUTE_PERSIST = 3,
  MK_GEMM_ROUTE_SHORT = 4,
  MK_GEMM_ROUTE_REG256 = 5,
  MK_GEMM_ROUTE_GENERIC256 = 6,
  MK_GEMM_ROUTE_GENERIC128 = 7,
  MK_GEMM_ROUTE_COUNT = 8
};

/* mk_gemm_bf16_epilogue (epilogue MK_EPI_NONE: mk_gemm_bf16, with
 * out_f32) on a given route; MK_GEMM_ROUTE_DEFAULT is the built-in choice.
 * A route that does not take the product is MK_EUNSUPPORTED. */
int mk_gemm_bf16_route(const void* a, const void* b, void* c, const void* aux, int epilogue, int64_t batch,
                       int64_t M, int64_t N, int64_t K, int out_f32, int route, void* stream);

/* 1 when the route takes the product, else 0.  Host-only. */
int mk_gemm_bf16_route_fits(int route, int64_t M, int64_t N, int64_t K, int epilogue, int out_f32);

/* Times every route that takes the product on `stream` (warm-up and timed
 * launches: MK_GEMM_AUTOTUNE_WARMUP, default 2, and MK_GEMM_AUTOTUNE_ITERS,
 * default 5, HIP events, the median per route), records the fastest in
 * the process's route table for the current device (architecture and CU
 * count), shape, epilogue class and output type, and returns it in *route
 * (and its median in *us); it creates and destroys two HIP events, and
 * allocates no device memory.  c holds the product afterwards.  Not under
 * stream capture, and aux may not be c (MK_EINVAL: every timed launch
 * rewrites c). */
int mk_gemm_bf16_autotune(const void* a, const void* b, void* c, const void* aux, int epilogue, int64_t batch,
                          int64_t M, int64_t N, int64_t K, int out_f32, void* stream, int* route, float* us);

/* The route table's entry for the product on the current device, or
 * MK_GEMM_ROUTE_DEFAULT when it has none. */
int mk_gemm_tuned_route(int64_t batch, int64_t M, int64_t N, int64_t K, int epilogue, int out_f32);

/* The route table as a text file: the header line that
 * mk_gemm_autotune_header returns ("mk-gemm-autotune 1 build <stamp>",
 * the stamp that of this library's build, so a table measured against
 * other kernels is refused), then one line per entry, "<arch> <CUs> <batch> <M> <N> <K>
 * <epilogue class> <out_f32> <route> <us>".  save writes it atomically
 * (a temporary file renamed) and returns the number of entries; load
 * merges a file's entries into the table and returns their number.  Both
 * return -MK_EINVAL on failure (load: a missing file, another header or a
 * malformed line, the table unchanged).  clear empties the table.
 * Host-only. */
int mk_gemm_autotune_save(const char* path);
int mk_gemm_autotune_load(const char* path);
void mk_gemm_autotune_clear(void);
const char* mk_gemm_autotune_header(void);

/* mk_dot_general: the dot_general cases the tiled GEMMs do not take,
 * with the reference's semantics (HandleDotGeneral,
 * src/pjrt_plugin/ops/binary_ops.mm:644-1100):
 *   - integer operands, exact in the result type (two's-complement
 *     wraparound, :806-809): S8 S16 S32 S64 U8 U16 U32 U64 inputs, any
 *     integer result (lax.dot preferred_element_type=int32 included);
 *   - K == 1 is a plain product, keeping XLA's signed zero (:904-1004);
 *   - any K and N, operands read through element strides (a transposed
 *     operand or a vector needs no copy);
 *   - F32 / BF16 / F16 inputs accumulate in f32 in k order; the result is
 *     F32 or the input type (round to nearest even).
 * C[b, m, n] = sum_k A[b, m, k] B[b, k, n]; A[b, m, k] is element
 * b*a_strides[0] + m*a_strides[1] + k*a_strides[2] of a, B[b, k, n] element
 * b*b_strides[0] + k*b_strides[1] + n*b_strides[2] of b; C is contiguous
 * [batch, M, N].  Types use the PJRT_Buffer_Type numbering below; both
 * operands must have the same type (MK_EUNSUPPORTED otherwise).  One
 * thread per output element: not a throughput path. */
enum {
  MK_TYPE_S8 = 2, MK_TYPE_S16 = 3, MK_TYPE_S32 = 4, MK_TYPE_S64 = 5, MK_TYPE_U8 = 6, MK_TYPE_U16 = 7,
  MK_TYPE_U32 = 8, MK_TYPE_U64 = 9, MK_TYPE_F16 = 10, MK_TYPE_F32 = 11, MK_TYPE_BF16 = 13
};

int mk_dot_general(int type_a, int type_b, int type_out, const void* a, const void* b, void* c, int64_t batch,
                   int64_t M, int64_t N, int64_t K, const int64_t* a_strides, const int64_t* b_strides,
                   void* stream);

/* ------------------------------------------------------------------------
 * Last-axis row operations on X [rows, cols] (row-major).
 *
 * Replace the reference's native row kernels and the MPSGraph reductions
 * around them: softmax (pattern FuseSoftmaxPatterns,
 * src/pjrt_plugin/core/mps_executable.mm:2091-2372; kernels
 * runtime/metal_kernels.mm:1579-1740 and the XLA rounding emulation
 * :1742-1819), last-axis sum/max (NativeIntrinsicReduceHandler,
 * mps_executable.mm:4911-5070; kernels metal_kernels.mm:769-1065), argmax
 * (HandleMultiResultReduce, ops/reduction_ops.mm:1407-1668) and RMSNorm
 * (the workload's x * rsqrt(mean(x^2) + eps) * g; the reference's closest
 * path is its LayerNorm fusion, mps_executable.mm:1457-1820).
 *
 * dtype: MK_DT_F32 or MK_DT_BF16 (x, g and y share it; argmax writes int32).
 * softmax: a row whose max is NaN or +-inf becomes all NaN.  argmax: index
 * of the first NaN, else of the first maximum, -0 == +0.  max / min: NaN
 * propagates, -0 < +0.  sum: f32 accumulation, result in dtype.  The
 * planner flattens a reduce over several trailing dims into one row and
 * combines a non-neutral init value afterwards (mps_executable.mm:955-975).
 * ---------------------------------------------------------------------- */
enum { MK_DT_F32 = 0, MK_DT_BF16 = 1 };
enum { MK_REDUCE_SUM = 0, MK_REDUCE_MAX = 1, MK_REDUCE_MIN = 2 };

int mk_softmax_lastdim(int dtype, const void* x, void* y, int64_t rows, int64_t cols, void* stream);

int mk_rmsnorm_lastdim(int dtype, const void* x, const void* g, void* y, int64_t rows, int64_t cols,
                       float eps, void* stream);

int mk_argmax_lastdim(int dtype, const void* x, void* out_i32, int64_t rows, int64_t cols,
                      void* stream);

int mk_reduce_lastdim(int dtype, int op, const void* x, void* y, int64_t rows, int64_t cols,
                      void* stream);

/* ------------------------------------------------------------------------
 * Decoder-layer data movement and masking (the workload's Llama-style
 * decoder config).  No single reference function corresponds: jax.jit
 * lowers these steps to generic StableHLO (the reference's own transformer
 * layer benchmark, benchmarks/vs_cpu.py:603-626: qkv reshape (B, T, 3, H,
 * Dh), q @ swapaxes(k) * scale, softmax, @ v, transpose back), which the
 * reference runs op by op on MPSGraph.  All bf16, head dim D = 128.
 *
 * mk_rope_qkv_split_bf16: qkv [B*S, 3*H*D] (blocks q | k | v) ->
 *   q [B*H, S, D], k, v [B*H, S, D]; q and k rotated:
 *   out[i] = x[i] c - x[i+D/2] s, out[i+D/2] = x[i+D/2] c + x[i] s with
 *   c, s = cos_table / sin_table [S, D/2] (f32).  k_rows = 0 writes k
 *   transposed, kT [B*H, D, S] (the B operand of q @ k^T for mk_gemm_bf16).
 *   Needs S % 64 == 0.
 * mk_softmax_causal_bf16: scores [batches, S, S] -> probs: row i keeps
 *   columns j <= i, p = exp(scale s - m) / sum in f32, zeros for j > i.
 *   Needs S % 8 == 0, S <= 8192.
 * mk_merge_heads_bf16: o [B*H, S, D] -> out [B*S, H*D].
 * mk_attention_causal_bf16: the three steps above in one pass (scores,
 *   causal softmax in f32 with the online max/sum rescaling, P rounded to
 *   bf16 for P @ V, f32 accumulation) from q, k, v [B*H, S, D] (k_rows = 1)
 *   straight to out [B*S, H*D].  Needs S % 128 == 0 and a positive finite
 *   scale (MK_EINVAL otherwise).
 * ---------------------------------------------------------------------- */
int mk_rope_qkv_split_bf16(const void* qkv, const float* cos_table, const float* sin_table, void* q,
                           void* k, void* v, int64_t B, int64_t S, int64_t H, int64_t D, int k_rows,
                           void* stream);

int mk_attention_causal_bf16(const void* q, const void* k, const void* v, void* out, int64_t B, int64_t H,
                             int64_t S, int64_t D, float scale, void* stream);

int mk_softmax_causal_bf16(const void* scores, void* probs, int64_t batches, int64_t S, float scale,
                           void* stream);

int mk_merge_heads_bf16(const void* o, void* out, int64_t B, int64_t H, int64_t S, int64_t D,
                        void* stream);

/* ------------------------------------------------------------------------
 * Fused elementwise program (one pass over memory).
 *
 * Replaces the reference's elementwise MPSGraph segments
 * (core/mps_executable.mm:7393-7508) and its opt-in generated fusion kernels
 * (FusionSnippet :4303-4351, GenerateFusedKernelSource :4445-4586).  The
 * executor lowers a chain of StableHLO elementwise ops to instructions over
 * 12 register slots; MK_EW_LOAD reads input `a` (n elements; 1 element,
 * broadcast; or a divisor p of n elements read periodically, element i from
 * i mod p -- a broadcast that adds leading dimensions, such as a [T, T] mask
 * over [B, H, T, T] scores); its `b` field gives the input's element type
 * (MK_EW_IN_DEFAULT: the program's dtype, MK_EW_IN_F32, MK_EW_IN_BF16 --
 * the convert ops of mixed bf16 / f32 programs), MK_EW_CONST writes `imm`, every other op reads slots a (b, c)
 * and writes slot dst.  bf16 programs round each float result to bf16
 * (XLA:CPU's per-op rounding, reference ops/registry.h:273-287), except
 * for ops or'ed with MK_EW_KEEP_F32: an f32-typed node of a program whose
 * result is bf16 (f32 arithmetic between converts), computed and kept in
 * f32 (a no-op flag in f32 programs).
 * Comparisons give 1.0 / 0.0; SELECT yields b where a != 0, else c.
 * At most 32 instructions and 4 inputs; every source slot must be written
 * before it is read (checked on the host).
 * ---------------------------------------------------------------------- */
enum {
  MK_EW_LOAD = 0, MK_EW_CONST = 1,
  MK_EW_ADD = 2, MK_EW_SUB = 3, MK_EW_MUL = 4, MK_EW_DIV = 5, MK_EW_MAX = 6, MK_EW_MIN = 7,
  MK_EW_POW = 8,
  MK_EW_NEG = 9, MK_EW_ABS = 10, MK_EW_EXP = 11, MK_EW_LOG = 12, MK_EW_LOG1P = 13,
  MK_EW_EXPM1 = 14, MK_EW_TANH = 15, MK_EW_RSQRT = 16, MK_EW_SQRT = 17, MK_EW_LOGISTIC = 18,
  MK_EW_FLOOR = 19, MK_EW_CEIL = 20,
  MK_EW_CMP_EQ = 21, MK_EW_CMP_NE = 22, MK_EW_CMP_LT = 23, MK_EW_CMP_LE = 24,
  MK_EW_CMP_GT = 25, MK_EW_CMP_GE = 26,
  MK_EW_SELECT = 27, MK_EW_ROUND_BF16 = 28,
  MK_EW_NUM_OPS = 29
};

enum { MK_EW_IN_DEFAULT = 0, MK_EW_IN_F32 = 1, MK_EW_IN_BF16 = 2 };
enum { MK_EW_KEEP_F32 = 64 };

typedef struct mk_ew_instr {
  int32_t op;
  int32_t dst;
  int32_t a, b, c;
  float imm;
} mk_ew_instr;

int mk_elementwise(int dtype, const mk_ew_instr* prog, int n_instr, const void* const* inputs,
                   const int64_t* input_numel, int n_inputs, int out_slot, void* out, int64_t n,
                   void* stream);

/* The first mk_elementwise call of a program on a device compiles a
 * specialised straight-line kernel for it (hiprtc, gfx950) and caches it;
 * mk_elementwise_prepare does that ahead of time (at plan-build time, and
 * always before capturing a HIP graph).  Setting MK_EW_JIT=0 uses the
 * precompiled register-program interpreter instead (same results). */
int mk_elementwise_prepare(int dtype, const mk_ew_instr* prog, int n_instr, int n_inputs,
                           int out_slot);

/* ------------------------------------------------------------------------
 * Layout ops.
 *
 * mk_strided_copy replaces the reference's MPSGraph transpose / slice /
 * broadcast_in_dim / concatenate handlers (ops/shape_ops.mm:
 * HandleTranspose :304-333, HandleSlice :831-865, HandleBroadcastInDim
 * :137-153, HandleConcatenate :1208-1265): for every index (i_0 .. i_{r-1})
 * of `shape` (rank r <= 8),
 *   dst[dst_offset + sum_d i_d dst_strides[d]] =
 *       src[src_offset + sum_d i_d src_strides[d]]
 * with strides and offsets in elements of `elem_bytes` (1, 2, 4 or 8)
 * bytes.  A stride of 0 broadcasts; a concatenate is one call per operand
 * with its destination offset.  Strides and offsets must be >= 0.
 *
 * mk_iota replaces HandleIota (ops/tensor_creation_ops.mm:126-148): a
 * contiguous tensor of `shape` holding each element's index along `dim`,
 * of element type `dtype` (PJRT_Buffer_Type numbering, below).
 * ---------------------------------------------------------------------- */
enum {
  MK_IOTA_S8 = 2, MK_IOTA_S16 = 3, MK_IOTA_S32 = 4, MK_IOTA_S64 = 5, MK_IOTA_U8 = 6, MK_IOTA_U16 = 7,
  MK_IOTA_U32 = 8, MK_IOTA_U64 = 9, MK_IOTA_F16 = 10, MK_IOTA_F32 = 11, MK_IOTA_F64 = 12, MK_IOTA_BF16 = 13
};

int mk_strided_copy(const void* src, void* dst, int elem_bytes, int rank, const int64_t* shape,
                    const int64_t* src_strides, int64_t src_offset, const int64_t* dst_strides,
                    int64_t dst_offset, void* stream);
int mk_iota(void* dst, int dtype, int rank, const int64_t* shape, int dim, void* stream);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif  /* MK_KERNELS_H_ */
