// Execution plan: the parsed StableHLO function mapped onto the hot-path
// kernels (mk_kernels.h).  The reference keeps the same split between a
// compile-time support check and a plan of native steps built once and then
// replayed per call (ExecutionPlan / NativeStep,
// src/pjrt_plugin/core/mps_executable.mm:97-287; BuildExecutionPlan :7627).
#pragma once

#include <stdint.h>

#include <stdexcept>
#include <string>
#include <vector>

#include "mk_kernels.h"
#include "shlo.h"

namespace mkrt {

enum SlotKind { SLOT_ARG = 0, SLOT_TEMP = 1, SLOT_CONST = 2, SLOT_VIEW = 3 };

// A device buffer the plan reads or writes.  Arguments are the caller's
// buffers; temporaries are allocated per execute; constants are uploaded once.
struct Slot {
  SlotKind kind = SLOT_TEMP;
  int64_t bytes = 0;
  int arg_index = -1;
  std::vector<uint8_t> data;  // SLOT_CONST contents
  int base = -1;              // SLOT_VIEW: the argument or constant slot it reads (an earlier slot)
  int64_t offset = 0;         // SLOT_VIEW: byte offset into that slot
};

enum StepKind {
  ST_GEMM_BF16,
  ST_GEMM_F32,
  ST_QMM_INT4,
  ST_QMM_INT8,
  ST_SOFTMAX,
  ST_RMSNORM,
  ST_ARGMAX,
  ST_REDUCE,
  ST_EW,
  ST_COPY,
  ST_ZERO,
  ST_DOT_GENERIC,
  ST_LAYOUT,  // strided copy (transpose, slice, broadcast, one concatenate operand)
  ST_IOTA,
  ST_ROPE,    // mk_rope_qkv_split_bf16: in {qkv, cos, sin}, out q, outs {k, v}
  ST_ATTN,    // mk_attention_causal_bf16: in {q, k, v}, out [B, S, H, D]
  ST_QMM_PAIR_INT4,  // mk_int4g64_matmul_swiglu_pair_bf16: in {x, wg, sg, zg, wu, su, zu}
  ST_QMM_PAIR_INT8   // mk_int8pc_matmul_swiglu_pair_bf16: in {x, wg, sg, wu, su}
};

struct Step {
  StepKind kind = ST_COPY;
  int dt = MK_DT_F32;     // MK_DT_* of the kernel
  std::vector<int> in;    // slot ids
  int out = -1;           // slot id
  int64_t batch = 1, M = 0, N = 0, K = 0;
  int out_f32 = 0;
  int b_t = 0;            // ST_GEMM_BF16: in[1] holds B^T [batch, N, K]
  int route = 0;          // ST_GEMM_BF16: MK_GEMM_ROUTE_* chosen when the plan is prepared (0: built-in)
  int epi = MK_EPI_NONE;  // ST_QMM_*: store epilogue against in.back()
  int64_t rows = 0, cols = 0;
  float eps = 0.f;
  int reduce_op = MK_REDUCE_SUM;
  std::vector<mk_ew_instr> prog;
  std::vector<int64_t> in_numel;
  int prog_out = 0;
  int64_t n = 0;      // elementwise element count
  int64_t bytes = 0;  // copy / zero size
  int type_a = 0, type_out = 0;            // ST_DOT_GENERIC: PJRT element types
  int64_t sa[3] = {0, 0, 0}, sb[3] = {0, 0, 0};  // ST_DOT_GENERIC strides (batch, m, k) / (batch, k, n)
  // ST_LAYOUT: dst[dst_off + sum i_d dst_st[d]] = src[src_off + sum i_d src_st[d]]
  // over `shape`, elements of elem_bytes; ST_IOTA: `shape`, iota_dim, type_out.
  std::vector<int64_t> shape, src_st, dst_st;
  int64_t src_off = 0, dst_off = 0;
  int elem_bytes = 0;
  int iota_dim = 0;
  // ST_ROPE / ST_ATTN: sizes, the score scale, further outputs.
  int64_t B = 0, H = 0, S = 0, D = 0;
  float scale = 1.f;
  std::vector<int> outs;
  std::string desc;
};

struct Plan {
  std::vector<Slot> slots;
  std::vector<Step> steps;
  std::vector<int> in_slot;   // per argument
  std::vector<int> out_slot;  // per result (a TEMP slot written by a step)
  std::vector<TensorType> in_type, out_type;
  int64_t workspace_bytes = 0;  // shared by the dequant-matmul steps
  std::string describe() const;
};

struct PlanError : std::runtime_error {
  int code;  // MKRT_* error code
  PlanError(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

// Maps every value the function returns onto kernel steps.  Throws
// PlanError(UNIMPLEMENTED) listing every op that has no kernel route.
Plan build_plan(const Function& fn);

}  // namespace mkrt
