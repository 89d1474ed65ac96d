// StableHLO (MLIR text form) intermediate representation used by the
// plugin's compile path.  The reference parses the same programs with MLIR
// and its StableHLO dialect (core/stablehlo_parser.mm:568-586); this build
// has no MLIR, so it reads the text form that jax's lowering prints, for the
// ops of the hot path, into this small SSA graph.
#pragma once

#include <stdint.h>

#include <stdexcept>
#include <string>
#include <vector>

namespace mkrt {

// PJRT_Buffer_Type numbering (include/mk_runtime.h).
enum DType : int {
  DT_INVALID = 0,
  DT_PRED = 1,
  DT_S8 = 2,
  DT_S16 = 3,
  DT_S32 = 4,
  DT_S64 = 5,
  DT_U8 = 6,
  DT_U16 = 7,
  DT_U32 = 8,
  DT_U64 = 9,
  DT_F16 = 10,
  DT_F32 = 11,
  DT_F64 = 12,
  DT_BF16 = 13
};

int dtype_bytes(int dt);
const char* dtype_name(int dt);

struct TensorType {
  int dtype = DT_INVALID;
  std::vector<int64_t> dims;
  int64_t numel() const;
  int64_t bytes() const { return numel() * dtype_bytes(dtype); }
  bool operator==(const TensorType& o) const { return dtype == o.dtype && dims == o.dims; }
  std::string str() const;
};

struct Value {
  TensorType type;
  int def_op = -1;  // -1: function argument
  int result_index = 0;
  int arg_index = -1;
  std::string name;
};

struct Op {
  std::string name;  // "add", "dot_general", ... (dialect prefix stripped); "return"
  std::vector<int> operands;
  std::vector<int> results;
  // Attributes used by the planner.
  std::vector<int64_t> dims;  // broadcast_in_dim dims, reduce dimensions, transpose permutation
  int64_t dim = -1;           // iota / concatenate dimension
  std::vector<int64_t> slice_start, slice_limit, slice_stride;  // slice
  std::vector<int64_t> lhs_batch, rhs_batch, lhs_contract, rhs_contract;
  std::string compare_dir;     // EQ NE LT LE GT GE
  std::string reduce_body;     // reduce: "add" "maximum" "minimum" "multiply" ... or "argmax" "argmin"
  std::vector<double> const_values;  // constant payload (one value when splat)
  bool const_splat = false;
  std::string text;  // the statement, for messages
};

struct Function {
  std::vector<Value> values;
  std::vector<Op> ops;
  std::vector<int> args;
  std::vector<int> rets;
};

struct ParseError : std::runtime_error {
  explicit ParseError(const std::string& m) : std::runtime_error(m) {}
};

// Parse the module's public entry function (@main, or the only public
// function); private functions reached by func.call are inlined.
Function parse_stablehlo_text(const std::string& text);

}  // namespace mkrt
