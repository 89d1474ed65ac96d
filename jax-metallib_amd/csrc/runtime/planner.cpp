// Planner: StableHLO graph -> kernel steps.
//
// Walks back from the returned values.  Each value is produced by one of:
//   - a fused pattern rooted at it (softmax, RMSNorm, argmax, last-axis
//     reduce, dot_general as GEMM, dot_general over a dequantized int4/int8
//     weight as one dequant-matmul), matched structurally the way the
//     reference's fusion passes match MLIR (IsSoftmaxPattern,
//     core/mps_executable.mm:1922-2089; LayerNorm :1457-1820; argmax
//     detectArgReduceKind, ops/reduction_ops.mm:74-115; HandleDotGeneral,
//     ops/binary_ops.mm:644-1100);
//   - an elementwise program: the maximal elementwise DAG under the value,
//     scalars folded in as immediates, lowered to mk_elementwise
//     instructions (the reference's fused elementwise segments,
//     core/mps_executable.mm:7393-7508 and :4303-4586);
//   - a view (reshape, same-type convert, size-1 broadcast) of another value,
//     which shares its buffer;
//   - an argument or a constant.
// Pattern internals that something else also needs are simply computed
// again by that consumer, so matches never depend on use counts.
#include "planner.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <cmath>
#include <functional>
#include <map>
#include <set>
#include <sstream>
#include <stdexcept>
#include <tuple>

#include "mk_runtime.h"

namespace mkrt {

namespace {

bool is_float(int dt) { return dt == DT_F32 || dt == DT_BF16 || dt == DT_F16 || dt == DT_F64; }

int mk_dt(int dt) { return dt == DT_F32 ? MK_DT_F32 : dt == DT_BF16 ? MK_DT_BF16 : -1; }

float to_bf16_value(double v) {
  float f = (float)v;
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7f800000u) != 0x7f800000u) u += 0x7fffu + ((u >> 16) & 1u);
  else if (u & 0x007fffffu) u |= 0x00400000u;
  u &= 0xffff0000u;
  memcpy(&f, &u, 4);
  return f;
}

double round_to(double v, int dt) {
  if (dt == DT_F32) return (float)v;
  if (dt == DT_BF16) return to_bf16_value(v);
  return v;
}

const std::set<std::string>& unary_ops() {
  static const std::set<std::string> s = {"negate", "abs", "exponential", "log", "log_plus_one",
                                          "exponential_minus_one", "tanh", "rsqrt", "sqrt",
                                          "logistic", "floor", "ceil", "not", "convert"};
  return s;
}
const std::set<std::string>& binary_ops() {
  static const std::set<std::string> s = {"add", "subtract", "multiply", "divide", "maximum",
                                          "minimum", "power", "compare", "and", "or"};
  return s;
}

class Planner {
 public:
  explicit Planner(const Function& f) : f_(f), slot_of_(f.values.size(), -1), state_(f.values.size(), 0) {}

  Plan run() {
    for (size_t i = 0; i < f_.args.size(); ++i) {
      const int a = f_.args[i];
      Slot s;
      s.kind = SLOT_ARG;
      s.arg_index = (int)i;
      s.bytes = type(a).bytes();
      plan_.in_slot.push_back(new_slot(s));
      slot_of_[a] = plan_.in_slot.back();
      plan_.in_type.push_back(type(a));
    }
    std::set<int> used_out;
    for (int r : f_.rets) {
      int s = need(r);
      if (!unsupported_.empty()) continue;
      // Results own their memory: a result that is an argument, a constant
      // or a buffer already handed to another result gets its own copy.
      if (plan_.slots[s].kind != SLOT_TEMP || used_out.count(s)) {
        Step st;
        st.kind = ST_COPY;
        st.in = {s};
        st.bytes = type(r).bytes();
        Slot t;
        t.bytes = st.bytes;
        st.out = new_slot(t);
        st.desc = "copy " + type(r).str();
        plan_.steps.push_back(st);
        s = st.out;
      }
      used_out.insert(s);
      plan_.out_slot.push_back(s);
      plan_.out_type.push_back(type(r));
    }
    if (!unsupported_.empty()) {
      std::string m = "unsupported operations for the MI355X plugin: ";
      bool first = true;
      for (const std::string& u : unsupported_) {
        m += (first ? "" : "; ") + u;
        first = false;
      }
      throw PlanError(MKRT_UNIMPLEMENTED, m);
    }
    return plan_;
  }

 private:
  const Function& f_;
  Plan plan_;
  std::vector<int> slot_of_;
  std::vector<char> state_;  // 1 = in progress (cycle guard)
  std::set<std::string> unsupported_;

  // ---- graph helpers -------------------------------------------------------
  const TensorType& type(int v) const { return f_.values[v].type; }
  const Op* def(int v) const { return f_.values[v].def_op < 0 ? nullptr : &f_.ops[f_.values[v].def_op]; }
  bool is(int v, const char* name) const {
    const Op* o = def(v);
    return o && o->name == name;
  }
  int64_t numel(int v) const { return type(v).numel(); }
  int64_t last_dim(int v) const { return type(v).dims.empty() ? 1 : type(v).dims.back(); }

  int new_slot(const Slot& s) {
    plan_.slots.push_back(s);
    return (int)plan_.slots.size() - 1;
  }

  void reject(const Op* op, const std::string& why) {
    unsupported_.insert((op ? "stablehlo." + op->name : std::string("value")) + (why.empty() ? "" : " (" + why + ")"));
  }

  static bool monotonic(const std::vector<int64_t>& d) {
    for (size_t i = 1; i < d.size(); ++i)
      if (d[i] <= d[i - 1]) return false;
    return true;
  }

  // A broadcast_in_dim that only inserts size-1 dimensions (same element
  // order), i.e. a reshape.
  bool is_expand(const Op& op, int v) const {
    if (op.name != "broadcast_in_dim" || op.operands.empty()) return false;
    return numel(op.operands[0]) == numel(v) && monotonic(op.dims);
  }

  // Same buffer contents: reshape, same-type convert, size-1 expansion.
  int view_src(int v) const {
    const Op* op = def(v);
    if (!op || op->operands.empty()) return -1;
    const int s = op->operands[0];
    if (op->name == "reshape" && numel(s) == numel(v) && type(s).dtype == type(v).dtype) return s;
    if (op->name == "convert" && type(s).dtype == type(v).dtype) return s;
    if (is_expand(*op, v) && type(s).dtype == type(v).dtype) return s;
    if (op->name == "transpose" && trivial_perm(op->dims, type(s).dims)) return s;
    return -1;
  }
  // A permutation that keeps the relative order of every dimension larger
  // than 1 leaves the element order unchanged.
  static bool trivial_perm(const std::vector<int64_t>& perm, const std::vector<int64_t>& src_dims) {
    int64_t last = -1;
    for (int64_t p : perm) {
      if (p < 0 || p >= (int64_t)src_dims.size()) return false;
      if (src_dims[p] == 1) continue;
      if (p < last) return false;
      last = p;
    }
    return true;
  }
  int peel_view(int v) const {
    for (int s; (s = view_src(v)) >= 0;) v = s;
    return v;
  }
  // Views and converts (for dtype-changing converts the caller checks the
  // source type it ends at).
  int peel_cvt(int v) const {
    while (true) {
      int s = view_src(v);
      if (s < 0 && is(v, "convert")) s = def(v)->operands[0];
      if (s < 0) return v;
      v = s;
    }
  }

  // v is a splat constant (through broadcasts, reshapes, converts).
  bool splat(int v, double* out) const {
    const int dt = type(v).dtype;
    int u = v;
    while (true) {
      const Op* op = def(u);
      if (!op) return false;
      if (op->name == "constant") {
        if (op->const_values.empty()) return false;
        const double c = op->const_values[0];
        for (double x : op->const_values)
          if (!(x == c || (x != x && c != c))) return false;
        *out = round_to(c, is_float(dt) ? dt : DT_F64);
        return true;
      }
      if ((op->name == "broadcast_in_dim" || op->name == "reshape" || op->name == "convert") && !op->operands.empty()) {
        u = op->operands[0];
        continue;
      }
      return false;
    }
  }
  bool splat_is(int v, double c) const {
    double x;
    return splat(v, &x) && (x == c || (x != x && c != c));
  }

  // v[i*C + j] == s[i] (broadcast along the last axis); returns s or -1.
  int row_src(int v, int64_t C) const {
    while (true) {
      const Op* op = def(v);
      if (!op || op->operands.empty()) return -1;
      const int s = op->operands[0];
      if ((op->name == "reshape" || (op->name == "convert" && type(s).dtype == type(v).dtype)) &&
          numel(s) == numel(v) && last_dim(s) == C && last_dim(v) == C) {
        v = s;
        continue;
      }
      if (op->name != "broadcast_in_dim" || !monotonic(op->dims) || C <= 0 || numel(s) * C != numel(v))
        return -1;
      const int last = (int)type(v).dims.size() - 1;
      for (size_t i = 0; i < op->dims.size(); ++i)
        if (op->dims[i] == last && type(s).dims[i] != 1) return -1;
      return s;
    }
  }
  // v[i*C + j] == s[j]; returns s or -1.
  int col_src(int v, int64_t C) const {
    while (true) {
      const Op* op = def(v);
      if (!op || op->operands.empty()) return -1;
      const int s = op->operands[0];
      if (op->name == "reshape" && numel(s) == numel(v) && last_dim(s) == C && last_dim(v) == C &&
          numel(s) == C) {
        return s;
      }
      if (op->name != "broadcast_in_dim" || !monotonic(op->dims) || numel(s) != C) return -1;
      const int last = (int)type(v).dims.size() - 1;
      bool ok = false;
      for (size_t i = 0; i < op->dims.size(); ++i) {
        if (op->dims[i] == last && type(s).dims[i] == C) ok = true;
      }
      return ok || C == 1 ? s : -1;
    }
  }

  // Last-axis reduce: returns the reduced input of `v`'s defining op (with
  // body `body` and the neutral init) or -1.
  int reduce_last_input(int v, const char* body) const {
    const Op* op = def(v);
    if (!op || op->name != "reduce" || op->operands.size() != 2 || op->reduce_body != body) return -1;
    const int x = op->operands[0];
    const int rank = (int)type(x).dims.size();
    if (rank == 0 || op->dims.size() != 1 || op->dims[0] != rank - 1) return -1;
    double init;
    if (!splat(op->operands[1], &init)) return -1;
    if (strcmp(body, "add") == 0 && init != 0.0) return -1;
    if (strcmp(body, "maximum") == 0 && !(init == -INFINITY)) return -1;
    return x;
  }

  // Reduce over the trailing dims (one or several, in order) with an add,
  // maximum or minimum body and a splat init: the input, the kernel op, the
  // flattened row length and whether the init is the body's neutral value.
  bool reduce_trailing(int v, int* x, int* op_kind, int64_t* cols, double* init, bool* neutral) const {
    const Op* op = def(v);
    if (!op || op->name != "reduce" || op->operands.size() != 2 || op->dims.empty()) return false;
    *x = op->operands[0];
    const std::vector<int64_t>& xd = type(*x).dims;
    const int rank = (int)xd.size(), nd = (int)op->dims.size();
    for (int i = 0; i < nd; ++i)
      if (op->dims[i] != rank - nd + i) return false;
    if (!splat(op->operands[1], init)) return false;
    *cols = 1;
    for (int i = rank - nd; i < rank; ++i) *cols *= xd[i];
    if (op->reduce_body == "add") {
      *op_kind = MK_REDUCE_SUM;
      *neutral = *init == 0.0;
    } else if (op->reduce_body == "maximum") {
      *op_kind = MK_REDUCE_MAX;
      *neutral = *init == -INFINITY;
    } else if (op->reduce_body == "minimum") {
      *op_kind = MK_REDUCE_MIN;
      *neutral = *init == INFINITY;
    } else {
      return false;
    }
    return true;
  }

  // ---- materialisation -----------------------------------------------------
  int need(int v) {
    if (slot_of_[v] >= 0) return slot_of_[v];
    if (state_[v]) throw PlanError(MKRT_INVALID_ARGUMENT, "cyclic value graph");
    state_[v] = 1;
    const int s = produce(v);
    state_[v] = 0;
    slot_of_[v] = s;
    return s;
  }

  int temp_for(int v) {
    Slot s;
    s.bytes = type(v).bytes();
    return new_slot(s);
  }

  int produce(int v) {
    const Op* op = def(v);
    if (!op) return 0;  // arguments are pre-assigned
    const int src = view_src(v);
    if (src >= 0) return need(src);
    if (numel(v) == 0) return temp_for(v);  // nothing to compute
    if (op->name == "slice") {
      const int sv = slice_view(v, *op);
      if (sv >= 0) return sv;
    }
    const std::string& n = op->name;
    if (n == "constant") {
      double c;
      if (numel(v) > 4096 && splat(v, &c) && mk_dt(type(v).dtype) >= 0) return ew_root(v);
      return const_slot(v, *op);
    }
    if (n == "dot_general" || n == "dot") {
      int s;
      if ((s = attention_merged(v)) >= 0) return unmerge_heads(v, s);
      if (try_qmm(v, &s)) return s;
      if (try_gemm(v, *op, &s)) return s;
      return dummy(v);
    }
    if (n == "reduce") {
      int s;
      if (try_argmax(v, *op, &s)) return s;
      if (try_reduce(v, &s)) return s;
      reject(op, "reduce over " + type(op->operands[0]).str() + " with body " + op->reduce_body);
      return dummy(v);
    }
    if (n == "divide") {
      int s;
      if (try_softmax(v, &s)) return s;
    }
    if (n == "multiply") {
      int s;
      if (try_rmsnorm(v, &s)) return s;
    }
    if (n == "add" || n == "multiply") {
      int s;
      if (n == "multiply" && try_qmm_pair(v, &s)) return s;
      if (try_qmm_epilogue(v, &s)) return s;
    }
    if (n == "convert") {
      int s;
      if (try_qmm(v, &s)) return s;
      if (try_reduce(v, &s)) return s;
    }
    if (is_elementwise(v)) return ew_root(v);
    {
      int s;
      if (n == "transpose" && (s = decoder_transpose(v)) >= 0) return s;
      if (try_layout(v, *op, &s)) return s;
    }
    reject(op, "");
    return dummy(v);
  }

  // ---- decoder patterns ------------------------------------------------------
  // Causal attention and rotate-half RoPE as jnp writes them (the workload's
  // decoder layer, the reference's transformer-layer benchmark,
  // benchmarks/vs_cpu.py:603-626) run on the decoder kernels
  // (mk_attention_causal_bf16, mk_rope_qkv_split_bf16) instead of op by op.
  // The attention kernel keeps scores and probabilities in f32 until P @ V
  // (P rounded to bf16) where the jnp form rounds each bf16 op: results agree
  // at the bf16 tolerance, not bit for bit.  MK_PLAN_DECODER_FUSION=0 turns
  // both routes off.
  static bool decoder_fusion() {
    const char* e = getenv("MK_PLAN_DECODER_FUSION");
    return !(e && e[0] == '0');
  }
  static bool dims_eq(const std::vector<int64_t>& d, std::initializer_list<int64_t> w) {
    return d == std::vector<int64_t>(w);
  }

  // t [B, S, H, D] = reshape(slice(x5, dim 2 = [j, j+1))) with x5 [B, S, 3, H, D]
  // (qkv.reshape(B, S, 3, H, D)[:, :, j]); returns x5 and j through the pointers.
  bool head_slice(int t, int* x5, int* j) const {
    const std::vector<int64_t>& td = type(t).dims;
    if (td.size() != 4 || type(t).dtype != DT_BF16) return false;
    const Op* rs = def(t);
    if (!rs || rs->name != "reshape") return false;
    const int sl = rs->operands[0];
    const Op* so = def(sl);
    if (!so || so->name != "slice") return false;
    const int x = so->operands[0];
    const std::vector<int64_t>& xd = type(x).dims;
    if (!(xd.size() == 5 && xd[0] == td[0] && xd[1] == td[1] && xd[2] == 3 && xd[3] == td[2] && xd[4] == td[3]))
      return false;
    for (int d = 0; d < 5; ++d) {
      if (so->slice_stride[d] != 1) return false;
      if (d == 2) continue;
      if (so->slice_start[d] != 0 || so->slice_limit[d] != xd[d]) return false;
    }
    if (so->slice_limit[2] != so->slice_start[2] + 1) return false;
    *x5 = x;
    *j = (int)so->slice_start[2];
    return true;
  }

  // cb [B, S, H, D/2] = table [S, D/2] broadcast over B and H (through a
  // reshape to [1, S, 1, D/2]); returns the table or -1.
  int rope_table(int cb, int64_t S, int64_t Dh) const {
    const Op* b = def(cb);
    if (!b || b->name != "broadcast_in_dim" || type(cb).dtype != DT_F32) return -1;
    int u = b->operands[0];
    if (dims_eq(b->dims, {1, 3}) && dims_eq(type(u).dims, {S, Dh})) return u;
    if (!dims_eq(b->dims, {0, 1, 2, 3}) || !dims_eq(type(u).dims, {1, S, 1, Dh})) return -1;
    const Op* r = def(u);
    if (!r || r->name != "reshape" || !dims_eq(type(r->operands[0]).dims, {S, Dh})) return -1;
    return r->operands[0];
  }

  // The two factors of a multiply, or false.
  bool factors(int v, int* a, int* b) const {
    const Op* m = def(v);
    if (!m || m->name != "multiply" || m->operands.size() != 2) return false;
    *a = m->operands[0];
    *b = m->operands[1];
    return true;
  }
  // v = x * t or t * x with t a broadcast RoPE table: returns x and the table.
  bool rope_term(int v, int64_t S, int64_t Dh, int* x, int* table) const {
    int a, b;
    if (!factors(v, &a, &b)) return false;
    int t;
    if ((t = rope_table(b, S, Dh)) >= 0) {
      *x = a;
      *table = t;
      return true;
    }
    if ((t = rope_table(a, S, Dh)) >= 0) {
      *x = b;
      *table = t;
      return true;
    }
    return false;
  }
  // xs = slice(xf, last axis [lo, lo + Dh)) of xf [B, S, H, D]; returns xf or -1.
  int half_slice(int xs, int64_t lo) const {
    const Op* so = def(xs);
    if (!so || so->name != "slice") return -1;
    const int xf = so->operands[0];
    const std::vector<int64_t>& d = type(xf).dims;
    if (d.size() != 4) return -1;
    for (int k = 0; k < 4; ++k) {
      if (so->slice_stride[k] != 1) return -1;
      const int64_t a = k == 3 ? lo : 0, b = k == 3 ? lo + d[3] / 2 : d[k];
      if (so->slice_start[k] != a || so->slice_limit[k] != b) return -1;
    }
    return xf;
  }

  struct RopeMatch {
    int x5 = -1, j = -1, cos = -1, sin = -1;
    int64_t B = 0, S = 0, H = 0, D = 0;
  };
  // r [B, S, H, D] bf16 = concatenate([x0 c - x1 s, x1 c + x0 s], -1) in f32
  // with x = head j of the fused qkv, x0 / x1 its halves, c / s the tables
  // [S, D/2]: the rotate-half RoPE of mk_rope_qkv_split_bf16.
  bool match_rope(int r, RopeMatch* m) const {
    const Op* cv = def(r);
    if (!cv || cv->name != "convert" || type(r).dtype != DT_BF16 || type(r).dims.size() != 4) return false;
    const int cat = cv->operands[0];
    const Op* co = def(cat);
    if (!co || co->name != "concatenate" || co->operands.size() != 2 || co->dim != 3 ||
        type(cat).dtype != DT_F32)
      return false;
    const std::vector<int64_t>& d = type(r).dims;
    const int64_t S = d[1], Dh = d[3] / 2;
    const Op* lo = def(co->operands[0]);
    const Op* hi = def(co->operands[1]);
    if (!lo || lo->name != "subtract" || !hi || hi->name != "add") return false;
    int a0, t0, a1, t1;  // lo = a0 * t0 - a1 * t1
    if (!rope_term(lo->operands[0], S, Dh, &a0, &t0) || !rope_term(lo->operands[1], S, Dh, &a1, &t1)) return false;
    const int xf = half_slice(a0, 0);
    if (xf < 0 || half_slice(a1, Dh) != xf) return false;
    for (int order = 0; order < 2; ++order) {  // hi = x1 * c + x0 * s, either order
      int b0, u0, b1, u1;
      if (!rope_term(hi->operands[order], S, Dh, &b0, &u0) || !rope_term(hi->operands[1 - order], S, Dh, &b1, &u1))
        continue;
      if (b0 != a1 || u0 != t0 || b1 != a0 || u1 != t1) continue;
      const Op* xc = def(xf);
      if (!xc || xc->name != "convert" || type(xf).dtype != DT_F32) return false;
      int x5, j;
      if (!head_slice(xc->operands[0], &x5, &j) || j > 1) return false;
      m->x5 = x5;
      m->j = j;
      m->cos = t0;
      m->sin = t1;
      m->B = d[0];
      m->S = S;
      m->H = d[2];
      m->D = d[3];
      return true;
    }
    return false;
  }

  struct RopeOut {
    int q = -1, k = -1, v = -1;
  };
  std::map<std::tuple<int, int, int>, RopeOut> rope_steps_;  // (x5, cos, sin)
  std::map<int, RopeOut> rope_by_qkv_;                       // x5 -> the first rope step on it

  RopeOut rope_step(const RopeMatch& m) {
    const auto key = std::make_tuple(m.x5, m.cos, m.sin);
    auto it = rope_steps_.find(key);
    if (it != rope_steps_.end()) return it->second;
    Step st;
    st.kind = ST_ROPE;
    st.dt = MK_DT_BF16;
    st.in = {need(m.x5), need(m.cos), need(m.sin)};
    const int64_t bytes = m.B * m.H * m.S * m.D * 2;
    RopeOut o;
    for (int* p : {&o.q, &o.k, &o.v}) {
      Slot t;
      t.bytes = bytes;
      *p = new_slot(t);
    }
    st.out = o.q;
    st.outs = {o.k, o.v};
    st.B = m.B;
    st.S = m.S;
    st.H = m.H;
    st.D = m.D;
    st.desc = "rope_qkv_split B=" + std::to_string(m.B) + " S=" + std::to_string(m.S) + " H=" + std::to_string(m.H) +
              " D=" + std::to_string(m.D) + " bf16";
    plan_.steps.push_back(st);
    rope_steps_[key] = o;
    if (!rope_by_qkv_.count(m.x5)) rope_by_qkv_[m.x5] = o;
    return o;
  }

  // transpose(t, [0, 2, 1, 3]) of a RoPE'd head (q or k), of the v head of a
  // fused qkv already split by a rope step, or of a fused attention's
  // [B, H, S, D] output: the slot holding it, or -1.
  int decoder_transpose(int v) {
    if (!decoder_fusion()) return -1;
    const Op* op = def(v);
    if (!dims_eq(op->dims, {0, 2, 1, 3})) return -1;
    const int t = op->operands[0];
    int s;
    if ((s = attention_merged(t)) >= 0) return s;
    RopeMatch m;
    if (match_rope(t, &m) && m.D == 128 && m.S % 64 == 0) {
      const RopeOut o = rope_step(m);
      return m.j == 0 ? o.q : o.k;
    }
    int x5, j;
    if (head_slice(t, &x5, &j) && j == 2) {
      auto it = rope_by_qkv_.find(x5);
      if (it != rope_by_qkv_.end()) return it->second.v;
    }
    return -1;
  }

  struct AttnMatch {
    int q = -1, k = -1, v = -1;
    int64_t B = 0, H = 0, S = 0, D = 0;
    float scale = 1.f;
  };
  // o [B, H, S, D] = softmax(where(causal, (q @ k^T) * scale, -inf)) @ v, all
  // bf16, batched over (B, H); k^T a transpose of k or k contracted on its
  // last axis; the mask i >= j a compile-time constant [S, S] broadcast over
  // (B, H).
  bool match_attention(int o, AttnMatch* m) {
    const Op* pv = def(o);
    if (!pv || pv->name != "dot_general" || pv->operands.size() != 2 || type(o).dtype != DT_BF16) return false;
    const std::vector<int64_t>& od = type(o).dims;
    if (od.size() != 4) return false;
    if (!dims_eq(pv->lhs_batch, {0, 1}) || !dims_eq(pv->rhs_batch, {0, 1}) || !dims_eq(pv->lhs_contract, {3}) ||
        !dims_eq(pv->rhs_contract, {2}))
      return false;
    const int64_t B = od[0], H = od[1], S = od[2], D = od[3];
    const int p = pv->operands[0], v = pv->operands[1];
    if (!dims_eq(type(p).dims, {B, H, S, S}) || !dims_eq(type(v).dims, {B, H, S, D}) ||
        type(p).dtype != DT_BF16 || type(v).dtype != DT_BF16)
      return false;
    const int x = softmax_src(p);
    if (x < 0) return false;
    const Op* sel = def(x);
    if (!sel || sel->name != "select" || !splat_is(sel->operands[2], -INFINITY)) return false;
    int mask = sel->operands[0];
    const int per = periodic_src(mask);
    if (per >= 0) mask = per;
    if (numel(mask) != S * S || !fold(mask)) return false;
    const std::vector<double>& mv = folded_.at(mask);
    for (int64_t i = 0; i < S; ++i)
      for (int64_t jj = 0; jj < S; ++jj)
        if ((mv[i * S + jj] != 0.0) != (i >= jj)) return false;
    int sc = sel->operands[1];
    double scale = 1.0;
    int a, b;
    if (factors(sc, &a, &b)) {
      if (splat(b, &scale)) sc = a;
      else if (splat(a, &scale)) sc = b;
      else return false;
    }
    const Op* qk = def(sc);
    if (!qk || qk->name != "dot_general" || !dims_eq(type(sc).dims, {B, H, S, S}) || type(sc).dtype != DT_BF16 ||
        !dims_eq(qk->lhs_batch, {0, 1}) || !dims_eq(qk->rhs_batch, {0, 1}) || !dims_eq(qk->lhs_contract, {3}))
      return false;
    const int q = qk->operands[0], r = qk->operands[1];
    if (!dims_eq(type(q).dims, {B, H, S, D}) || type(q).dtype != DT_BF16 || type(r).dtype != DT_BF16) return false;
    int k = -1;
    if (dims_eq(qk->rhs_contract, {3}) && dims_eq(type(r).dims, {B, H, S, D})) {
      k = r;
    } else if (dims_eq(qk->rhs_contract, {2}) && dims_eq(type(r).dims, {B, H, D, S})) {
      const Op* tr = def(r);
      if (!tr || tr->name != "transpose" || !dims_eq(tr->dims, {0, 1, 3, 2})) return false;
      k = tr->operands[0];
    } else {
      return false;
    }
    // The kernel takes a positive finite scale (its max is taken before
    // scaling); anything else runs op by op.
    if (D != 128 || S % 128 != 0 || !(scale > 0.0) || !std::isfinite(scale)) return false;
    m->q = q;
    m->k = k;
    m->v = v;
    m->B = B;
    m->H = H;
    m->S = S;
    m->D = D;
    m->scale = (float)scale;
    return true;
  }

  std::map<int, int> attn_merged_;  // attention output o -> slot of o.transpose(0, 2, 1, 3)

  int attention_merged(int o) {
    auto it = attn_merged_.find(o);
    if (it != attn_merged_.end()) return it->second;
    int r = -1;
    AttnMatch m;
    if (decoder_fusion() && match_attention(o, &m)) {
      Step st;
      st.kind = ST_ATTN;
      st.dt = MK_DT_BF16;
      st.in = {need(m.q), need(m.k), need(m.v)};
      Slot t;
      t.bytes = type(o).bytes();
      st.out = new_slot(t);
      st.B = m.B;
      st.H = m.H;
      st.S = m.S;
      st.D = m.D;
      st.scale = m.scale;
      std::ostringstream ds;
      ds << "attention_causal B=" << m.B << " H=" << m.H << " S=" << m.S << " D=" << m.D << " scale=" << m.scale
         << " bf16";
      st.desc = ds.str();
      plan_.steps.push_back(st);
      r = st.out;
    }
    attn_merged_[o] = r;
    return r;
  }

  // o [B, H, S, D] from the attention kernel's [B, S, H, D] output.
  int unmerge_heads(int o, int merged) {
    const std::vector<int64_t>& d = type(o).dims;
    const int out = temp_for(o);
    // o[b, h, s, e] = merged[b, s, h, e]
    layout_step(merged, out, 2, d, {d[1] * d[2] * d[3], d[3], d[1] * d[3], 1}, 0, row_strides(d), 0,
                "attention output to [B,H,S,D]");
    return out;
  }

  // ---- layout ops ------------------------------------------------------------
  static std::vector<int64_t> row_strides(const std::vector<int64_t>& d) {
    std::vector<int64_t> st(d.size(), 1);
    for (int i = (int)d.size() - 2; i >= 0; --i) st[i] = st[i + 1] * d[i + 1];
    return st;
  }
  static std::string dims_str(const std::vector<int64_t>& d) {
    std::string r = "[";
    for (size_t i = 0; i < d.size(); ++i) r += (i ? "," : "") + std::to_string(d[i]);
    return r + "]";
  }

  void layout_step(int src_slot, int dst_slot, int eb, const std::vector<int64_t>& shape,
                   const std::vector<int64_t>& ss, int64_t so, const std::vector<int64_t>& ds, int64_t dof,
                   const std::string& desc) {
    // The kernel cannot see buffer sizes: every element the copy touches
    // must lie inside its two slots.
    int64_t smax = so, dmax = dof;
    bool empty = false;
    for (size_t k = 0; k < shape.size(); ++k) {
      empty = empty || shape[k] == 0;
      smax += (shape[k] - 1) * ss[k];
      dmax += (shape[k] - 1) * ds[k];
    }
    if (!empty && ((smax + 1) * eb > plan_.slots[src_slot].bytes || (dmax + 1) * eb > plan_.slots[dst_slot].bytes))
      throw std::logic_error("layout step outside its buffers: " + desc);
    Step st;
    st.kind = ST_LAYOUT;
    st.in = {src_slot};
    st.out = dst_slot;
    st.elem_bytes = eb;
    st.shape = shape;
    st.src_st = ss;
    st.src_off = so;
    st.dst_st = ds;
    st.dst_off = dof;
    st.desc = desc;
    plan_.steps.push_back(st);
  }

  // transpose, slice, broadcast_in_dim, concatenate (one strided copy per
  // operand) and iota, as kernel steps.
  bool try_layout(int v, const Op& op, int* out) {
    const TensorType& t = type(v);
    const int eb = dtype_bytes(t.dtype);
    const int rank = (int)t.dims.size();
    if (eb == 0 || rank > 8) return false;
    const std::vector<int64_t> ods = row_strides(t.dims);
    const std::string ty = std::string(dtype_name(t.dtype)) + " " + dims_str(t.dims);
    if (op.name == "iota") {
      if (rank == 0 || op.dim < 0 || op.dim >= rank || !(is_int_type(t.dtype) || is_float(t.dtype))) return false;
      Step st;
      st.kind = ST_IOTA;
      st.shape = t.dims;
      st.iota_dim = (int)op.dim;
      st.type_out = t.dtype;
      st.out = temp_for(v);
      st.desc = "iota " + ty + " dim=" + std::to_string(op.dim);
      plan_.steps.push_back(st);
      *out = st.out;
      return true;
    }
    if (op.operands.empty()) return false;
    if (op.name == "concatenate") {
      if (op.dim < 0 || op.dim >= rank) return false;
      std::vector<int> srcs;
      for (int x : op.operands) {
        if (type(x).dtype != t.dtype || (int)type(x).dims.size() != rank) return false;
        srcs.push_back(need(x));
      }
      const int o = temp_for(v);
      int64_t off = 0;
      for (size_t i = 0; i < op.operands.size(); ++i) {
        const int x = op.operands[i];
        layout_step(srcs[i], o, eb, type(x).dims, row_strides(type(x).dims), 0, ods, off * ods[op.dim],
                    "concatenate part " + std::to_string(i) + " " + dtype_name(t.dtype) + " " +
                        dims_str(type(x).dims) + " -> " + dims_str(t.dims) + " dim=" + std::to_string(op.dim));
        off += type(x).dims[op.dim];
      }
      *out = o;
      return true;
    }
    const int x = op.operands[0];
    if (type(x).dtype != t.dtype) return false;
    const std::vector<int64_t>& xd = type(x).dims;
    const std::vector<int64_t> xs = row_strides(xd);
    std::vector<int64_t> ss(rank, 0);
    int64_t so = 0;
    std::string desc;
    if (op.name == "transpose") {
      if ((int)op.dims.size() != rank || (int)xd.size() != rank) return false;
      for (int i = 0; i < rank; ++i) ss[i] = xs[op.dims[i]];
      desc = "transpose " + ty + " perm=" + dims_str(op.dims);
    } else if (op.name == "slice") {
      if ((int)xd.size() != rank || (int)op.slice_start.size() != rank) return false;
      for (int i = 0; i < rank; ++i) {
        ss[i] = xs[i] * op.slice_stride[i];
        so += op.slice_start[i] * xs[i];
      }
      desc = "slice " + dims_str(xd) + " -> " + ty;
    } else if (op.name == "broadcast_in_dim") {
      if (op.dims.size() != xd.size()) return false;
      for (size_t j = 0; j < xd.size(); ++j) {
        const int64_t i = op.dims[j];
        if (i < 0 || i >= rank) return false;
        if (xd[j] == t.dims[i]) ss[i] = xs[j];
        else if (xd[j] != 1) return false;
      }
      desc = "broadcast " + dims_str(xd) + " -> " + ty;
    } else {
      return false;
    }
    const int src = need(x);
    const int o = temp_for(v);
    layout_step(src, o, eb, t.dims, ss, so, ods, 0, desc);
    *out = o;
    return true;
  }

  // A slice that is one contiguous run of its operand's elements (leading
  // dimensions of extent 1 in the result, one partial dimension, full
  // trailing ones, unit strides) of an argument or constant -- read-only
  // buffers -- is a view at a byte offset: no copy.  A scanned layer stack
  // takes each layer's weights this way.  Otherwise -1.
  int slice_view(int v, const Op& op) {
    const int x = op.operands[0];
    const std::vector<int64_t>& xd = type(x).dims;
    const size_t r = xd.size();
    if (type(x).dtype != type(v).dtype || op.slice_start.size() != r || r == 0) return -1;
    size_t k = 0;  // the partial dimension
    while (k < r && op.slice_limit[k] - op.slice_start[k] == 1) ++k;
    for (size_t i = 0; i < r; ++i) {
      if (op.slice_stride[i] != 1) return -1;
      if (i > k && (op.slice_start[i] != 0 || op.slice_limit[i] != xd[i])) return -1;
    }
    const std::vector<int64_t> xs = row_strides(xd);
    int64_t off = 0;
    for (size_t i = 0; i < r; ++i) off += op.slice_start[i] * xs[i];
    int base = need(x);
    off *= dtype_bytes(type(v).dtype);
    if (plan_.slots[base].kind == SLOT_VIEW) {
      off += plan_.slots[base].offset;
      base = plan_.slots[base].base;
    }
    if (plan_.slots[base].kind != SLOT_ARG && plan_.slots[base].kind != SLOT_CONST) return -1;
    Slot s;
    s.kind = SLOT_VIEW;
    s.bytes = type(v).bytes();
    s.base = base;
    s.offset = off;
    if (off < 0 || off + s.bytes > plan_.slots[base].bytes) return -1;
    return new_slot(s);
  }

  int dummy(int v) { return temp_for(v); }

  int const_slot(int v, const Op& op) {
    Slot s;
    s.kind = SLOT_CONST;
    const TensorType& t = type(v);
    s.bytes = t.bytes();
    const int64_t n = t.numel();
    const int eb = dtype_bytes(t.dtype);
    if (eb == 0) {
      reject(&op, "constant of type " + t.str());
      return new_slot(s);
    }
    s.data.resize((size_t)s.bytes);
    for (int64_t i = 0; i < n; ++i) {
      const double x = op.const_values.size() == 1 ? op.const_values[0]
                       : (size_t)i < op.const_values.size() ? op.const_values[i] : 0.0;
      uint8_t* p = s.data.data() + i * eb;
      switch (t.dtype) {
        case DT_F32: { float f = (float)x; memcpy(p, &f, 4); break; }
        case DT_F64: memcpy(p, &x, 8); break;
        case DT_BF16: { float f = to_bf16_value(x); uint32_t u; memcpy(&u, &f, 4); uint16_t h = (uint16_t)(u >> 16); memcpy(p, &h, 2); break; }
        case DT_PRED: case DT_S8: case DT_U8: { int8_t b = (int8_t)(int64_t)x; memcpy(p, &b, 1); break; }
        case DT_S16: case DT_U16: { int16_t b = (int16_t)(int64_t)x; memcpy(p, &b, 2); break; }
        case DT_S32: case DT_U32: { int32_t b = (int32_t)(int64_t)x; memcpy(p, &b, 4); break; }
        case DT_S64: case DT_U64: { int64_t b = (int64_t)x; memcpy(p, &b, 8); break; }
        default: reject(&op, "constant of type " + t.str());
      }
    }
    return new_slot(s);
  }

  // ---- GEMM ------------------------------------------------------------------
  static bool is_int_type(int t) { return t >= DT_S8 && t <= DT_U64; }

  struct DotShape {
    int64_t batch = 1, M = 0, N = 0, K = 0;
  };
  // Canonical [B..., M..., K] x [B..., K, N] (the reference's NN fast path,
  // ops/binary_ops.mm:1011-1019).
  bool dot_shape(const Op& op, DotShape* d) const {
    if (op.operands.size() != 2) return false;
    const TensorType& ta = type(op.operands[0]);
    const TensorType& tb = type(op.operands[1]);
    const int ra = (int)ta.dims.size(), rb = (int)tb.dims.size();
    std::vector<int64_t> lb = op.lhs_batch, rbt = op.rhs_batch, lc = op.lhs_contract, rc = op.rhs_contract;
    if (op.name == "dot") {
      if (ra < 1 || rb < 1 || rb > 2) return false;
      lc = {ra - 1};
      rc = {0};
    }
    const int nb = (int)lb.size();
    if (rbt.size() != lb.size()) return false;
    for (int i = 0; i < nb; ++i)
      if (lb[i] != i || rbt[i] != i || ta.dims[i] != tb.dims[i]) return false;
    if (lc.size() != 1 || rc.size() != 1 || lc[0] != ra - 1 || rc[0] != nb) return false;
    if (rb != nb + 2 && !(rb == nb + 1)) return false;
    if (nb > 0 && ra != nb + 2) return false;
    d->batch = 1;
    for (int i = 0; i < nb; ++i) d->batch *= ta.dims[i];
    d->K = ta.dims[ra - 1];
    if (tb.dims[nb] != d->K) return false;
    d->N = rb == nb + 2 ? tb.dims[nb + 1] : 1;
    d->M = d->batch * d->K == 0 ? 0 : ta.numel() / (d->batch * d->K);
    return true;
  }

  // Any dot_general: batch, contracting and free dimensions anywhere on
  // either side (the result is [batch..., lhs free..., rhs free...] in
  // StableHLO's order), several contracting dimensions or none (K = 1), and
  // operands that are arguments, computed values or transposes of them. Each
  // group of dimensions collapses into one index with one stride when the
  // strides allow it (always, for row-major operands whose groups are
  // adjacent and in order); an operand whose groups do not collapse is
  // copied to [batch, M, K] / [batch, K, N] first (copy_a / copy_b).
  struct GeneralDot {
    int a = -1, b = -1;  // source values (a folded transpose's input)
    int64_t batch = 1, M = 1, N = 1, K = 0;
    int64_t sa[3] = {0, 0, 0}, sb[3] = {0, 0, 0};
    bool transposed = false;
    bool copy_a = false, copy_b = false;
    // copy_*: the operand's dims in [batch, free, contract] (a) or
    // [batch, contract, free] (b) order and their strides in the source.
    std::vector<int64_t> a_shape, a_st, b_shape, b_st;
  };

  bool general_dot(const Op& op, GeneralDot* g) const {
    if (op.operands.size() != 2) return false;
    std::vector<int64_t> lb = op.lhs_batch, rbt = op.rhs_batch, lc = op.lhs_contract, rc = op.rhs_contract;
    const int ra = (int)type(op.operands[0]).dims.size(), rb = (int)type(op.operands[1]).dims.size();
    if (op.name == "dot") {
      if (ra < 1 || rb < 1 || rb > 2) return false;
      lc = {ra - 1};
      rc = {0};
    }
    if (lc.size() != rc.size() || lb.size() != rbt.size()) return false;
    // Every dim named at most once per side, and in range.
    auto distinct = [](const std::vector<int64_t>& x, const std::vector<int64_t>& y, int r) {
      std::vector<bool> seen(r, false);
      for (const auto* v : {&x, &y})
        for (int64_t i : *v) {
          if (i < 0 || i >= r || seen[i]) return false;
          seen[i] = true;
        }
      return true;
    };
    if (!distinct(lb, lc, ra) || !distinct(rbt, rc, rb)) return false;
    // Operand dims -> (source value, stride of each operand dim in the source).
    auto layout = [&](int x, int* src, std::vector<int64_t>* st, bool* tr) {
      const Op* d = def(x);
      std::vector<int64_t> perm;
      *src = x;
      if (d && d->name == "transpose" && !d->operands.empty()) {
        *src = d->operands[0];
        perm = d->dims;
      }
      const std::vector<int64_t>& sd = type(*src).dims;
      std::vector<int64_t> rs(sd.size(), 1);
      for (int i = (int)sd.size() - 2; i >= 0; --i) rs[i] = rs[i + 1] * sd[i + 1];
      const size_t r = type(x).dims.size();
      st->assign(r, 0);
      if (perm.empty()) {
        if (sd.size() != r) return false;
        for (size_t i = 0; i < r; ++i) (*st)[i] = rs[i];
        return true;
      }
      if (perm.size() != r || sd.size() != r) return false;
      for (size_t i = 0; i < r; ++i) {
        if (perm[i] < 0 || perm[i] >= (int64_t)r) return false;
        (*st)[i] = rs[perm[i]];
        if (perm[i] != (int64_t)i) *tr = true;
      }
      return true;
    };
    std::vector<int64_t> as, bs;
    if (!layout(op.operands[0], &g->a, &as, &g->transposed) || !layout(op.operands[1], &g->b, &bs, &g->transposed))
      return false;
    const std::vector<int64_t>& ad = type(op.operands[0]).dims;
    const std::vector<int64_t>& bd = type(op.operands[1]).dims;
    // Collapse a list of dims (in order) into one index with one stride.
    auto collapse = [](const std::vector<int64_t>& dims, const std::vector<int64_t>& st,
                       const std::vector<int>& idx, int64_t* size, int64_t* stride) {
      *size = 1;
      *stride = 0;
      std::vector<int> keep;
      for (int i : idx)
        if (dims[i] != 1) keep.push_back(i);
      for (int i : idx) *size *= dims[i];
      if (keep.empty()) return true;
      *stride = st[keep.back()];
      for (size_t j = 0; j + 1 < keep.size(); ++j)
        if (st[keep[j]] != st[keep[j + 1]] * dims[keep[j + 1]]) return false;
      return true;
    };
    std::vector<int> a_batch, b_batch, a_con, b_con, a_free, b_free;
    for (size_t i = 0; i < lb.size(); ++i) {
      if (ad[lb[i]] != bd[rbt[i]]) return false;
      a_batch.push_back((int)lb[i]);
      b_batch.push_back((int)rbt[i]);
    }
    for (size_t i = 0; i < lc.size(); ++i) {
      if (ad[lc[i]] != bd[rc[i]]) return false;
      a_con.push_back((int)lc[i]);
      b_con.push_back((int)rc[i]);
    }
    auto named = [](const std::vector<int64_t>& x, int i) { return std::find(x.begin(), x.end(), i) != x.end(); };
    for (int i = 0; i < ra; ++i)
      if (!named(lb, i) && !named(lc, i)) a_free.push_back(i);
    for (int i = 0; i < rb; ++i)
      if (!named(rbt, i) && !named(rc, i)) b_free.push_back(i);
    int64_t bsz, kb, n_, m_;
    // lhs: batch, free (M), contract (K)
    bool ok_a = collapse(ad, as, a_batch, &g->batch, &g->sa[0]) && collapse(ad, as, a_free, &g->M, &g->sa[1]) &&
                collapse(ad, as, a_con, &g->K, &g->sa[2]);
    bool ok_b = collapse(bd, bs, b_batch, &bsz, &g->sb[0]) && collapse(bd, bs, b_con, &kb, &g->sb[1]) &&
                collapse(bd, bs, b_free, &g->N, &g->sb[2]);
    if (!ok_a) {
      // sizes of the groups, then the canonical copy's row-major strides
      collapse(ad, std::vector<int64_t>(ra, 0), a_batch, &g->batch, &bsz);
      collapse(ad, std::vector<int64_t>(ra, 0), a_free, &g->M, &m_);
      collapse(ad, std::vector<int64_t>(ra, 0), a_con, &g->K, &kb);
      g->copy_a = true;
      for (const auto* grp : {&a_batch, &a_free, &a_con})
        for (int i : *grp) {
          g->a_shape.push_back(ad[i]);
          g->a_st.push_back(as[i]);
        }
      g->sa[0] = g->M * g->K;
      g->sa[1] = g->K;
      g->sa[2] = 1;
    }
    if (!ok_b) {
      collapse(bd, std::vector<int64_t>(rb, 0), b_free, &g->N, &n_);
      g->copy_b = true;
      for (const auto* grp : {&b_batch, &b_con, &b_free})
        for (int i : *grp) {
          g->b_shape.push_back(bd[i]);
          g->b_st.push_back(bs[i]);
        }
      g->sb[0] = g->K * g->N;
      g->sb[1] = g->N;
      g->sb[2] = 1;
    }
    if ((g->copy_a && g->a_shape.size() > 8) || (g->copy_b && g->b_shape.size() > 8)) return false;
    if (g->copy_a || g->copy_b) g->transposed = true;
    return true;
  }

  // The slot holding dot operand `which` (0: lhs, 1: rhs) in the layout
  // general_dot's strides describe: the source value itself, or its copy in
  // canonical order when the operand's dimension groups do not collapse.
  int dot_operand(const GeneralDot& gd, int which, int eb) {
    const bool copy = which == 0 ? gd.copy_a : gd.copy_b;
    const int src = which == 0 ? gd.a : gd.b;
    const int slot = need(src);
    if (!copy) return slot;
    const std::vector<int64_t>& shape = which == 0 ? gd.a_shape : gd.b_shape;
    const std::vector<int64_t>& st = which == 0 ? gd.a_st : gd.b_st;
    int64_t n = 1;
    for (int64_t d : shape) n *= d;
    const int o = new_slot(Slot{SLOT_TEMP, n * eb, -1, {}});
    layout_step(slot, o, eb, shape, st, 0, row_strides(shape), 0,
                std::string("dot operand ") + (which == 0 ? "a" : "b") + " to " + dims_str(shape));
    return o;
  }

  bool try_gemm(int v, const Op& op, int* out) {
    DotShape d;
    GeneralDot gd;
    const bool general = general_dot(op, &gd);
    const int ta = type(op.operands[0]).dtype, tb = type(op.operands[1]).dtype, tr = type(v).dtype;
    const bool fast_types = (ta == DT_F32 && tb == DT_F32 && tr == DT_F32) ||
                            (ta == DT_BF16 && tb == DT_BF16 && (tr == DT_BF16 || tr == DT_F32));
    if (general && gd.K == 0) {
      Step z;
      z.kind = ST_ZERO;
      z.bytes = type(v).bytes();
      z.out = temp_for(v);
      z.desc = "zero " + type(v).str() + " (empty contraction)";
      plan_.steps.push_back(z);
      *out = z.out;
      return true;
    }
    const bool fast = !(general && gd.transposed) && dot_shape(op, &d) && fast_types && d.K > 0 &&
                      d.K % 8 == 0 && d.N % 8 == 0 && numel(v) == d.batch * d.M * d.N;
    if (!fast && general && fast_types && gd.K > 0 && gd.K % 8 == 0 && gd.N % 8 == 0 &&
        numel(v) == gd.batch * gd.M * gd.N && gd.M * gd.N * gd.K >= (int64_t(1) << 18)) {
      // Operands in another layout (a transposed operand, e.g. q @ k^T written
      // as einsum 'bhtd,bhsd->bhts') are copied to [batch, M, K] and
      // [batch, K, N] first, then multiplied by the tiled GEMM.
      const int eb = dtype_bytes(ta);
      auto canon = [&](int which, const int64_t* st, int64_t R, int64_t C, const char* what) {
        const int slot = dot_operand(gd, which, eb);
        if (st[2] == 1 && st[1] == C && (gd.batch == 1 || st[0] == R * C)) return slot;
        const std::vector<int64_t> shape = {gd.batch, R, C};
        const int o = new_slot(Slot{SLOT_TEMP, gd.batch * R * C * eb, -1, {}});
        layout_step(slot, o, eb, shape, {st[0], st[1], st[2]}, 0, row_strides(shape), 0,
                    std::string("gemm operand ") + what + " to " + dims_str(shape));
        return o;
      };
      Step st;
      // An rhs that already is B^T [batch, N, K] (its contracting dimension
      // last: x @ W.T, q @ k^T) on shapes the 256 x 256 kernel takes goes to
      // the GEMM that reads B^T as it lies: no copy, the same bits
      // (MK_PLAN_GEMM_NT=0 copies it instead).
      const char* pnt = getenv("MK_PLAN_GEMM_NT");
      st.b_t = ta == DT_BF16 && tr == DT_BF16 && !gd.copy_b && gd.sb[1] == 1 && gd.sb[2] == gd.K &&
               (gd.batch == 1 || gd.sb[0] == gd.N * gd.K) && gd.M % 256 == 0 && gd.N % 256 == 0 &&
               gd.K % 32 == 0 && !(pnt && pnt[0] == '0');
      st.in = {canon(0, gd.sa, gd.M, gd.K, "a"),
               st.b_t ? dot_operand(gd, 1, eb) : canon(1, gd.sb, gd.K, gd.N, "b")};
      if (ta == DT_F32) {
        st.kind = ST_GEMM_F32;
        st.dt = MK_DT_F32;
      } else {
        st.kind = ST_GEMM_BF16;
        st.dt = MK_DT_BF16;
        st.out_f32 = tr == DT_F32;
      }
      st.batch = gd.batch;
      st.M = gd.M;
      st.N = gd.N;
      st.K = gd.K;
      st.out = temp_for(v);
      std::ostringstream ds;
      ds << (st.kind == ST_GEMM_F32 ? "gemm_f32" : st.b_t ? "gemm_bf16_nt" : "gemm_bf16") << " batch=" << gd.batch
         << " M=" << gd.M << " N=" << gd.N << " K=" << gd.K << " -> " << dtype_name(tr);
      st.desc = ds.str();
      plan_.steps.push_back(st);
      *out = st.out;
      return true;
    }
    if (!fast) {
      if (!general) {
        reject(&op, "dimension numbers whose operand layouts cannot be mapped (rank above 8 or mismatched sizes)");
        return false;
      }
      const bool ints = is_int_type(ta) && is_int_type(tr);
      const bool floats = (ta == DT_F32 || ta == DT_BF16 || ta == DT_F16) && (tr == ta || tr == DT_F32);
      if (ta != tb || !(ints || floats) || numel(v) != gd.batch * gd.M * gd.N) {
        reject(&op, std::string("operand types ") + dtype_name(ta) + " x " + dtype_name(tb) + " -> " + dtype_name(tr));
        return false;
      }
      Step st;
      st.kind = ST_DOT_GENERIC;
      st.type_a = ta;
      st.type_out = tr;
      st.in = {dot_operand(gd, 0, dtype_bytes(ta)), dot_operand(gd, 1, dtype_bytes(ta))};
      st.batch = gd.batch;
      st.M = gd.M;
      st.N = gd.N;
      st.K = gd.K;
      for (int i = 0; i < 3; ++i) {
        st.sa[i] = gd.sa[i];
        st.sb[i] = gd.sb[i];
      }
      st.out = temp_for(v);
      std::ostringstream ds;
      ds << "dot_general " << dtype_name(ta) << " batch=" << gd.batch << " M=" << gd.M << " N=" << gd.N
         << " K=" << gd.K << (gd.transposed ? " (strided)" : "") << " -> " << dtype_name(tr);
      st.desc = ds.str();
      plan_.steps.push_back(st);
      *out = st.out;
      return true;
    }
    Step st;
    if (ta == DT_F32) {
      st.kind = ST_GEMM_F32;
      st.dt = MK_DT_F32;
    } else {
      st.kind = ST_GEMM_BF16;
      st.dt = MK_DT_BF16;
      st.out_f32 = tr == DT_F32;
    }
    st.in = {need(op.operands[0]), need(op.operands[1])};
    st.batch = d.batch;
    st.M = d.M;
    st.N = d.N;
    st.K = d.K;
    st.out = temp_for(v);
    std::ostringstream ds;
    ds << (st.kind == ST_GEMM_F32 ? "gemm_f32" : "gemm_bf16") << " batch=" << d.batch << " M=" << d.M << " N=" << d.N
       << " K=" << d.K << " -> " << dtype_name(tr);
    st.desc = ds.str();
    plan_.steps.push_back(st);
    *out = st.out;
    return true;
  }

  // ---- dequant-matmul ----------------------------------------------------------
  // Recognises X @ dequant(W) where the weight is built in jnp as
  //   int4 g64: (interleave(P & 15, P >> 4).astype(f) - repeat(z, 64)) * repeat(s, 64)
  //   int8 per-channel: W.astype(f) * s[None, :]
  // (any order of the commutative operands, converts anywhere), followed by
  // a bf16 result.  The packing and group layout are the quantized formats
  // of mk_kernels.h.

  static int64_t prod(const std::vector<int64_t>& d, size_t a, size_t b) {
    int64_t p = 1;
    for (size_t i = a; i < b; ++i) p *= d[i];
    return p;
  }

  // v [K, N] == src[k / g, n] (jnp.repeat(src, g, axis=0), which lowers to
  // expand_dims / tile / reshape chains); returns src or -1.
  int rep_rows(int v, int64_t K, int64_t N, int64_t g) const {
    if (numel(v) != K * N || K / g <= 1 || N <= 1 || g <= 1) return -1;
    const int u = peel_cvt(v);
    const Op* b = def(u);
    if (!b || b->name != "broadcast_in_dim" || !monotonic(b->dims) || numel(u) != K * N) return -1;
    const int s = b->operands[0];
    const std::vector<int64_t>& R = type(u).dims;
    const std::vector<int64_t>& S = type(s).dims;
    if (numel(s) * g != K * N || S.size() != b->dims.size()) return -1;
    std::vector<char> bc(R.size(), 1);
    for (size_t i = 0; i < S.size(); ++i) {
      if (S[i] == R[b->dims[i]]) bc[b->dims[i]] = 0;
      else if (S[i] != 1) return -1;
    }
    int first = -1, last = -1;
    for (size_t j = 0; j < R.size(); ++j)
      if (bc[j] && R[j] > 1) {
        if (first < 0) first = (int)j;
        last = (int)j;
      }
    if (first < 0) return -1;
    for (int j = first; j <= last; ++j)
      if (!bc[j] && R[j] != 1) return -1;
    if (prod(R, 0, first) != K / g || prod(R, first, last + 1) != g || prod(R, last + 1, R.size()) != N) return -1;
    return peel_cvt(s);
  }

  // v [K, N] == nibble (k % 2) of P[k / 2, n], low nibble first
  // (jnp.stack([P & 15, P >> 4], axis=1).reshape(K, N)); returns P or -1.
  int interleave_src(int v, int64_t K, int64_t N) const {
    if (numel(v) != K * N) return -1;
    const int u = peel_cvt(v);
    const Op* c = def(u);
    if (!c || c->name != "concatenate" || c->operands.size() != 2 || numel(u) != K * N) return -1;
    const std::vector<int64_t>& R = type(u).dims;
    if (c->dim < 0 || c->dim >= (int64_t)R.size() || R[c->dim] != 2) return -1;
    if (prod(R, 0, c->dim) != K / 2 || prod(R, c->dim + 1, R.size()) != N) return -1;
    const int lo = peel_cvt(c->operands[0]), hi = peel_cvt(c->operands[1]);
    const int p_lo = nibble_src(lo, false), p_hi = nibble_src(hi, true);
    if (p_lo < 0 || p_lo != p_hi) return -1;
    if (type(p_lo).dtype != DT_U8 || numel(p_lo) != (K / 2) * N) return -1;
    return p_lo;
  }
  int nibble_src(int v, bool high) const {
    v = peel_view(v);
    const Op* op = def(v);
    if (!op || op->operands.size() != 2) return -1;
    int a = op->operands[0], b = op->operands[1];
    if (op->name == "and") {
      if (!splat_is(b, 15) && splat_is(a, 15)) std::swap(a, b);
      if (!splat_is(b, 15)) return -1;
      if (!high) return peel_view(a);
      return shr4_src(a);
    }
    if (high) return shr4_src(v);
    return -1;
  }
  int shr4_src(int v) const {
    v = peel_view(v);
    const Op* op = def(v);
    if (!op || op->name != "shift_right_logical" || op->operands.size() != 2 || !splat_is(op->operands[1], 4))
      return -1;
    return peel_view(op->operands[0]);
  }

  struct QmmMatch {
    int fmt = -1;              // MK_QFMT_INT4_G64 / MK_QFMT_INT8_PC
    int x = -1, w = -1, s = -1, z = -1;  // z: int4 only
    int64_t M = 0, K = 0, N = 0;
  };
  bool match_qmm(int v, QmmMatch* q) const {
    const Op* top = def(v);
    if (!top) return false;
    int dv = v;
    if (top->name == "convert") {
      dv = top->operands[0];
      if (type(v).dtype != DT_BF16 || !is(dv, "dot_general")) return false;
    } else if (type(v).dtype != DT_BF16) {
      return false;
    }
    const Op* dot = def(dv);
    if (!dot || dot->name != "dot_general") return false;
    DotShape d;
    if (!dot_shape(*dot, &d) || d.batch != 1 || type(dot->operands[1]).dims.size() != 2) return false;
    const int x = peel_cvt(dot->operands[0]);
    if (type(x).dtype != DT_BF16 || numel(x) != d.M * d.K || numel(v) != d.M * d.N) return false;
    const int w = peel_cvt(dot->operands[1]);
    const Op* mul = def(w);
    if (!mul || mul->name != "multiply") return false;
    const int64_t K = d.K, N = d.N, M = d.M;
    q->x = x;
    q->M = M;
    q->K = K;
    q->N = N;
    for (int order = 0; order < 2; ++order) {
      const int f0 = mul->operands[order], f1 = mul->operands[1 - order];
      // int4: f0 = (q - z), f1 = repeat(s)
      const int sub = peel_cvt(f0);
      if (K % 64 == 0 && is(sub, "subtract")) {
        const int s = rep_rows(f1, K, N, 64);
        const int z = rep_rows(def(sub)->operands[1], K, N, 64);
        const int p = interleave_src(def(sub)->operands[0], K, N);
        if (s >= 0 && z >= 0 && p >= 0 && type(s).dtype == DT_BF16 && type(z).dtype == DT_U8) {
          q->fmt = MK_QFMT_INT4_G64;
          q->w = p;
          q->s = s;
          q->z = z;
          return true;
        }
      }
      // int8: f0 = W, f1 = s[None, :]
      const int wq = peel_cvt(f0);
      if (type(wq).dtype == DT_S8 && type(wq).dims == std::vector<int64_t>{K, N}) {
        const int sc = col_src(f1, N);
        if (sc < 0) continue;
        const int s = peel_cvt(sc);
        if (type(s).dtype != DT_F32 || numel(s) != N) continue;
        q->fmt = MK_QFMT_INT8_PC;
        q->w = wq;
        q->s = s;
        return true;
      }
    }
    return false;
  }

  // Emits the dequant-matmul q for value v, with a store epilogue against
  // aux (a bf16 value of v's size) unless epi is MK_EPI_NONE.
  bool emit_qmm(int v, const QmmMatch& q, int epi, int aux, int* out) {
    const int64_t ws = mk_qmatmul_workspace_bytes(q.fmt, q.M, q.K, q.N);
    if (ws < 0) return false;
    Step st;
    st.kind = q.fmt == MK_QFMT_INT4_G64 ? ST_QMM_INT4 : ST_QMM_INT8;
    st.dt = MK_DT_BF16;
    st.in = {need(q.x), need(q.w), need(q.s)};
    if (q.fmt == MK_QFMT_INT4_G64) st.in.push_back(need(q.z));
    st.epi = epi;
    if (epi != MK_EPI_NONE) st.in.push_back(need(aux));
    st.M = q.M;
    st.K = q.K;
    st.N = q.N;
    st.out = temp_for(v);
    plan_.workspace_bytes = std::max(plan_.workspace_bytes, ws);
    static const char* epi_name[] = {"", " + add epilogue", " + swiglu epilogue", " + swiglu pairs"};
    st.desc = std::string(q.fmt == MK_QFMT_INT4_G64 ? "int4_g64_matmul" : "int8_pc_matmul") +
              " M=" + std::to_string(q.M) + " K=" + std::to_string(q.K) + " N=" + std::to_string(q.N) + " -> bf16" +
              epi_name[epi];
    plan_.steps.push_back(st);
    *out = st.out;
    return true;
  }

  bool try_qmm(int v, int* out) {
    QmmMatch q;
    return match_qmm(v, &q) && emit_qmm(v, q, MK_EPI_NONE, -1, out);
  }

  // Operand references of each value (ops and returns), counted once.
  std::vector<int> uses_;
  int uses(int v) {
    if (uses_.empty()) {
      uses_.assign(f_.values.size(), 0);
      for (const Op& op : f_.ops)
        for (int o : op.operands) ++uses_[o];
      for (int r : f_.rets) ++uses_[r];
    }
    return uses_[v];
  }

  // bf16 `aux + qmm(...)` and `silu(g) * qmm(...)` (silu written g *
  // logistic(g)) where nothing else reads the product: the dequant-matmul
  // with its store epilogue (MK_EPI_ADD / MK_EPI_SWIGLU), which rounds where
  // the elementwise program would, so the result is bit-identical.
  // Residual adds are folded by default. The SwiGLU epilogue reads the gate
  // operand in the product's store, which on the dequantise-then-GEMM route
  // costs more than the separate program (the decoder layer measured 1.268
  // vs 1.255 ms per call with and without it), so it is folded only with
  // MK_PLAN_EPILOGUES=all; MK_PLAN_EPILOGUES=0 folds nothing.
  // silu(x @ Wg) * (x @ Wu) with both products dequant-matmuls of one x, one
  // format and one shape, read by nothing else, on the many-row route: one
  // paired step (both weights dequantised into an interleaved buffer, one
  // GEMM with the SwiGLU store), bit-identical to the two products and the
  // SwiGLU program.  MK_PLAN_PAIRS=0 (or MK_PLAN_EPILOGUES=0) keeps them
  // apart.
  bool try_qmm_pair(int v, int* out) {
    const char* env = getenv("MK_PLAN_EPILOGUES");
    const char* pe = getenv("MK_PLAN_PAIRS");
    if ((env && env[0] == '0') || (pe && pe[0] == '0')) return false;
    const Op* op = def(v);
    if (op->name != "multiply" || type(v).dtype != DT_BF16 || op->operands.size() != 2) return false;
    for (int order = 0; order < 2; ++order) {
      const int up = op->operands[order], act = op->operands[1 - order];
      int a, b;
      if (uses(up) != 1 || uses(act) != 1 || !factors(act, &a, &b)) continue;
      int g = -1;
      if (is(b, "logistic") && def(b)->operands[0] == a) g = a;
      else if (is(a, "logistic") && def(a)->operands[0] == b) g = b;
      if (g < 0 || uses(g) != 2 || uses(g == a ? b : a) != 1) continue;
      QmmMatch qg, qu;
      if (!match_qmm(g, &qg) || !match_qmm(up, &qu)) continue;
      if (qg.x != qu.x || qg.fmt != qu.fmt || qg.M != qu.M || qg.K != qu.K || qg.N != qu.N) continue;
      if (type(g).dims != type(v).dims || type(up).dims != type(v).dims) continue;
      const int64_t ws = mk_qmatmul_swiglu_pair_workspace_bytes(qg.fmt, qg.M, qg.K, qg.N);
      if (ws < 0) continue;
      Step st;
      st.kind = qg.fmt == MK_QFMT_INT4_G64 ? ST_QMM_PAIR_INT4 : ST_QMM_PAIR_INT8;
      st.dt = MK_DT_BF16;
      if (qg.fmt == MK_QFMT_INT4_G64)
        st.in = {need(qg.x), need(qg.w), need(qg.s), need(qg.z), need(qu.w), need(qu.s), need(qu.z)};
      else
        st.in = {need(qg.x), need(qg.w), need(qg.s), need(qu.w), need(qu.s)};
      st.M = qg.M;
      st.K = qg.K;
      st.N = qg.N;
      st.out = temp_for(v);
      plan_.workspace_bytes = std::max(plan_.workspace_bytes, ws);
      st.desc = std::string(qg.fmt == MK_QFMT_INT4_G64 ? "int4_g64" : "int8_pc") + " swiglu pair matmul M=" +
                std::to_string(qg.M) + " K=" + std::to_string(qg.K) + " N=" + std::to_string(qg.N) + " -> bf16";
      plan_.steps.push_back(st);
      *out = st.out;
      return true;
    }
    return false;
  }

  bool try_qmm_epilogue(int v, int* out) {
    const char* env = getenv("MK_PLAN_EPILOGUES");
    if (env && env[0] == '0') return false;
    if (!(env && strcmp(env, "all") == 0) && def(v)->name != "add") return false;
    const Op* op = def(v);
    if (type(v).dtype != DT_BF16 || op->operands.size() != 2) return false;
    for (int order = 0; order < 2; ++order) {
      const int acc = op->operands[order], other = op->operands[1 - order];
      if (uses(acc) != 1 || type(acc).dims != type(v).dims || type(other).dims != type(v).dims ||
          type(other).dtype != DT_BF16)
        continue;
      QmmMatch q;
      if (!match_qmm(acc, &q)) continue;
      int epi = MK_EPI_ADD, aux = other;
      if (op->name == "multiply") {
        int a, b;
        if (!factors(other, &a, &b)) continue;
        if (is(b, "logistic") && def(b)->operands[0] == a) aux = a;
        else if (is(a, "logistic") && def(a)->operands[0] == b) aux = b;
        else continue;
        epi = MK_EPI_SWIGLU;
      } else if (op->name != "add") {
        return false;
      }
      if (!mk_qmatmul_epilogue_supported(q.fmt, q.M, q.K, q.N, epi)) continue;
      return emit_qmm(v, q, epi, aux, out);
    }
    return false;
  }

  // ---- row patterns ----------------------------------------------------------------
  // jax.nn.softmax: the input x of v = exp(x - max(x)) / sum(exp(x - max(x)))
  // over the last axis (bf16 sums may be upcast to f32 and back, jnp.sum), or -1.
  int softmax_src(int v) const {
    const Op* div = def(v);
    const int dt = type(v).dtype;
    if (!div || div->name != "divide" || mk_dt(dt) < 0 || div->operands.size() != 2) return -1;
    const int64_t C = last_dim(v);
    const int e = div->operands[0];
    int s = row_src(div->operands[1], C);
    if (s < 0) return -1;
    s = peel_cvt(s);
    const int ein = reduce_last_input(s, "add");
    if (ein < 0 || peel_cvt(ein) != peel_view(e)) return -1;
    const int ev = peel_view(e);
    if (!is(ev, "exponential") || type(ev).dtype != dt) return -1;
    const int dsub = peel_view(def(ev)->operands[0]);
    if (!is(dsub, "subtract")) return -1;
    const int x = peel_view(def(dsub)->operands[0]);
    int m = row_src(def(dsub)->operands[1], C);
    if (m < 0) return -1;
    m = peel_view(m);
    if (is(m, "maximum")) {  // jnp.max(..., initial=-inf)
      const Op* mx = def(m);
      if (splat_is(mx->operands[1], -INFINITY)) m = peel_view(mx->operands[0]);
      else if (splat_is(mx->operands[0], -INFINITY)) m = peel_view(mx->operands[1]);
      else return -1;
    }
    const int xm = reduce_last_input(m, "maximum");
    if (xm < 0 || peel_view(xm) != x || type(x).dtype != dt || numel(x) != numel(v)) return -1;
    return x;
  }

  bool try_softmax(int v, int* out) {
    const int dt = type(v).dtype;
    const int64_t C = last_dim(v);
    const int x = softmax_src(v);
    if (x < 0) return false;
    Step st;
    st.kind = ST_SOFTMAX;
    st.dt = mk_dt(dt);
    st.in = {need(x)};
    st.cols = C;
    st.rows = numel(v) / C;
    st.out = temp_for(v);
    st.desc = "softmax rows=" + std::to_string(st.rows) + " cols=" + std::to_string(C) + " " + dtype_name(dt);
    plan_.steps.push_back(st);
    *out = st.out;
    return true;
  }

  // x * rsqrt(mean(x*x, -1, keepdims) + eps) * g, any association of the
  // three factors.
  bool try_rmsnorm(int v, int* out) {
    const int dt = type(v).dtype;
    if (mk_dt(dt) < 0) return false;
    const int64_t C = last_dim(v);
    std::vector<int> fac;
    std::function<void(int, int)> flat = [&](int u, int depth) {
      u = peel_view(u);
      if (depth < 2 && is(u, "multiply") && type(u).dtype == dt && numel(u) == numel(v)) {
        flat(def(u)->operands[0], depth + 1);
        flat(def(u)->operands[1], depth + 1);
      } else {
        fac.push_back(u);
      }
    };
    flat(def(v)->operands[0], 1);
    flat(def(v)->operands[1], 1);
    if (fac.size() != 3) return false;
    int x = -1, g = -1, r = -1;
    for (int u : fac) {
      int t;
      if (g < 0 && (t = col_src(u, C)) >= 0 && numel(peel_view(t)) == C && numel(u) != C) {
        g = peel_view(t);
        continue;
      }
      if (r < 0 && (t = row_src(u, C)) >= 0 && numel(u) != numel(t)) {
        r = t;
        continue;
      }
      if (x < 0 && numel(u) == numel(v)) {
        x = u;
        continue;
      }
      return false;
    }
    if (x < 0 || g < 0 || r < 0 || type(x).dtype != dt || type(g).dtype != dt) return false;
    // r = rsqrt(ms + eps)
    int rs = peel_cvt(r);
    if (!is(rs, "rsqrt")) return false;
    int add = peel_cvt(def(rs)->operands[0]);
    if (!is(add, "add")) return false;
    double eps;
    int ms;
    if (splat(def(add)->operands[1], &eps)) ms = def(add)->operands[0];
    else if (splat(def(add)->operands[0], &eps)) ms = def(add)->operands[1];
    else return false;
    ms = peel_cvt(ms);
    // ms = sum / C or sum * (1/C)
    int sum;
    double c;
    const Op* mo = def(ms);
    if (!mo || mo->operands.size() != 2) return false;
    if (mo->name == "divide" && splat(mo->operands[1], &c) && c == (double)C) sum = mo->operands[0];
    else if (mo->name == "multiply" && splat(mo->operands[1], &c) && fabs(c * C - 1.0) < 1e-6) sum = mo->operands[0];
    else if (mo->name == "multiply" && splat(mo->operands[0], &c) && fabs(c * C - 1.0) < 1e-6) sum = mo->operands[1];
    else return false;
    const int sq_in = reduce_last_input(peel_view(sum), "add");
    if (sq_in < 0) return false;
    const int sq = peel_cvt(sq_in);
    if (!is(sq, "multiply")) return false;
    const int xv = peel_cvt(x);
    if (peel_cvt(def(sq)->operands[0]) != xv || peel_cvt(def(sq)->operands[1]) != xv) return false;
    Step st;
    st.kind = ST_RMSNORM;
    st.dt = mk_dt(dt);
    st.in = {need(x), need(g)};
    st.cols = C;
    st.rows = numel(v) / C;
    st.eps = (float)eps;
    st.out = temp_for(v);
    std::ostringstream ds;
    ds << "rmsnorm rows=" << st.rows << " cols=" << C << " eps=" << eps << " " << dtype_name(dt);
    st.desc = ds.str();
    plan_.steps.push_back(st);
    *out = st.out;
    return true;
  }

  // jnp.argmax: a two-operand reduce over (x, iota) along the last axis.
  bool try_argmax(int v, const Op& op, int* out) {
    if (op.operands.size() != 4 || op.reduce_body != "argmax" || op.results.size() != 2) return false;
    if (v != op.results[1]) {
      reject(&op, "value result of an argmax reduce");
      return false;
    }
    const int x = op.operands[0], idx = op.operands[1];
    const int rank = (int)type(x).dims.size();
    const int dt = type(x).dtype;
    const int id = peel_view(idx);
    if (mk_dt(dt) < 0 || rank == 0 || op.dims.size() != 1 || op.dims[0] != rank - 1) return false;
    if (!is(id, "iota") || def(id)->dim != rank - 1 || type(id).dims != type(x).dims) return false;
    if (type(v).dtype != DT_S32 || numel(v) * last_dim(x) != numel(x)) return false;
    double i0, x0;
    if (!splat(op.operands[3], &i0) || i0 != 0.0) return false;
    if (!splat(op.operands[2], &x0) || !(x0 == -INFINITY)) return false;
    Step st;
    st.kind = ST_ARGMAX;
    st.dt = mk_dt(dt);
    st.in = {need(x)};
    st.cols = last_dim(x);
    st.rows = numel(x) / st.cols;
    st.out = temp_for(v);
    st.desc = "argmax rows=" + std::to_string(st.rows) + " cols=" + std::to_string(st.cols) + " " + dtype_name(dt) +
              " -> i32";
    plan_.steps.push_back(st);
    *out = st.out;
    return true;
  }

  // Last-axis sum/max; bf16 sums written as convert(reduce_f32(convert(x)))
  // map to the bf16 kernel (f32 accumulation, one rounding).
  bool try_reduce(int v, int* out) {
    int r = v, x;
    int dt = type(v).dtype;
    if (is(v, "convert")) {
      r = def(v)->operands[0];
      if (!is(r, "reduce") || dt != DT_BF16 || type(r).dtype != DT_F32) return false;
    }
    int op = 0;
    int64_t cols = 0;
    double init = 0.0;
    bool neutral = true;
    if (!reduce_trailing(r, &x, &op, &cols, &init, &neutral)) return false;
    static const char* const kBody[] = {"sum", "max", "min"};
    if (r != v) {
      // bf16 sum accumulated in f32 (jnp.sum of bf16): convert -> reduce -> convert.
      x = peel_cvt(x);
      if (type(x).dtype != DT_BF16 || op != MK_REDUCE_SUM || !neutral) return false;
    }
    if (mk_dt(dt) < 0 || type(x).dtype != dt || cols <= 0 || numel(v) * cols != numel(x)) return false;
    Step st;
    st.kind = ST_REDUCE;
    st.dt = mk_dt(dt);
    st.reduce_op = op;
    st.in = {need(x)};
    st.cols = cols;
    st.rows = numel(x) / cols;
    st.out = temp_for(v);
    st.desc = std::string("reduce_") + kBody[op] + " rows=" + std::to_string(st.rows) + " cols=" +
              std::to_string(st.cols) + " " + dtype_name(dt);
    plan_.steps.push_back(st);
    if (!neutral) {
      // lax.reduce with a non-neutral init: the init joins the reduction
      // once (mps_executable.mm:955-975), as an elementwise step on the
      // reduced rows.
      Step e;
      e.kind = ST_EW;
      e.dt = mk_dt(dt);
      e.in = {st.out};
      e.in_numel = {st.rows};
      const int32_t ew_op = op == MK_REDUCE_SUM ? MK_EW_ADD : op == MK_REDUCE_MAX ? MK_EW_MAX : MK_EW_MIN;
      e.prog = {mk_ew_instr{MK_EW_LOAD, 0, 0, 0, 0, 0.f}, mk_ew_instr{MK_EW_CONST, 1, 0, 0, 0, (float)init},
                mk_ew_instr{ew_op, 2, 0, 1, 0, 0.f}};
      e.prog_out = 2;
      e.n = st.rows;
      e.out = temp_for(v);
      e.desc = "elementwise 3 instr, 1 inputs, n=" + std::to_string(st.rows) + " " + dtype_name(dt) +
               " (reduce init)";
      plan_.steps.push_back(e);
      *out = e.out;
      return true;
    }
    *out = st.out;
    return true;
  }

  // ---- elementwise programs ------------------------------------------------------------
  bool is_elementwise(int v) const {
    const Op* op = def(v);
    if (!op) return false;
    if (op->name == "select" || op->name == "clamp") return true;
    if (op->name == "broadcast_in_dim") return !op->operands.empty() && numel(op->operands[0]) == 1;
    if (op->name == "constant") return op->const_splat;
    return unary_ops().count(op->name) || binary_ops().count(op->name);
  }

  struct EwCtx {
    int dt;        // DT_F32 or DT_BF16 (program dtype)
    int64_t n;     // element count
    std::vector<mk_ew_instr> prog;
    std::map<int, int> reg;  // value -> virtual register (instruction index)
    std::vector<int> loads;  // value ids of inputs
    std::vector<int> load_slot;  // the input's slot when it is a folded constant, else -1
    std::vector<int64_t> load_numel;
    std::set<int> force;     // values to load instead of inlining
    std::string fail;        // reason the value cannot be expressed
    int split_hint = -1;     // largest inlined subexpression (split candidate)
    int split_size = 0;
  };

  // Unused operand fields are 0 (the kernel ignores them).
  int ew_emit(EwCtx& c, int op, int a = 0, int b = 0, int cc = 0, float imm = 0.f) {
    mk_ew_instr in{};
    in.op = op;
    in.dst = (int)c.prog.size();
    in.a = a;
    in.b = b;
    in.c = cc;
    in.imm = imm;
    c.prog.push_back(in);
    return in.dst;
  }

  int ew_load(EwCtx& c, int u) {
    // A broadcast that only adds leading dimensions repeats its operand:
    // load the operand periodically instead of materialising it.
    const int p = periodic_src(u);
    if (p >= 0 && numel(p) > 1) u = p;
    const int64_t ne = numel(u);
    if (ne != c.n && ne != 1 && (ne <= 0 || c.n % ne != 0)) {
      c.fail = "broadcast of a non-scalar " + type(u).str() + " into an elementwise op";
      return -1;
    }
    int slot = -1;
    int elem = MK_EW_IN_DEFAULT;
    const int ut = type(u).dtype;
    if (ut != c.dt && (ut == DT_F32 || ut == DT_BF16)) {
      elem = ut == DT_F32 ? MK_EW_IN_F32 : MK_EW_IN_BF16;  // the other float type, widened exactly
    } else if (ut != c.dt) {
      // Index-only values (iota / constant masks) are evaluated here and
      // loaded as constants of the program's type.
      slot = fold_const_slot(u, c.dt);
      if (slot < 0) {
        c.fail = std::string("elementwise input of type ") + dtype_name(ut) + " in a " + dtype_name(c.dt) +
                 " program";
        return -1;
      }
    }
    for (size_t i = 0; i < c.loads.size(); ++i)
      if (c.loads[i] == u && c.load_slot[i] == slot) return ew_emit(c, MK_EW_LOAD, (int)i, elem);
    c.loads.push_back(u);
    c.load_slot.push_back(slot);
    c.load_numel.push_back(ne);
    return ew_emit(c, MK_EW_LOAD, (int)c.loads.size() - 1, elem);
  }

  // v = broadcast_in_dim(x) whose elements repeat x's in order: x's
  // dimensions larger than 1 map, with equal sizes, onto a trailing block of
  // v's.  Returns x or -1.
  int periodic_src(int v) const {
    const Op* op = def(v);
    if (!op || op->name != "broadcast_in_dim" || op->operands.empty() || !monotonic(op->dims)) return -1;
    const int x = op->operands[0];
    const std::vector<int64_t>& xd = type(x).dims;
    const std::vector<int64_t>& vd = type(v).dims;
    if (op->dims.size() != xd.size() || type(x).dtype != type(v).dtype) return -1;
    int first = (int)vd.size();
    for (size_t j = 0; j < xd.size(); ++j)
      if (xd[j] != 1) {
        first = (int)op->dims[j];
        break;
      }
    for (int i = first; i < (int)vd.size(); ++i) {
      int j = -1;
      for (size_t k = 0; k < op->dims.size(); ++k)
        if (op->dims[k] == i) j = (int)k;
      if (j < 0 || xd[j] != vd[i]) return -1;
    }
    return x;
  }

  // ---- compile-time folding of index values ------------------------------------
  // Values computed only from iota and constants -- masks such as the causal
  // lower triangle, jnp.arange(T)[:, None] >= jnp.arange(T)[None, :] -- are
  // evaluated on the host (row-major, as doubles) up to kFoldMax elements.
  static constexpr int64_t kFoldMax = int64_t(1) << 24;
  std::map<int, std::vector<double>> folded_;
  std::map<std::pair<int, int>, int> folded_slot_;

  std::set<int> unfoldable_;

  bool fold(int v, int depth = 0) {
    if (folded_.count(v)) return true;
    if (unfoldable_.count(v)) return false;
    const bool ok = fold_uncached(v, depth);
    if (!ok) unfoldable_.insert(v);
    return ok;
  }

  bool fold_uncached(int v, int depth) {
    if (depth > 64 || numel(v) > kFoldMax) return false;
    const Op* op = def(v);
    if (!op) return false;
    static const std::set<std::string> foldable = {"constant", "iota", "reshape", "convert", "broadcast_in_dim",
                                                   "transpose", "compare", "select", "and", "or", "not", "add",
                                                   "subtract", "multiply", "maximum", "minimum", "negate"};
    if (!foldable.count(op->name)) return false;
    const TensorType& t = type(v);
    const int64_t n = numel(v);
    const std::vector<int64_t>& d = t.dims;
    for (int o : op->operands)
      if (!fold(o, depth + 1)) return false;
    std::vector<double> out((size_t)n);
    auto in = [&](int k) -> const std::vector<double>& { return folded_.at(op->operands[k]); };
    const std::string& nm = op->name;
    const int dt = t.dtype;
    auto cast = [&](double x) {
      if (dt == DT_PRED) return x != 0 ? 1.0 : 0.0;
      if (is_int_type(dt)) return ::trunc(x);
      return round_to(x, dt);
    };
    if (nm == "constant") {
      if (op->const_values.empty()) return false;
      for (int64_t i = 0; i < n; ++i)
        out[i] = cast(op->const_values.size() == 1 ? op->const_values[0]
                      : (size_t)i < op->const_values.size() ? op->const_values[i] : 0.0);
    } else if (nm == "iota") {
      if (op->dim < 0 || op->dim >= (int64_t)d.size()) return false;
      int64_t inner = 1;
      for (size_t k = op->dim + 1; k < d.size(); ++k) inner *= d[k];
      for (int64_t i = 0; i < n; ++i) out[i] = cast((double)((i / inner) % d[op->dim]));
    } else if (nm == "reshape" || nm == "convert") {
      const std::vector<double>& a = in(0);
      if ((int64_t)a.size() != n) return false;
      for (int64_t i = 0; i < n; ++i) out[i] = cast(a[i]);
    } else if (nm == "broadcast_in_dim" || nm == "transpose") {
      const std::vector<double>& a = in(0);
      const std::vector<int64_t>& xd = type(op->operands[0]).dims;
      const std::vector<int64_t> xs = row_strides(xd);
      std::vector<int64_t> st(d.size(), 0);
      if (nm == "transpose") {
        if (op->dims.size() != d.size()) return false;
        for (size_t i = 0; i < d.size(); ++i) st[i] = xs[op->dims[i]];
      } else {
        if (op->dims.size() != xd.size()) return false;
        for (size_t j = 0; j < xd.size(); ++j)
          if (xd[j] != 1) st[op->dims[j]] = xs[j];
      }
      for (int64_t i = 0; i < n; ++i) {
        int64_t r = i, src = 0;
        for (int k = (int)d.size() - 1; k >= 0; --k) {
          src += (r % d[k]) * st[k];
          r /= d[k];
        }
        out[i] = a[src];
      }
    } else if (nm == "compare") {
      const std::vector<double>&a = in(0), &b = in(1);
      const std::string& c = op->compare_dir;
      for (int64_t i = 0; i < n; ++i) {
        const double x = a[i], y = b[i];
        out[i] = (c == "EQ" ? x == y : c == "NE" ? x != y : c == "LT" ? x < y : c == "LE" ? x <= y
                  : c == "GT" ? x > y : x >= y) ? 1.0 : 0.0;
      }
      if (c != "EQ" && c != "NE" && c != "LT" && c != "LE" && c != "GT" && c != "GE") return false;
    } else if (nm == "select") {
      const std::vector<double>&p = in(0), &a = in(1), &b = in(2);
      for (int64_t i = 0; i < n; ++i) out[i] = p[i] != 0 ? a[i] : b[i];
    } else if ((nm == "and" || nm == "or") && dt == DT_PRED) {
      const std::vector<double>&a = in(0), &b = in(1);
      for (int64_t i = 0; i < n; ++i) out[i] = nm == "and" ? (a[i] != 0 && b[i] != 0) : (a[i] != 0 || b[i] != 0);
    } else if (nm == "not" && dt == DT_PRED) {
      const std::vector<double>& a = in(0);
      for (int64_t i = 0; i < n; ++i) out[i] = a[i] != 0 ? 0.0 : 1.0;
    } else if ((nm == "add" || nm == "subtract" || nm == "multiply" || nm == "maximum" || nm == "minimum") &&
               is_int_type(dt)) {
      const std::vector<double>&a = in(0), &b = in(1);
      for (int64_t i = 0; i < n; ++i)
        out[i] = nm == "add" ? a[i] + b[i] : nm == "subtract" ? a[i] - b[i] : nm == "multiply" ? a[i] * b[i]
                 : nm == "maximum" ? std::max(a[i], b[i]) : std::min(a[i], b[i]);
    } else if (nm == "negate" && is_int_type(dt)) {
      const std::vector<double>& a = in(0);
      for (int64_t i = 0; i < n; ++i) out[i] = -a[i];
    } else {
      return false;
    }
    folded_[v] = std::move(out);
    return true;
  }

  // The folded values of v as a constant slot of type dt (F32 or BF16), or -1.
  int fold_const_slot(int v, int dt) {
    const auto key = std::make_pair(v, dt);
    auto it = folded_slot_.find(key);
    if (it != folded_slot_.end()) return it->second;
    if (!(type(v).dtype == DT_PRED || is_int_type(type(v).dtype)) || !fold(v)) return -1;
    const std::vector<double>& a = folded_.at(v);
    Slot s;
    s.kind = SLOT_CONST;
    const int eb = dt == DT_F32 ? 4 : 2;
    s.bytes = (int64_t)a.size() * eb;
    s.data.resize((size_t)s.bytes);
    for (size_t i = 0; i < a.size(); ++i) {
      if (dt == DT_F32) {
        const float f = (float)a[i];
        memcpy(s.data.data() + 4 * i, &f, 4);
      } else {
        const float f = to_bf16_value(a[i]);
        uint32_t u;
        memcpy(&u, &f, 4);
        const uint16_t h = (uint16_t)(u >> 16);
        memcpy(s.data.data() + 2 * i, &h, 2);
      }
    }
    const int slot = new_slot(s);
    folded_slot_[key] = slot;
    return slot;
  }

  // Returns the virtual register holding u; `size` accumulates the number
  // of instructions generated for u's subtree.
  int ew_value(EwCtx& c, int u, bool root, int* size) {
    auto it = c.reg.find(u);
    if (it != c.reg.end()) return it->second;
    const int before = (int)c.prog.size();
    int r = ew_value_uncached(c, u, root);
    if (r < 0) return -1;
    const int sz = (int)c.prog.size() - before;
    *size += sz;
    if (!root && sz > c.split_size && is_elementwise(u) && numel(u) == c.n &&
        (type(u).dtype == DT_F32 || type(u).dtype == DT_BF16) && !c.force.count(u)) {
      c.split_size = sz;
      c.split_hint = u;
    }
    c.reg[u] = r;
    return r;
  }

  int ew_value_uncached(EwCtx& c, int u, bool root) {
    double k;
    const TensorType& t = type(u);
    if (splat(u, &k) && is_float(t.dtype)) return ew_emit(c, MK_EW_CONST, 0, 0, 0, (float)k);
    if (splat(u, &k) && t.dtype == DT_PRED) return ew_emit(c, MK_EW_CONST, 0, 0, 0, k != 0 ? 1.f : 0.f);
    const int vs = view_src(u);
    if (vs >= 0 && !c.force.count(u)) {
      int dummy = 0;
      return ew_value(c, vs, false, &dummy);
    }
    const Op* op = def(u);
    if (op && !root && (t.dtype == DT_PRED || is_int_type(t.dtype)) && numel(u) <= kFoldMax && fold(u))
      return ew_load(c, u);  // an index-only mask: a folded constant
    if (!op || (!root && c.force.count(u)) || !is_elementwise(u)) return ew_load(c, u);
    // A convert of a product or reduction is that kernel's output type (the
    // GEMM, dequant-matmul and reduce kernels write bf16 themselves): load it
    // rather than pull the f32 value into this program.
    if (!root && op->name == "convert" && (is(peel_view(op->operands[0]), "dot_general") ||
                                          is(peel_view(op->operands[0]), "dot") ||
                                          is(peel_view(op->operands[0]), "reduce")))
      return ew_load(c, u);
    if (op->name == "broadcast_in_dim") return ew_load(c, op->operands[0]);  // scalar broadcast
    // Per-node type rules: f32 programs round bf16-typed nodes explicitly
    // (MK_EW_ROUND_BF16); bf16 programs mark f32-typed arithmetic
    // MK_EW_KEEP_F32 so that it is neither rounded nor shortened.
    const int dt = t.dtype;
    if (dt != DT_PRED && dt != DT_F32 && dt != DT_BF16) {
      c.fail = std::string("elementwise ") + op->name + " on " + dtype_name(dt);
      return -1;
    }
    std::vector<int> r;
    int sz = 0;
    for (int o : op->operands) {
      if (op->name == "compare" && type(o).dtype != DT_F32 && type(o).dtype != DT_BF16) {
        c.fail = std::string("compare on ") + dtype_name(type(o).dtype);
        return -1;
      }
      const int x = ew_value(c, o, false, &sz);
      if (x < 0) return -1;
      r.push_back(x);
    }
    const size_t first_new = c.prog.size();  // this node's own instructions start here
    int res = -1;
    const std::string& n = op->name;
    static const std::map<std::string, int> un = {
        {"negate", MK_EW_NEG}, {"abs", MK_EW_ABS}, {"exponential", MK_EW_EXP}, {"log", MK_EW_LOG},
        {"log_plus_one", MK_EW_LOG1P}, {"exponential_minus_one", MK_EW_EXPM1}, {"tanh", MK_EW_TANH},
        {"rsqrt", MK_EW_RSQRT}, {"sqrt", MK_EW_SQRT}, {"logistic", MK_EW_LOGISTIC}, {"floor", MK_EW_FLOOR},
        {"ceil", MK_EW_CEIL}};
    static const std::map<std::string, int> bin = {
        {"add", MK_EW_ADD}, {"subtract", MK_EW_SUB}, {"multiply", MK_EW_MUL}, {"divide", MK_EW_DIV},
        {"maximum", MK_EW_MAX}, {"minimum", MK_EW_MIN}, {"power", MK_EW_POW}};
    static const std::map<std::string, int> cmp = {{"EQ", MK_EW_CMP_EQ}, {"NE", MK_EW_CMP_NE},
                                                    {"LT", MK_EW_CMP_LT}, {"LE", MK_EW_CMP_LE},
                                                    {"GT", MK_EW_CMP_GT}, {"GE", MK_EW_CMP_GE}};
    if (un.count(n)) {
      if (dt == DT_PRED) {
        c.fail = n + " on a predicate";
        return -1;
      }
      res = ew_emit(c, un.at(n), r[0]);
    } else if (bin.count(n)) {
      if (dt == DT_PRED) {
        c.fail = n + " on a predicate";
        return -1;
      }
      res = ew_emit(c, bin.at(n), r[0], r[1]);
    } else if (n == "compare") {
      if (!cmp.count(op->compare_dir)) {
        c.fail = "compare direction '" + op->compare_dir + "'";
        return -1;
      }
      res = ew_emit(c, cmp.at(op->compare_dir), r[0], r[1]);
    } else if (n == "select") {
      res = ew_emit(c, MK_EW_SELECT, r[0], r[1], r[2]);
    } else if (n == "clamp") {  // clamp(lo, x, hi)
      const int m = ew_emit(c, MK_EW_MAX, r[1], r[0]);
      res = ew_emit(c, MK_EW_MIN, m, r[2]);
    } else if (n == "and" || n == "or") {
      if (dt != DT_PRED) {
        c.fail = n + " on " + dtype_name(dt);
        return -1;
      }
      res = ew_emit(c, n == "and" ? MK_EW_MUL : MK_EW_MAX, r[0], r[1]);
    } else if (n == "not") {
      if (dt != DT_PRED) {
        c.fail = "not on " + std::string(dtype_name(dt));
        return -1;
      }
      const int one = ew_emit(c, MK_EW_CONST, 0, 0, 0, 1.f);
      res = ew_emit(c, MK_EW_SUB, one, r[0]);
    } else if (n == "convert") {
      const int st = type(op->operands[0]).dtype;
      if (dt == DT_PRED) {
        if (!is_float(st)) {
          c.fail = std::string("convert ") + dtype_name(st) + " -> i1";
          return -1;
        }
        const int z = ew_emit(c, MK_EW_CONST, 0, 0, 0, 0.f);
        res = ew_emit(c, MK_EW_CMP_NE, r[0], z);
      } else if (st == DT_PRED || st == DT_F32 || st == DT_BF16) {
        // Widening (bf16 / i1 -> f32) is exact; f32 -> bf16 rounds.
        res = r[0];
        if (dt == DT_BF16 && st == DT_F32) res = ew_emit(c, MK_EW_ROUND_BF16, r[0]);
        return res;
      } else {
        c.fail = std::string("convert ") + dtype_name(st) + " -> " + dtype_name(dt);
        return -1;
      }
    } else {
      c.fail = "elementwise " + n;
      return -1;
    }
    // bf16-typed results inside an f32 program round like XLA's bf16 ops.
    if (c.dt == DT_F32 && dt == DT_BF16) res = ew_emit(c, MK_EW_ROUND_BF16, res);
    if (c.dt == DT_BF16 && dt == DT_F32)
      for (size_t i = first_new; i < c.prog.size(); ++i)
        if (c.prog[i].op >= MK_EW_ADD && c.prog[i].op <= MK_EW_CEIL) c.prog[i].op |= MK_EW_KEEP_F32;
    return res;
  }

  // Number of register operands an instruction reads.
  static int n_src(int op) {
    op &= ~MK_EW_KEEP_F32;
    if (op == MK_EW_LOAD || op == MK_EW_CONST) return 0;
    if (op == MK_EW_SELECT) return 3;
    if ((op >= MK_EW_ADD && op <= MK_EW_POW) || (op >= MK_EW_CMP_EQ && op <= MK_EW_CMP_GE)) return 2;
    return 1;
  }

  // Virtual registers -> the kernel's 12 slots (linear scan; a register is
  // freed after its last read).  Returns false when more than 12 are live.
  static bool assign_slots(std::vector<mk_ew_instr>& prog, int root, int* out_slot) {
    const int n = (int)prog.size();
    std::vector<int> last(n, -1);
    for (int i = 0; i < n; ++i) {
      const mk_ew_instr& in = prog[i];
      const int src[3] = {in.a, in.b, in.c};
      for (int k = 0; k < n_src(in.op); ++k) last[src[k]] = i;
    }
    last[root] = n;
    std::vector<int> phys(n, -1);
    std::vector<int> owner(12, -1);
    for (int i = 0; i < n; ++i) {
      mk_ew_instr& in = prog[i];
      const int ns = n_src(in.op);
      int src[3] = {in.a, in.b, in.c};
      int mapped[3] = {0, 0, 0};
      for (int k = 0; k < ns; ++k) mapped[k] = phys[src[k]];
      for (int k = 0; k < ns; ++k)
        if (last[src[k]] == i) owner[phys[src[k]]] = -1;
      int p = -1;
      for (int k = 0; k < 12 && p < 0; ++k)
        if (owner[k] < 0) p = k;
      if (p < 0) return false;
      owner[p] = i;
      phys[i] = p;
      if (last[i] < 0) owner[p] = -1;  // dead result
      in.dst = p;
      if (ns > 0) {
        in.a = mapped[0];
        in.b = mapped[1];
        in.c = mapped[2];
      }
    }
    *out_slot = phys[root];
    return true;
  }

  int ew_root(int v) {
    const int dt = type(v).dtype;
    if (dt != DT_F32 && dt != DT_BF16) {
      reject(def(v), std::string("elementwise result of type ") + dtype_name(dt));
      return dummy(v);
    }
    std::set<int> force;
    for (int attempt = 0; attempt < 24; ++attempt) {
      EwCtx c;
      c.dt = dt;
      c.n = numel(v);
      c.force = force;
      int sz = 0;
      const int r = ew_value(c, v, true, &sz);
      if (r < 0) {
        reject(def(v), c.fail);
        return dummy(v);
      }
      std::vector<mk_ew_instr> prog = c.prog;
      int out_slot = 0;
      const bool fits = c.loads.size() <= 4 && prog.size() <= 32 && assign_slots(prog, r, &out_slot);
      if (!fits) {
        if (c.split_hint < 0) {
          reject(def(v), "elementwise program does not fit the kernel's limits");
          return dummy(v);
        }
        force.insert(c.split_hint);
        continue;
      }
      Step st;
      st.kind = ST_EW;
      st.dt = mk_dt(dt);
      for (size_t i = 0; i < c.loads.size(); ++i) st.in.push_back(c.load_slot[i] >= 0 ? c.load_slot[i] : need(c.loads[i]));
      st.in_numel = c.load_numel;
      st.prog = prog;
      st.prog_out = out_slot;
      st.n = c.n;
      st.out = temp_for(v);
      st.desc = "elementwise " + std::to_string(prog.size()) + " instr, " + std::to_string(c.loads.size()) +
                " inputs, n=" + std::to_string(c.n) + " " + dtype_name(dt);
      plan_.steps.push_back(st);
      return st.out;
    }
    reject(def(v), "elementwise program does not fit the kernel's limits");
    return dummy(v);
  }
};

}  // namespace

std::string Plan::describe() const {
  std::string s;
  for (const Step& st : steps) s += st.desc + "\n";
  return s;
}

Plan build_plan(const Function& fn) { return Planner(fn).run(); }

}  // namespace mkrt
