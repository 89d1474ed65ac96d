// Reader for the StableHLO text that jax prints (lowered.as_text()): a
// module of func.func definitions whose bodies hold one op per line, reduce
// ops optionally followed by a body region.  Covers the pretty and the
// generic ("stablehlo.op"(...) {attrs}) forms of the hot-path ops; anything
// else is kept by name so the planner can reject it with a list, as the
// reference rejects unsupported ops at compile (core/stablehlo_parser.mm:521-537).
#include <ctype.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <map>
#include <set>

#include "shlo.h"

namespace mkrt {

int dtype_bytes(int dt) {
  switch (dt) {
    case DT_PRED: case DT_S8: case DT_U8: return 1;
    case DT_S16: case DT_U16: case DT_F16: case DT_BF16: return 2;
    case DT_S32: case DT_U32: case DT_F32: return 4;
    case DT_S64: case DT_U64: case DT_F64: return 8;
    default: return 0;
  }
}

const char* dtype_name(int dt) {
  switch (dt) {
    case DT_PRED: return "i1";
    case DT_S8: return "i8";
    case DT_S16: return "i16";
    case DT_S32: return "i32";
    case DT_S64: return "i64";
    case DT_U8: return "ui8";
    case DT_U16: return "ui16";
    case DT_U32: return "ui32";
    case DT_U64: return "ui64";
    case DT_F16: return "f16";
    case DT_F32: return "f32";
    case DT_F64: return "f64";
    case DT_BF16: return "bf16";
    default: return "?";
  }
}

int64_t TensorType::numel() const {
  int64_t n = 1;
  for (int64_t d : dims) n *= d;
  return n;
}

std::string TensorType::str() const {
  std::string s = "tensor<";
  for (int64_t d : dims) s += std::to_string(d) + "x";
  return s + dtype_name(dtype) + ">";
}

namespace {

int parse_elem(const std::string& t) {
  static const std::map<std::string, int> m = {
      {"i1", DT_PRED}, {"i8", DT_S8}, {"i16", DT_S16}, {"i32", DT_S32}, {"i64", DT_S64},
      {"ui8", DT_U8}, {"ui16", DT_U16}, {"ui32", DT_U32}, {"ui64", DT_U64},
      {"f16", DT_F16}, {"f32", DT_F32}, {"f64", DT_F64}, {"bf16", DT_BF16}};
  auto it = m.find(t);
  if (it == m.end()) throw ParseError("unsupported element type '" + t + "'");
  return it->second;
}

std::string trim(const std::string& s) {
  size_t a = 0, b = s.size();
  while (a < b && isspace((unsigned char)s[a])) ++a;
  while (b > a && isspace((unsigned char)s[b - 1])) --b;
  return s.substr(a, b - a);
}

bool starts_with(const std::string& s, const char* p) { return s.compare(0, strlen(p), p) == 0; }

// Parses "tensor<AxBxT>" starting at pos (skipping spaces); advances pos.
TensorType parse_type_at(const std::string& s, size_t& pos) {
  while (pos < s.size() && isspace((unsigned char)s[pos])) ++pos;
  if (s.compare(pos, 7, "tensor<") != 0)
    throw ParseError("expected tensor type at '" + s.substr(pos, 40) + "'");
  pos += 7;
  const size_t end = s.find('>', pos);
  if (end == std::string::npos) throw ParseError("unterminated tensor type");
  std::string body = s.substr(pos, end - pos);
  pos = end + 1;
  TensorType t;
  size_t p = 0;
  while (true) {
    const size_t x = body.find('x', p);
    if (x == std::string::npos || !isdigit((unsigned char)body[p])) break;
    t.dims.push_back(strtoll(body.c_str() + p, nullptr, 10));
    p = x + 1;
  }
  t.dtype = parse_elem(body.substr(p));
  return t;
}

// Every tensor type in a string, in order.
std::vector<TensorType> all_types(const std::string& s) {
  std::vector<TensorType> v;
  size_t pos = 0;
  while ((pos = s.find("tensor<", pos)) != std::string::npos) v.push_back(parse_type_at(s, pos));
  return v;
}

// Index of the last " : " at bracket depth 0 (separates an op from its types).
size_t type_colon(const std::string& s) {
  int depth = 0;
  size_t last = std::string::npos;
  for (size_t i = 0; i < s.size(); ++i) {
    const char c = s[i];
    if (c == '(' || c == '[' || c == '{' || c == '<') ++depth;
    else if (c == ')' || c == ']' || c == '}' || (c == '>' && !(i > 0 && s[i - 1] == '-'))) --depth;
    else if (c == ':' && depth == 0 && i > 0 && s[i - 1] == ' ' && i + 1 < s.size() && s[i + 1] == ' ')
      last = i;
  }
  return last;
}

std::vector<std::string> value_names(const std::string& s) {
  std::vector<std::string> v;
  for (size_t i = 0; i < s.size(); ++i) {
    if (s[i] != '%') continue;
    size_t j = i + 1;
    while (j < s.size() && (isalnum((unsigned char)s[j]) || s[j] == '_' || s[j] == '#' || s[j] == '.')) ++j;
    v.push_back(s.substr(i, j - i));
    i = j - 1;
  }
  return v;
}

std::vector<int64_t> int_list(const std::string& s) {
  std::vector<int64_t> v;
  const char* p = s.c_str();
  while (*p) {
    if (isdigit((unsigned char)*p) || (*p == '-' && isdigit((unsigned char)p[1]))) {
      char* e;
      v.push_back(strtoll(p, &e, 10));
      p = e;
    } else {
      ++p;
    }
  }
  return v;
}

// The [..] list following `key` (e.g. "dims = [0, 1]"), or empty.
// The integer list following `key`: "[0, 1]" (pretty form), "array<i64: 0, 1>"
// (generic form) or "dense<[0, 1]>" (older printers).
bool list_after(const std::string& s, const std::string& key, std::vector<int64_t>* out, size_t* after = nullptr) {
  size_t k = s.find(key);
  if (k == std::string::npos) return false;
  size_t a = k + key.size();
  while (a < s.size() && isspace((unsigned char)s[a])) ++a;
  size_t b;
  if (s.compare(a, 6, "array<") == 0) {
    b = s.find('>', a);
    if (b == std::string::npos) return false;
    const size_t colon = s.find(':', a);
    *out = colon != std::string::npos && colon < b ? int_list(s.substr(colon + 1, b - colon - 1))
                                                   : std::vector<int64_t>();
  } else if (s.compare(a, 6, "dense<") == 0) {
    b = s.find('>', a);
    if (b == std::string::npos) return false;
    *out = int_list(s.substr(a + 6, b - a - 6));
  } else {
    a = s.find('[', a);
    b = s.find(']', a);
    if (a == std::string::npos || b == std::string::npos) return false;
    *out = int_list(s.substr(a + 1, b - a - 1));
  }
  if (after) *after = b + 1;
  return true;
}

// Payload of dense<...>: a splat number / hex bit pattern / bool, or a
// (nested) list of numbers, or a quoted hex blob.
void parse_dense(const std::string& s, int dtype, Op* op) {
  size_t a = s.find("dense<");
  if (a == std::string::npos) throw ParseError("constant without dense<> payload: " + s);
  a += 6;
  int depth = 1;
  size_t b = a;
  while (b < s.size() && depth > 0) {
    if (s[b] == '<') ++depth;
    if (s[b] == '>') --depth;
    ++b;
  }
  std::string body = trim(s.substr(a, b - 1 - a));
  auto from_bits = [&](uint64_t bits) -> double {
    switch (dtype) {
      case DT_F32: { float f; uint32_t u = (uint32_t)bits; memcpy(&f, &u, 4); return f; }
      case DT_BF16: { float f; uint32_t u = (uint32_t)bits << 16; memcpy(&f, &u, 4); return f; }
      case DT_F64: { double d; memcpy(&d, &bits, 8); return d; }
      case DT_F16: {
        const uint32_t h = (uint32_t)bits, sgn = (h >> 15) & 1, e = (h >> 10) & 31, m = h & 1023;
        double v = e == 0 ? ldexp((double)m, -24) : e == 31 ? (m ? NAN : INFINITY) : ldexp(1024.0 + m, (int)e - 25);
        return sgn ? -v : v;
      }
      default: return (double)(int64_t)bits;
    }
  };
  if (!body.empty() && body[0] == '"') {
    // "0x..." raw little-endian bytes of the whole tensor.
    std::string hex = body.substr(3, body.size() - 4);
    const int eb = dtype_bytes(dtype);
    std::vector<uint8_t> bytes(hex.size() / 2);
    for (size_t i = 0; i < bytes.size(); ++i) bytes[i] = (uint8_t)strtol(hex.substr(2 * i, 2).c_str(), nullptr, 16);
    for (size_t i = 0; i + eb <= bytes.size(); i += eb) {
      uint64_t bits = 0;
      memcpy(&bits, &bytes[i], eb);
      op->const_values.push_back(from_bits(bits));
    }
    op->const_splat = op->const_values.size() == 1;
    return;
  }
  std::vector<double> vals;
  const char* p = body.c_str();
  while (*p) {
    if (*p == 't' && strncmp(p, "true", 4) == 0) { vals.push_back(1.0); p += 4; continue; }
    if (*p == 'f' && strncmp(p, "false", 5) == 0) { vals.push_back(0.0); p += 5; continue; }
    if (p[0] == '0' && p[1] == 'x') {
      char* e;
      const uint64_t bits = strtoull(p + 2, &e, 16);
      vals.push_back(from_bits(bits));
      p = e;
      continue;
    }
    if (isdigit((unsigned char)*p) || *p == '-' || *p == '+' || *p == '.') {
      char* e;
      const double v = strtod(p, &e);
      if (e != p) {
        vals.push_back(v);
        p = e;
        continue;
      }
    }
    if (strncmp(p, "inf", 3) == 0) { vals.push_back(INFINITY); p += 3; continue; }
    if (strncmp(p, "nan", 3) == 0) { vals.push_back(NAN); p += 3; continue; }
    ++p;
  }
  if (vals.empty()) throw ParseError("cannot read constant payload: " + body);
  op->const_values = vals;
  op->const_splat = vals.size() == 1;
}

// Joins raw body lines into statements: an op line that opens a region
// (by '{' balance) continues until the region closes, and a line starting a
// pretty-form region of the previous op ("reducer", "cond", "do") is
// appended to that op.
std::vector<std::string> join_statements(const std::vector<std::string>& raw) {
  std::vector<std::string> out;
  std::string pending;
  int pdepth = 0;
  for (const std::string& l : raw) {
    const std::string s = trim(l);
    int d = 0;
    for (char c : s) d += (c == '{') - (c == '}');
    if (!pending.empty() || (d > 0 && !s.empty())) {
      if (pending.empty() && !out.empty() &&
          (starts_with(s, "reducer") || starts_with(s, "cond") || starts_with(s, "do ") || starts_with(s, "do{"))) {
        pending = out.back();
        out.pop_back();
      }
      pending += (pending.empty() ? "" : "\n") + s;
      pdepth += d;
      if (pdepth <= 0) {
        out.push_back(pending);
        pending.clear();
        pdepth = 0;
      }
      continue;
    }
    if (!s.empty()) out.push_back(s);
  }
  if (!pending.empty()) out.push_back(pending);  // unbalanced: the op parser reports it
  return out;
}

struct RawFunc {
  std::string name;
  bool is_public = false;
  std::vector<std::pair<std::string, TensorType>> args;
  std::vector<std::string> lines;  // body statements (regions joined)
};

// Splits the module text into functions and their body statements.
std::vector<RawFunc> split_functions(const std::string& text) {
  std::vector<RawFunc> fns;
  std::vector<std::string> lines;
  size_t p = 0;
  while (p <= text.size()) {
    size_t e = text.find('\n', p);
    if (e == std::string::npos) e = text.size();
    lines.push_back(text.substr(p, e - p));
    p = e + 1;
  }
  for (size_t i = 0; i < lines.size(); ++i) {
    std::string l = trim(lines[i]);
    if (!starts_with(l, "func.func")) continue;
    RawFunc f;
    f.is_public = l.find(" private ") == std::string::npos;
    size_t at = l.find('@');
    size_t lp = l.find('(', at);
    f.name = l.substr(at + 1, lp - at - 1);
    // Arguments: "%argN: tensor<...> {attrs}" up to the matching ')'.
    int depth = 0;
    size_t rp = lp;
    for (; rp < l.size(); ++rp) {
      if (l[rp] == '(' || l[rp] == '<' || l[rp] == '{' || l[rp] == '[') ++depth;
      if (l[rp] == ')' || l[rp] == '>' || l[rp] == '}' || l[rp] == ']') --depth;
      if (depth == 0) break;
    }
    const std::string argtext = l.substr(lp + 1, rp - lp - 1);
    size_t q = 0;
    while ((q = argtext.find('%', q)) != std::string::npos) {
      size_t c = argtext.find(':', q);
      const std::string nm = trim(argtext.substr(q, c - q));
      size_t tp = c + 1;
      TensorType t = parse_type_at(argtext, tp);
      f.args.push_back({nm, t});
      q = tp;
    }
    // Body: lines until the function's closing brace (depth tracking).
    int bd = 0;
    for (char c : l) bd += (c == '{') - (c == '}');
    std::vector<std::string> raw;
    for (++i; i < lines.size() && bd > 0; ++i) {
      const std::string s = trim(lines[i]);
      int d = 0;
      for (char c : s) d += (c == '{') - (c == '}');
      if (bd + d <= 0) {
        bd += d;
        break;
      }
      bd += d;
      raw.push_back(s);
    }
    f.lines = join_statements(raw);
    --i;
    fns.push_back(f);
  }
  return fns;
}

std::string strip_dialect(std::string n) {
  for (const char* pfx : {"stablehlo.", "chlo.", "mhlo.", "func.", "\"stablehlo.", "\"chlo.", "\"func."}) {
    if (starts_with(n, pfx)) {
      n = n.substr(strlen(pfx));
      break;
    }
  }
  if (!n.empty() && n.back() == '"') n.pop_back();
  return n;
}

// Classifies a reduce body region (lines between the braces).
std::string classify_reduce_body(const std::string& body, int nresults) {
  if (nresults == 1) {
    for (const char* op : {"add", "maximum", "minimum", "multiply", "and", "or"}) {
      const std::string key = std::string("stablehlo.") + op;
      if (body.find(key + " ") != std::string::npos || body.find(key + "\"") != std::string::npos) return op;
    }
    return "unknown";
  }
  if (nresults == 2) {
    // jnp.argmax / argmin comparators: the value comparison decides.
    if (body.find("compare  GT") != std::string::npos || body.find("compare GT") != std::string::npos ||
        body.find("comparison_direction = #stablehlo<comparison_direction GT>") != std::string::npos)
      return "argmax";
    if (body.find("compare  LT") != std::string::npos || body.find("compare LT") != std::string::npos ||
        body.find("comparison_direction = #stablehlo<comparison_direction LT>") != std::string::npos)
      return "argmin";
  }
  return "unknown";
}

struct Builder {
  Function fn;
  std::map<std::string, int> names;  // SSA name -> value id (current scope)

  int new_value(const TensorType& t, const std::string& name) {
    Value v;
    v.type = t;
    v.name = name;
    fn.values.push_back(v);
    return (int)fn.values.size() - 1;
  }
  int lookup(const std::string& n) const {
    auto it = names.find(n);
    if (it == names.end()) throw ParseError("use of undefined value " + n);
    return it->second;
  }
};


// Structural checks of one parsed op of the plugin's set, so that later
// passes may index its operands, results and dimension attributes: operand
// counts by op kind, one typed result, and every dimension number inside the
// rank it refers to.  A malformed program is a ParseError (INVALID_ARGUMENT
// at compile), never an out-of-bounds read.
void validate_op(const Builder& B, const Op& op, const std::string& s) {
  static const std::set<std::string> unary = {"negate", "abs", "exponential", "log", "log_plus_one",
                                              "exponential_minus_one", "tanh", "rsqrt", "sqrt", "logistic",
                                              "floor", "ceil", "convert", "not", "reshape", "broadcast_in_dim",
                                              "transpose", "slice"};
  static const std::set<std::string> binary = {"add", "subtract", "multiply", "divide", "maximum", "minimum",
                                               "power", "compare", "and", "or", "dot_general", "dot",
                                               "shift_right_logical"};
  static const std::set<std::string> ternary = {"select", "clamp"};
  const size_t n = op.operands.size();
  auto bad = [&](const std::string& why) { throw ParseError(op.name + ": " + why + ": " + s); };
  if (unary.count(op.name) && n != 1) bad("takes 1 operand, has " + std::to_string(n));
  if (binary.count(op.name) && n != 2) bad("takes 2 operands, has " + std::to_string(n));
  if (ternary.count(op.name) && n != 3) bad("takes 3 operands, has " + std::to_string(n));
  if ((op.name == "constant" || op.name == "iota") && n != 0) bad("takes no operands");
  if (op.name == "reduce" && (n < 2 || n % 2 != 0)) bad("needs input / init operand pairs");
  if (op.name == "concatenate" && n < 1) bad("needs operands");
  const bool known = unary.count(op.name) || binary.count(op.name) || ternary.count(op.name) ||
                     op.name == "constant" || op.name == "iota" || op.name == "reduce" || op.name == "concatenate";
  if (!known) return;
  if (op.results.empty()) bad("has no result");
  auto rank = [&](int v) { return (int64_t)B.fn.values[v].type.dims.size(); };
  const int64_t rr = rank(op.results[0]);
  auto in_range = [&](const std::vector<int64_t>& d, int64_t r, const char* what) {
    std::set<int64_t> seen;
    for (int64_t x : d)
      if (x < 0 || x >= r || !seen.insert(x).second) bad(std::string(what) + " dimension out of range or repeated");
  };
  if (op.name == "dot_general") {
    const int64_t ra = rank(op.operands[0]), rb = rank(op.operands[1]);
    if (op.lhs_batch.size() != op.rhs_batch.size() || op.lhs_contract.size() != op.rhs_contract.size())
      bad("batching / contracting dimension lists differ in length");
    in_range(op.lhs_batch, ra, "lhs batching");
    in_range(op.rhs_batch, rb, "rhs batching");
    in_range(op.lhs_contract, ra, "lhs contracting");
    in_range(op.rhs_contract, rb, "rhs contracting");
    for (int64_t x : op.lhs_contract)
      for (int64_t y : op.lhs_batch)
        if (x == y) bad("a dimension both batching and contracting");
    for (int64_t x : op.rhs_contract)
      for (int64_t y : op.rhs_batch)
        if (x == y) bad("a dimension both batching and contracting");
  } else if (op.name == "broadcast_in_dim") {
    if ((int64_t)op.dims.size() != rank(op.operands[0])) bad("needs one dimension per operand dimension");
    for (int64_t x : op.dims)
      if (x < 0 || x >= rr) bad("broadcast dimension out of range");
  } else if (op.name == "transpose") {
    if ((int64_t)op.dims.size() != rank(op.operands[0]) || rank(op.operands[0]) != rr) bad("permutation rank");
    in_range(op.dims, rr, "permutation");
  } else if (op.name == "reduce") {
    in_range(op.dims, rank(op.operands[0]), "reduce");
    for (size_t i = 1; i < n / 2; ++i)
      if (rank(op.operands[i]) != rank(op.operands[0])) bad("inputs of different rank");
  } else if (op.name == "iota" || op.name == "concatenate") {
    if (op.dim < 0 || op.dim >= rr) bad("dimension out of range");
    if (op.name == "concatenate") {
      for (int v : op.operands)
        if (rank(v) != rr) bad("operands of different rank");
    }
  } else if (op.name == "slice") {
    const TensorType& in = B.fn.values[op.operands[0]].type;
    const TensorType& out = B.fn.values[op.results[0]].type;
    const size_t r = in.dims.size();
    if (op.slice_start.size() != r || op.slice_limit.size() != r || op.slice_stride.size() != r || out.dims.size() != r)
      bad("slice ranges do not match the rank");
    for (size_t i = 0; i < r; ++i) {
      const int64_t a = op.slice_start[i], b = op.slice_limit[i], st = op.slice_stride[i];
      if (a < 0 || b < a || b > in.dims[i] || st < 1) bad("slice range out of bounds");
      if (out.dims[i] != (b - a + st - 1) / st) bad("slice result shape");
    }
  }
}

void parse_body(const RawFunc& f, const std::vector<RawFunc>& all, Builder& B, const std::vector<int>& arg_ids,
                std::vector<int>* rets, int inline_depth);

void parse_while(const std::string& stmt, const std::vector<RawFunc>& all, Builder& B, int inline_depth);
bool fold_scalar(const Builder& B, int v, double* out, int depth = 0);

// The op name of a statement's first line ("while", "add", ...).
std::string statement_op(const std::string& stmt) {
  std::string first = stmt.substr(0, stmt.find('\n'));
  const size_t eq = first.find(" = ");
  std::string rhs = (!first.empty() && first[0] == '%' && eq != std::string::npos) ? trim(first.substr(eq + 3)) : first;
  size_t te = 0;
  while (te < rhs.size() && !isspace((unsigned char)rhs[te]) && rhs[te] != '(') ++te;
  return strip_dialect(rhs.substr(0, te));
}

void parse_statement(const std::string& stmt, const std::vector<RawFunc>& all, Builder& B,
                     std::vector<int>* rets, int inline_depth) {
  if (statement_op(stmt) == "while") {
    parse_while(stmt, all, B, inline_depth);
    return;
  }
  std::string s = stmt;
  // Separate a region body (reduce comparators) from the op line.
  // Multi-line statements: the op header is the first line, plus the last
  // line when it closes a generic-form region ("}) {attrs} : types").
  std::string region;
  const size_t nl = s.find('\n');
  if (nl != std::string::npos) {
    const size_t ll = s.rfind('\n');
    const std::string last = trim(s.substr(ll + 1));
    region = s.substr(nl + 1);
    s = s.substr(0, nl);
    if (starts_with(last, "})")) s += " " + last;
  }
  if (starts_with(s, "return") || starts_with(s, "func.return") || starts_with(s, "\"func.return\"") ||
      starts_with(s, "stablehlo.return") || starts_with(s, "\"stablehlo.return\"")) {
    const size_t tc = type_colon(s);
    for (const std::string& n : value_names(s.substr(0, tc))) rets->push_back(B.lookup(n));
    return;
  }
  // Results.
  std::vector<std::string> res_names;
  int nres_decl = 1;
  std::string rhs = s;
  const size_t eq = s.find(" = ");
  if (!s.empty() && s[0] == '%' && eq != std::string::npos) {
    const std::string lhs = s.substr(0, eq);
    rhs = trim(s.substr(eq + 3));
    const size_t colon = lhs.find(':');
    if (colon != std::string::npos) {
      nres_decl = atoi(lhs.c_str() + colon + 1);
      res_names.push_back(trim(lhs.substr(0, colon)));
    } else {
      for (const std::string& n : value_names(lhs)) res_names.push_back(n);
      nres_decl = (int)res_names.size();
    }
  }
  // Op name: first token of the RHS.
  size_t te = 0;
  while (te < rhs.size() && !isspace((unsigned char)rhs[te]) && rhs[te] != '(') ++te;
  std::string opname = strip_dialect(rhs.substr(0, te));
  const size_t tc = type_colon(rhs);
  const std::string body = tc == std::string::npos ? rhs : rhs.substr(0, tc);
  const std::string types = tc == std::string::npos ? "" : rhs.substr(tc + 1);

  if (opname == "call") {
    // Inline the private callee.
    const size_t at = rhs.find('@');
    size_t e = at + 1;
    while (e < rhs.size() && (isalnum((unsigned char)rhs[e]) || rhs[e] == '_' || rhs[e] == '.')) ++e;
    const std::string callee = rhs.substr(at + 1, e - at - 1);
    const RawFunc* cf = nullptr;
    for (const RawFunc& g : all)
      if (g.name == callee) cf = &g;
    if (!cf) throw ParseError("call to unknown function @" + callee);
    if (inline_depth > 16) throw ParseError("call nesting too deep at @" + callee);
    std::vector<int> args;
    for (const std::string& n : value_names(body)) args.push_back(B.lookup(n));
    std::vector<int> cret;
    std::map<std::string, int> saved = B.names;
    parse_body(*cf, all, B, args, &cret, inline_depth + 1);
    B.names = saved;
    if (cret.size() != res_names.size() && !(res_names.size() == 1 && nres_decl == (int)cret.size()))
      throw ParseError("call result count mismatch at @" + callee);
    if (res_names.size() == 1 && nres_decl > 1) {
      for (int i = 0; i < nres_decl; ++i) B.names[res_names[0] + "#" + std::to_string(i)] = cret[i];
    } else {
      for (size_t i = 0; i < cret.size(); ++i) B.names[res_names[i]] = cret[i];
    }
    return;
  }

  Op op;
  op.name = opname;
  op.text = s;
  // Operands: SSA names in the op body (excluding region-internal names).
  std::vector<std::string> opnd = value_names(body);
  if (opname == "dynamic_slice" && !opnd.empty()) {
    // With start indices that fold to constants (a counted loop unrolled
    // above, or constant operands) it is a static slice.  StableHLO clamps
    // each start to [0, dim - size].
    std::vector<int64_t> sizes;
    if (!list_after(rhs, "slice_sizes = ", &sizes)) list_after(rhs, "sizes = ", &sizes);
    const int src = B.lookup(opnd[0]);
    const TensorType& st = B.fn.values[src].type;
    bool folded = sizes.size() == st.dims.size() && opnd.size() == st.dims.size() + 1;
    std::vector<int64_t> start;
    for (size_t i = 1; folded && i < opnd.size(); ++i) {
      double c;
      folded = fold_scalar(B, B.lookup(opnd[i]), &c);
      const int64_t size = sizes[i - 1];
      if (folded && (size < 0 || size > st.dims[i - 1])) throw ParseError("dynamic_slice size out of bounds: " + s);
      if (folded) start.push_back(std::min(std::max<int64_t>((int64_t)c, 0), st.dims[i - 1] - size));
    }
    if (folded) {
      op.name = "slice";
      op.operands = {src};
      op.slice_start = start;
      for (size_t i = 0; i < start.size(); ++i) op.slice_limit.push_back(start[i] + sizes[i]);
      op.slice_stride.assign(start.size(), 1);
      std::vector<TensorType> rt = all_types(types.substr(types.rfind("->") == std::string::npos ? 0 : types.rfind("->") + 2));
      if (rt.empty() || res_names.size() != 1) throw ParseError("cannot read dynamic_slice result: " + s);
      const int v = B.new_value(rt.back(), res_names[0]);
      B.fn.values[v].def_op = (int)B.fn.ops.size();
      op.results.push_back(v);
      B.names[res_names[0]] = v;
      validate_op(B, op, s);
      B.fn.ops.push_back(op);
      return;
    }
  }
  if (opname == "reduce") {
    // Operands become inputs then init values.  Pretty form pairs them,
    // "(%x init: %c), (%y init: %d)"; the generic form already lists inputs
    // first.
    if (body.find("init:") != std::string::npos) {
      std::vector<std::string> ins, inits;
      for (size_t i = 0; i + 1 < opnd.size(); i += 2) {
        ins.push_back(opnd[i]);
        inits.push_back(opnd[i + 1]);
      }
      opnd = ins;
      opnd.insert(opnd.end(), inits.begin(), inits.end());
    } else {
      // Generic form: "(%x, %y, %c, %d) ({ ^bb0(...) ... })": region block
      // arguments are not operands.
      const size_t close = body.find(')');
      opnd = value_names(body.substr(0, close == std::string::npos ? body.size() : close));
    }
    list_after(s, "dimensions = ", &op.dims);
    const size_t ap = rhs.find("applies ");
    if (ap != std::string::npos) {
      size_t e = ap + 8;
      while (e < rhs.size() && !isspace((unsigned char)rhs[e])) ++e;
      op.reduce_body = strip_dialect(rhs.substr(ap + 8, e - ap - 8));
    } else {
      op.reduce_body = classify_reduce_body(region, nres_decl);
    }
  }
  static const std::set<std::string> known = {
      "add", "subtract", "multiply", "divide", "maximum", "minimum", "power", "compare", "and", "or", "not",
      "negate", "abs", "exponential", "log", "log_plus_one", "exponential_minus_one", "tanh", "rsqrt", "sqrt",
      "logistic", "floor", "ceil", "convert", "select", "clamp", "reshape", "broadcast_in_dim", "transpose",
      "dot_general", "dot", "reduce", "constant", "iota", "concatenate", "shift_right_logical", "slice"};
  for (const std::string& n : opnd) {
    // Ops outside the plugin's set may carry region-local names; they are
    // rejected by name later, so unknown operands are skipped here.
    if (!known.count(opname) && !B.names.count(n)) continue;
    op.operands.push_back(B.lookup(n));
  }

  // Attributes.
  if (opname == "dot_general") {
    list_after(rhs, "lhs_batching_dimensions = ", &op.lhs_batch);
    list_after(rhs, "rhs_batching_dimensions = ", &op.rhs_batch);
    list_after(rhs, "lhs_contracting_dimensions = ", &op.lhs_contract);
    list_after(rhs, "rhs_contracting_dimensions = ", &op.rhs_contract);
    size_t after;
    if (list_after(rhs, "batching_dims = ", &op.lhs_batch, &after) && rhs.find("lhs_batching") == std::string::npos)
      list_after(rhs.substr(after), "x ", &op.rhs_batch);
    if (list_after(rhs, "contracting_dims = ", &op.lhs_contract, &after) &&
        rhs.find("lhs_contracting") == std::string::npos)
      list_after(rhs.substr(after), "x ", &op.rhs_contract);
  } else if (opname == "broadcast_in_dim") {
    if (!list_after(rhs, "broadcast_dimensions = ", &op.dims)) list_after(rhs, "dims = ", &op.dims);
  } else if (opname == "transpose") {
    if (!list_after(rhs, "permutation = ", &op.dims)) list_after(rhs, "dims = ", &op.dims);
  } else if (opname == "iota" || opname == "concatenate") {
    size_t k = rhs.find("dim = ");
    if (k == std::string::npos) k = rhs.find("dimension = ");
    if (k != std::string::npos) op.dim = strtoll(rhs.c_str() + rhs.find('=', k) + 1, nullptr, 10);
  } else if (opname == "slice") {
    // Pretty form "stablehlo.slice %x [a:b, c:d:s]" or the generic
    // start_indices / limit_indices / strides attributes.
    if (!list_after(rhs, "start_indices = ", &op.slice_start)) {
      const size_t lb = body.find('[');
      const size_t rbk = body.find(']', lb == std::string::npos ? 0 : lb);
      if (lb == std::string::npos || rbk == std::string::npos) throw ParseError("slice without its ranges: " + s);
      const std::string r = body.substr(lb + 1, rbk - lb - 1);
      size_t p0 = 0;
      while (p0 <= r.size()) {
        size_t e = r.find(',', p0);
        if (e == std::string::npos) e = r.size();
        const std::string item = trim(r.substr(p0, e - p0));
        if (!item.empty()) {
          const std::vector<int64_t> v = int_list(item);
          if (v.size() < 2 || v.size() > 3 || item.find(':') == std::string::npos)
            throw ParseError("bad slice range '" + item + "': " + s);
          op.slice_start.push_back(v[0]);
          op.slice_limit.push_back(v[1]);
          op.slice_stride.push_back(v.size() == 3 ? v[2] : 1);
        }
        p0 = e + 1;
      }
    } else {
      list_after(rhs, "limit_indices = ", &op.slice_limit);
      if (!list_after(rhs, "strides = ", &op.slice_stride)) op.slice_stride.assign(op.slice_start.size(), 1);
    }
  } else if (opname == "compare") {
    for (const char* d : {"EQ", "NE", "LT", "LE", "GT", "GE"}) {
      const std::string ds(d);
      if (body.find(" " + ds + ",") != std::string::npos || body.find(" " + ds + " ") != std::string::npos ||
          rhs.find("comparison_direction " + ds + ">") != std::string::npos)
        op.compare_dir = ds;
    }
  }

  // Result types: after "->" when present, else the single type.
  std::vector<TensorType> rtypes;
  const size_t arrow = types.rfind("->");
  rtypes = all_types(arrow == std::string::npos ? types : types.substr(arrow + 2));
  if (arrow == std::string::npos && rtypes.size() > 1) rtypes = {rtypes.back()};  // select: "pred, value"
  if (opname == "constant") {
    if (rtypes.empty()) throw ParseError("constant without a type: " + s);
    parse_dense(rhs, rtypes[0].dtype, &op);
  }
  const int nres = res_names.empty() ? 0 : nres_decl;
  if ((int)rtypes.size() < nres) throw ParseError("cannot read result types of: " + s);
  for (int i = 0; i < nres; ++i) {
    const std::string nm = nres_decl > 1 && res_names.size() == 1 ? res_names[0] + "#" + std::to_string(i)
                                                                  : res_names[i];
    const int v = B.new_value(rtypes[i], nm);
    B.fn.values[v].def_op = (int)B.fn.ops.size();
    B.fn.values[v].result_index = i;
    op.results.push_back(v);
    B.names[nm] = v;
  }
  validate_op(B, op, s);
  B.fn.ops.push_back(op);
  // Integer and predicate scalars computed from constants (a counted loop's
  // index math once the loop is unrolled, and converts of it) become
  // constants, as the reference folds the index math of unrolled loops.
  auto int_like = [](int dt) { return dt != DT_F16 && dt != DT_F32 && dt != DT_F64 && dt != DT_BF16; };
  if (op.results.size() == 1 && op.name != "constant" && !op.operands.empty() &&
      B.fn.values[op.results[0]].type.numel() == 1 &&
      (int_like(B.fn.values[op.results[0]].type.dtype) ||
       (op.name == "convert" && int_like(B.fn.values[op.operands[0]].type.dtype)))) {
    double c;
    if (fold_scalar(B, op.results[0], &c)) {
      Op& k = B.fn.ops.back();
      k.name = "constant";
      k.operands.clear();
      k.const_values = {c};
      k.const_splat = true;
    }
  }
}

// Scalar value of v when it folds to a compile-time constant: a constant op
// (splat), or an integer/float scalar op (convert, reshape, broadcast of a
// scalar, add, subtract, multiply, maximum, minimum, negate, compare,
// select, and, or, not, clamp) of constants.
bool fold_scalar(const Builder& B, int v, double* out, int depth) {
  if (v < 0 || depth > 64) return false;
  const Value& val = B.fn.values[v];
  if (val.def_op < 0 || val.type.numel() != 1) return false;
  const Op& op = B.fn.ops[val.def_op];
  const bool is_int = val.type.dtype != DT_F16 && val.type.dtype != DT_F32 && val.type.dtype != DT_F64 &&
                      val.type.dtype != DT_BF16;
  if (op.name == "constant") {
    if (op.const_values.empty()) return false;
    *out = op.const_values[0];
    return true;
  }
  std::vector<double> a(op.operands.size());
  for (size_t i = 0; i < op.operands.size(); ++i) {
    const int u = op.operands[i];
    if (B.fn.values[u].type.numel() != 1 || !fold_scalar(B, u, &a[i], depth + 1)) return false;
  }
  auto as_int = [&](double x) { return is_int ? (double)(int64_t)x : x; };
  const size_t n = a.size();
  if ((op.name == "convert" || op.name == "reshape" || op.name == "broadcast_in_dim") && n == 1) {
    *out = val.type.dtype == DT_PRED ? (a[0] != 0) : as_int(a[0]);
    return true;
  }
  if (op.name == "negate" && n == 1) { *out = -a[0]; return true; }
  if (op.name == "not" && n == 1) {
    if (val.type.dtype != DT_PRED) return false;
    *out = a[0] == 0;
    return true;
  }
  if (n == 2) {
    if (op.name == "add") { *out = as_int(a[0] + a[1]); return true; }
    if (op.name == "subtract") { *out = as_int(a[0] - a[1]); return true; }
    if (op.name == "multiply") { *out = as_int(a[0] * a[1]); return true; }
    if (op.name == "maximum") { *out = std::max(a[0], a[1]); return true; }
    if (op.name == "minimum") { *out = std::min(a[0], a[1]); return true; }
    if (op.name == "and") { *out = (a[0] != 0 && a[1] != 0); return true; }
    if (op.name == "or") { *out = (a[0] != 0 || a[1] != 0); return true; }
    if (op.name == "compare") {
      const std::string& d = op.compare_dir;
      if (d == "EQ") *out = a[0] == a[1];
      else if (d == "NE") *out = a[0] != a[1];
      else if (d == "LT") *out = a[0] < a[1];
      else if (d == "LE") *out = a[0] <= a[1];
      else if (d == "GT") *out = a[0] > a[1];
      else if (d == "GE") *out = a[0] >= a[1];
      else return false;
      return true;
    }
  }
  if (n == 3 && op.name == "select") { *out = a[0] != 0 ? a[1] : a[2]; return true; }
  if (n == 3 && op.name == "clamp") { *out = std::min(std::max(a[1], a[0]), a[2]); return true; }
  return false;
}

// The text between the '{' at `open` and its matching '}'; `close` receives
// the position of that '}'.
std::string braced(const std::string& s, size_t open, size_t* close) {
  int d = 0;
  for (size_t i = open; i < s.size(); ++i) {
    if (s[i] == '{') ++d;
    if (s[i] == '}' && --d == 0) {
      *close = i;
      return s.substr(open + 1, i - open - 1);
    }
  }
  throw ParseError("unbalanced region braces in: " + s.substr(0, s.find('\n')));
}

std::vector<std::string> split_lines(const std::string& t) {
  std::vector<std::string> v;
  size_t p = 0;
  while (p <= t.size()) {
    size_t e = t.find('\n', p);
    if (e == std::string::npos) e = t.size();
    v.push_back(t.substr(p, e - p));
    p = e + 1;
  }
  return v;
}

// A region of a while op: its block-argument names and statements.
struct WhileRegion {
  std::vector<std::string> args;
  std::vector<std::string> stmts;
};

WhileRegion while_region(const std::string& text, const std::vector<std::string>& pretty_args) {
  WhileRegion r;
  std::vector<std::string> lines = split_lines(text);
  std::vector<std::string> raw;
  for (const std::string& l0 : lines) {
    const std::string l = trim(l0);
    if (l.empty()) continue;
    if (starts_with(l, "^bb") && r.args.empty() && raw.empty()) {
      // "^bb0(%arg2: tensor<i32>, %arg3: tensor<..>):" (generic form)
      const size_t lp = l.find('('), rp = l.rfind(')');
      const std::string a = l.substr(lp + 1, rp - lp - 1);
      size_t q = 0;
      while ((q = a.find('%', q)) != std::string::npos) {
        size_t e = q + 1;
        while (e < a.size() && (isalnum((unsigned char)a[e]) || a[e] == '_' || a[e] == '.')) ++e;
        r.args.push_back(a.substr(q, e - q));
        q = e;
      }
      continue;
    }
    raw.push_back(l);
  }
  if (r.args.empty()) r.args = pretty_args;
  r.stmts = join_statements(raw);
  return r;
}

// stablehlo.while, unrolled at parse time when it is a counted loop: the
// condition must fold to a constant for the loop-carried values of every
// trip (jax's lax.scan / fori_loop counters), and at most kMaxTrips trips
// run.  The body is inlined once per trip; loop-carried values flow from one
// copy to the next, and dynamic_slice ops indexed by the counter become
// static slices.  The reference unrolls short counted loops before planning
// the same way (core/stablehlo_parser.mm:462-519).  Other loops are an error
// naming the reason.
void parse_while(const std::string& stmt, const std::vector<RawFunc>& all, Builder& B, int inline_depth) {
  constexpr int kMaxTrips = 16;
  const size_t nl = stmt.find('\n');
  const std::string head = nl == std::string::npos ? stmt : stmt.substr(0, nl);
  // Results: "%0:3 = ..." or "%a, %b = ...".
  std::vector<std::string> res_names;
  int nres = 0;
  const size_t eq = head.find(" = ");
  if (eq == std::string::npos || head[0] != '%') throw ParseError("stablehlo.while without results: " + head);
  {
    const std::string lhs = head.substr(0, eq);
    const size_t colon = lhs.find(':');
    if (colon != std::string::npos) {
      nres = atoi(lhs.c_str() + colon + 1);
      const std::string base = trim(lhs.substr(0, colon));
      for (int i = 0; i < nres; ++i) res_names.push_back(nres > 1 ? base + "#" + std::to_string(i) : base);
    } else {
      res_names = value_names(lhs);
      nres = (int)res_names.size();
    }
  }
  const std::string rhs = trim(head.substr(eq + 3));
  const bool generic = starts_with(rhs, "\"stablehlo.while\"");
  std::vector<int> inits;
  std::vector<std::string> pretty_args;
  std::string cond_text, body_text;
  std::vector<TensorType> rtypes;
  const size_t lp = rhs.find('(');
  if (lp == std::string::npos) throw ParseError("stablehlo.while without operands: " + head);
  if (generic) {
    const size_t rp = rhs.find(')', lp);
    for (const std::string& n : value_names(rhs.substr(lp, rp - lp))) inits.push_back(B.lookup(n));
    const size_t o1 = stmt.find('{', nl == std::string::npos ? 0 : stmt.find(") ({", 0) + 3);
    size_t c1 = 0, c2 = 0;
    cond_text = braced(stmt, o1, &c1);
    const size_t o2 = stmt.find('{', c1 + 1);
    if (o2 == std::string::npos) throw ParseError("stablehlo.while without its body region");
    body_text = braced(stmt, o2, &c2);
    const std::string tail = stmt.substr(c2 + 1);
    const size_t arrow = tail.rfind("->");
    rtypes = all_types(arrow == std::string::npos ? tail : tail.substr(arrow + 2));
  } else {
    // "stablehlo.while(%iterArg = %c, %iterArg_0 = %x) : tensor<i32>, tensor<..>"
    int d = 0;
    size_t rp = lp;
    for (; rp < rhs.size(); ++rp) {
      if (rhs[rp] == '(') ++d;
      if (rhs[rp] == ')' && --d == 0) break;
    }
    const std::string pairs = rhs.substr(lp + 1, rp - lp - 1);
    const std::vector<std::string> names = value_names(pairs);
    if (names.size() % 2) throw ParseError("stablehlo.while operand list: " + head);
    for (size_t i = 0; i < names.size(); i += 2) {
      pretty_args.push_back(names[i]);
      inits.push_back(B.lookup(names[i + 1]));
    }
    const size_t colon = rhs.find(':', rp);
    if (colon != std::string::npos) rtypes = all_types(rhs.substr(colon + 1));
    const size_t cpos = stmt.find("cond", nl == std::string::npos ? stmt.size() : nl);
    if (cpos == std::string::npos) throw ParseError("stablehlo.while without its cond region");
    size_t c1 = 0, c2 = 0;
    cond_text = braced(stmt, stmt.find('{', cpos), &c1);
    const size_t dpos = stmt.find("do", c1);
    if (dpos == std::string::npos) throw ParseError("stablehlo.while without its do region");
    body_text = braced(stmt, stmt.find('{', dpos), &c2);
  }
  if ((int)inits.size() != nres || (int)rtypes.size() != nres)
    throw ParseError("stablehlo.while: " + std::to_string(inits.size()) + " operands, " + std::to_string(nres) +
                     " results, " + std::to_string(rtypes.size()) + " result types");
  for (int i = 0; i < nres; ++i)
    if (!(B.fn.values[inits[i]].type == rtypes[i]))
      throw ParseError("stablehlo.while: operand " + std::to_string(i) + " type differs from its result type");
  const WhileRegion cond = while_region(cond_text, pretty_args);
  const WhileRegion body = while_region(body_text, pretty_args);
  if ((int)cond.args.size() != nres || (int)body.args.size() != nres)
    throw ParseError("stablehlo.while: region arguments differ from the loop-carried values");

  std::vector<int> carried = inits;
  for (int trip = 0;; ++trip) {
    std::map<std::string, int> saved = B.names;
    for (int i = 0; i < nres; ++i) B.names[cond.args[i]] = carried[i];
    std::vector<int> cret;
    for (const std::string& st : cond.stmts) parse_statement(st, all, B, &cret, inline_depth);
    B.names = saved;
    double c = 0;
    if (cret.size() != 1 || !fold_scalar(B, cret[0], &c))
      throw ParseError("stablehlo.while: the loop condition does not fold to a constant; only counted loops of at "
                       "most " + std::to_string(kMaxTrips) + " trips are unrolled");
    if (c == 0) break;
    if (trip >= kMaxTrips)
      throw ParseError("stablehlo.while: more than " + std::to_string(kMaxTrips) +
                       " trips; only counted loops of at most " + std::to_string(kMaxTrips) + " trips are unrolled");
    saved = B.names;
    for (int i = 0; i < nres; ++i) B.names[body.args[i]] = carried[i];
    std::vector<int> bret;
    for (const std::string& st : body.stmts) parse_statement(st, all, B, &bret, inline_depth);
    B.names = saved;
    if ((int)bret.size() != nres) throw ParseError("stablehlo.while: the body returns the wrong number of values");
    for (int i = 0; i < nres; ++i)
      if (!(B.fn.values[bret[i]].type == rtypes[i]))
        throw ParseError("stablehlo.while: the body changes the type of loop-carried value " + std::to_string(i));
    carried = bret;
  }
  for (int i = 0; i < nres; ++i) B.names[res_names[i]] = carried[i];
}

void parse_body(const RawFunc& f, const std::vector<RawFunc>& all, Builder& B, const std::vector<int>& arg_ids,
                std::vector<int>* rets, int inline_depth) {
  if (arg_ids.size() != f.args.size()) throw ParseError("argument count mismatch for @" + f.name);
  for (size_t i = 0; i < f.args.size(); ++i) B.names[f.args[i].first] = arg_ids[i];
  for (const std::string& line : f.lines) parse_statement(line, all, B, rets, inline_depth);
}

}  // namespace

Function parse_stablehlo_text(const std::string& text) {
  std::vector<RawFunc> fns = split_functions(text);
  if (fns.empty()) throw ParseError("no func.func found in module text");
  const RawFunc* entry = nullptr;
  for (const RawFunc& f : fns)
    if (f.name == "main") entry = &f;
  if (!entry)
    for (const RawFunc& f : fns)
      if (f.is_public) entry = &f;
  if (!entry) throw ParseError("no public entry function");
  Builder B;
  std::vector<int> args;
  for (size_t i = 0; i < entry->args.size(); ++i) {
    const int v = B.new_value(entry->args[i].second, entry->args[i].first);
    B.fn.values[v].arg_index = (int)i;
    args.push_back(v);
  }
  B.fn.args = args;
  parse_body(*entry, fns, B, args, &B.fn.rets, 0);
  if (B.fn.rets.empty()) throw ParseError("entry function has no return");
  return B.fn;
}

}  // namespace mkrt
