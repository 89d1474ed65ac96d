// Reader for MLIR bytecode, the container jax's PJRT client hands to
// PJRT_Client_Compile with format "mlir": the StableHLO module serialized as
// a portable artifact (vhlo dialect) by StableHLO's serializePortableArtifact.
// The reference deserializes it with MLIR and StableHLO
// (core/stablehlo_parser.mm:568-586, pinned StableHLO 7b1b157 on LLVM
// 6d1ace547c9f, scripts/setup_deps.sh:38-40).  This build has neither: the
// reader below decodes the container itself and writes the module back out
// as MLIR text (module and func.func in the pretty form, every other op in
// the generic form) for the StableHLO text reader (shlo_parser.cpp).
//
// Container (MLIR's published bytecode format, versions 0-6):
//   file      magic "ML\xefR", version (varint), producer (NUL-terminated),
//             sections
//   section   id byte (bit 7: aligned), length (varint), [alignment (varint),
//             0xCB padding up to it, counted from the start of the file],
//             payload; ids 0 strings, 1 dialects, 2 attributes/types,
//             3 attribute/type offsets, 4 IR, 5 resources, 6 resource
//             offsets, 7 dialect versions, 8 properties
//   varint    the count of trailing zero bits of the first byte, plus one,
//             is the byte count (1-8); the value is the little-endian bytes
//             shifted right by that count; a first byte 0 is followed by the
//             8-byte value.  Signed varints are zigzag coded.
//   strings   count, byte sizes (NUL included) from the last string to the
//             first, then the strings in order
//   dialects  count, names (string << 1 | has_version, a nested dialect
//             versions section when set; the plain string before version 1),
//             [op-name count from version 4], groups of (dialect, count,
//             names (string, or string << 1 | registered from version 5))
//   offsets   attribute count, type count, dialect groups of entry sizes
//             (size << 1 | custom_encoding): attributes, then types
//   entries   text entries are the attribute's / type's MLIR text,
//             NUL-terminated; custom entries are the dialect's encoding
//   IR        a block holding the top-level op.  block: op count << 1 |
//             has_args, [arg count, args (type, location; type << 1 |
//             has_location [location] from version 4), use-list byte from
//             version 3], ops.  op: name, mask (1 attrs, 2 results,
//             4 operands, 8 successors, 16 regions, 32 use-list orders,
//             64 properties), location, [attribute dictionary],
//             [properties], [result count, types], [operand count, value
//             ids], [successors], [use-list orders],
//             [region count << 1 | isolated_from_above, regions -- inside
//             one nested IR section for an isolated op from version 2].
//             region: block count, [value count, blocks].
//   values    numbered per isolated-from-above op: each region reserves the
//             ids of its block arguments and op results as it opens, in
//             definition order; regions nested in it follow its range.
//
// Custom encodings decoded (each entry starts with the kind's code, a
// varint; lists are a varint count then the items):
//   builtin attributes  0 array (attrs), 1 dictionary ((name, value)
//     attrs), 2 string (string), 3 string with type (string, type),
//     4 flat symbol ref (string attr), 5 symbol ref (root, nested refs),
//     6 type (type), 7 unit, 8 integer (type, APInt), 9 float (type,
//     APFloat bits), 10-15 locations (never decoded), 17 dense array
//     (element type, count, blob), 18 dense elements (shaped type, blob)
//   builtin types  0 integer (width << 2 | signedness), 1 index,
//     2 function (inputs, results), 3 bf16, 4 f16, 5 f32, 6 f64, 12 none,
//     13 ranked tensor (shape svarints, element), 14 the same with an
//     encoding attribute first, 15 tuple, 18 unranked tensor
//   vhlo attributes (StableHLO's VhloBytecode.cpp)  0 array, 1 boolean
//     (varint), 2 comparison direction, 3 comparison type, 4 custom-call
//     API version (enums as varints), 5 dictionary, 6 FFT type, 7 float
//     (type, APFloat bits), 8 integer (type, APInt), 10 precision, 11 RNG
//     algorithm, 12 RNG distribution, 13 string, 14 tensor (type, blob),
//     15 transpose, 16 type, 17 type extensions (bounds svarints)
//   vhlo types  0 i1, 1 complex, 2 bf16, 3 f16, 4 f32, 5 f64, 6 f8E4M3FN,
//     7 f8E5M2, 8 function (inputs, results), 9 index, 10-14 i4 i8 i16 i32
//     i64, 15-19 ui4 ui8 ui16 ui32 ui64, 20 ranked tensor (shape svarints,
//     element), 21 the same with an encoding attribute first, 22 token,
//     23 tuple, 25 unranked tensor
//   APInt of a known width: width <= 8 one byte, <= 64 a signed varint.
//   blob: byte count (varint), bytes.
//
// vhlo ops are read under their stablehlo names (vhlo.add_v1 ->
// stablehlo.add, vhlo.func_v1 -> func.func, vhlo.call_v1 -> func.call,
// vhlo.return_v1 -> func.return / stablehlo.return by parent).  Entries of
// any other dialect with a custom encoding, op properties, successors,
// resources and multi-block regions are UNSUPPORTED; use-list orders are
// read and dropped (they do not change what the program computes).
#include "mlir_bytecode.h"

#include <ctype.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <initializer_list>
#include <memory>
#include <string>
#include <utility>
#include <vector>

namespace mkrt {

namespace {

[[noreturn]] void malformed(const std::string& m) { throw BytecodeError(BytecodeError::MALFORMED, m); }
[[noreturn]] void unsupported(const std::string& m) { throw BytecodeError(BytecodeError::UNSUPPORTED, m); }

constexpr int kMaxNesting = 128;          // regions in regions / entries in entries
constexpr int64_t kMaxArrayElems = 1 << 20;  // dimension lists rendered as array<...>

// Byte cursor over one section or entry.  `base` is the start of the file,
// for section alignment.
struct Cursor {
  const uint8_t* p = nullptr;
  const uint8_t* end = nullptr;
  const uint8_t* base = nullptr;
  const char* what = "";

  size_t left() const { return (size_t)(end - p); }
  [[noreturn]] void fail(const std::string& m) const { malformed(m + " in " + what); }
  uint8_t byte() {
    if (p >= end) fail("unexpected end");
    return *p++;
  }
  uint64_t varint() {
    const uint8_t first = byte();
    if (first & 1) return first >> 1;
    if (first == 0) {
      if (left() < 8) fail("truncated 9-byte varint");
      uint64_t v = 0;
      for (int i = 0; i < 8; ++i) v |= (uint64_t)p[i] << (8 * i);
      p += 8;
      return v;
    }
    int extra = 0;
    while (!(first & (1u << extra))) ++extra;  // 1..7: first != 0 and bit 0 clear
    if (left() < (size_t)extra) fail("truncated varint");
    uint64_t v = first;
    for (int i = 0; i < extra; ++i) v |= (uint64_t)p[i] << (8 * (i + 1));
    p += extra;
    return v >> (extra + 1);
  }
  uint64_t varint_flag(bool* flag) {
    const uint64_t v = varint();
    *flag = v & 1;
    return v >> 1;
  }
  int64_t svarint() {
    const uint64_t v = varint();
    return (int64_t)((v >> 1) ^ (~(v & 1) + 1));
  }
  // A count of items each taking at least one byte of what is left.
  uint64_t count() {
    const uint64_t n = varint();
    if (n > left()) fail("count larger than the remaining bytes");
    return n;
  }
  Cursor take(uint64_t n, const char* w) {
    if (n > left()) fail("length past the end");
    Cursor c{p, p + n, base, w};
    p += n;
    return c;
  }
  // One section header + payload; returns the section id.
  int section(Cursor* payload) {
    const uint8_t idb = byte();
    const uint64_t len = varint();
    if (idb & 0x80) {
      const uint64_t align = varint();
      if (align == 0 || (align & (align - 1)) || align > 4096) fail("bad section alignment");
      while (((size_t)(p - base) & (align - 1)) != 0)
        if (byte() != 0xCB) fail("bad section padding");
    }
    *payload = take(len, "section");
    return idb & 0x7F;
  }
};

enum Section { kString = 0, kDialect = 1, kAttrType = 2, kAttrTypeOffset = 3, kIR = 4, kResource = 5,
               kResourceOffset = 6, kDialectVersions = 7, kProperties = 8, kNumSections = 9 };

struct TypeInfo {
  std::string text;            // MLIR text
  bool tensor = false;         // ranked tensor
  std::vector<int64_t> shape;  // tensor dims
  std::string elem;            // element text (tensor) or the scalar's text
  int bits = 0;                // element width; 0 for non-number elements
  bool is_float = false;
  bool is_unsigned = false;
  bool is_func = false;
  std::vector<const TypeInfo*> inputs, results;  // function (inputs: tuple members)
};

struct AttrInfo {
  enum Kind { STRING, INTEGER, FLOAT, BOOL, ELEMENTS, ARRAY, DICT, TYPE, ENUM, SYMBOL, UNIT, TEXT, LOCATION };
  Kind kind = TEXT;
  std::string str;                 // STRING, ENUM, SYMBOL, TEXT
  uint64_t bits = 0;               // INTEGER / FLOAT / BOOL
  const TypeInfo* type = nullptr;  // INTEGER / FLOAT / ELEMENTS / TYPE
  std::vector<uint8_t> data;       // ELEMENTS: raw little-endian data
  std::vector<const AttrInfo*> elems;
  std::vector<std::pair<std::string, const AttrInfo*>> dict;
};

struct Entry {
  size_t dialect = 0;
  bool custom = false;
  Cursor data;
};

std::string hex_bytes(const uint8_t* d, size_t n) {
  static const char* k = "0123456789ABCDEF";
  std::string s = "0x";
  s.reserve(2 + 2 * n);
  for (size_t i = 0; i < n; ++i) {
    s += k[d[i] >> 4];
    s += k[d[i] & 15];
  }
  return s;
}

std::string quoted(const std::string& s) {
  std::string o = "\"";
  for (unsigned char c : s) {
    if (c == '"' || c == '\\') {
      o += '\\';
      o += (char)c;
    } else if (c < 0x20 || c >= 0x7F) {
      char b[4];
      snprintf(b, sizeof(b), "\\%02X", c);
      o += b;
    } else {
      o += (char)c;
    }
  }
  return o + "\"";
}

bool bare_identifier(const std::string& s) {
  if (s.empty() || !(isalpha((unsigned char)s[0]) || s[0] == '_')) return false;
  for (unsigned char c : s)
    if (!(isalnum(c) || c == '_' || c == '$' || c == '.')) return false;
  return true;
}

class Decoder {
 public:
  Decoder(const uint8_t* data, size_t size) : file_{data, data + size, data, "bytecode file"} {}

  std::string run() {
    static const uint8_t kMagic[4] = {'M', 'L', 0xEF, 'R'};
    if (file_.left() < 4 || memcmp(file_.p, kMagic, 4) != 0) malformed("not MLIR bytecode (no ML\\xefR magic)");
    file_.p += 4;
    version_ = file_.varint();
    if (version_ > 6)
      unsupported("MLIR bytecode version " + std::to_string(version_) + " (this reader takes versions 0-6)");
    while (file_.byte() != 0) {
    }  // producer string
    Cursor sec[kNumSections];
    bool present[kNumSections] = {};
    while (file_.left()) {
      Cursor payload;
      const int id = file_.section(&payload);
      if (id >= kNumSections) malformed("unknown section id " + std::to_string(id));
      if (present[id]) malformed("section " + std::to_string(id) + " appears twice");
      present[id] = true;
      sec[id] = payload;
    }
    for (int id : {kString, kDialect, kIR})
      if (!present[id]) malformed("missing section " + std::to_string(id));
    if (present[kAttrType] != present[kAttrTypeOffset]) malformed("attribute/type section without its offsets");
    if (present[kResource] && sec[kResource].left()) unsupported("bytecode resources (dense_resource) are not read");
    read_strings(sec[kString]);
    read_dialects(sec[kDialect]);
    if (present[kAttrTypeOffset]) read_offsets(sec[kAttrTypeOffset], sec[kAttrType]);

    Cursor ir = sec[kIR];
    ir.what = "IR section";
    std::string out;
    scopes_.emplace_back();
    open_region(0, ir);
    bool has_args = false;
    const uint64_t nops = ir.varint_flag(&has_args);
    if (has_args) ir.fail("top-level block with arguments");
    if (nops > ir.left()) ir.fail("op count larger than the section");
    for (uint64_t i = 0; i < nops; ++i) read_op(ir, &out, 0, "");
    if (ir.left()) ir.fail("trailing bytes after the top-level block");
    return out;
  }

 private:
  Cursor file_;
  uint64_t version_ = 0;
  std::vector<std::string> strings_;
  std::vector<std::string> dialects_;
  std::vector<std::pair<size_t, std::string>> ops_;  // (dialect, name)
  std::vector<Entry> attr_entries_, type_entries_;
  std::vector<std::unique_ptr<AttrInfo>> attrs_;
  std::vector<std::unique_ptr<TypeInfo>> types_;
  std::vector<std::unique_ptr<TypeInfo>> extra_types_;
  std::vector<char> attr_busy_, type_busy_;
  int entry_depth_ = 0;
  int next_name_ = 0;

  // Values of one isolated-from-above op: slots reserved per open region.
  struct Scope {
    std::vector<std::string> names, types;
    std::vector<size_t> next, base;
  };
  std::vector<Scope> scopes_;

  // ---- tables -----------------------------------------------------------

  const std::string& str(uint64_t i) const {
    if (i >= strings_.size()) malformed("string index " + std::to_string(i) + " out of range");
    return strings_[i];
  }

  void read_strings(Cursor r) {
    r.what = "string section";
    const uint64_t n = r.count();
    std::vector<uint64_t> size(n);
    for (uint64_t i = 0; i < n; ++i) size[n - 1 - i] = r.varint();
    strings_.resize(n);
    for (uint64_t i = 0; i < n; ++i) {
      if (size[i] == 0 || size[i] > r.left()) r.fail("string past the end");
      if (r.p[size[i] - 1] != 0) r.fail("string without its NUL");
      strings_[i].assign((const char*)r.p, size[i] - 1);
      r.p += size[i];
    }
    if (r.left()) r.fail("trailing bytes");
  }

  void read_dialects(Cursor r) {
    r.what = "dialect section";
    const uint64_t n = r.count();
    for (uint64_t i = 0; i < n; ++i) {
      bool has_version = false;
      const uint64_t s = version_ >= 1 ? r.varint_flag(&has_version) : r.varint();
      dialects_.push_back(str(s));
      if (has_version) {
        Cursor v;
        if (r.section(&v) != kDialectVersions) r.fail("dialect version outside a dialect-versions section");
      }
    }
    if (version_ >= 4) (void)r.varint();  // op-name count (a reservation hint)
    while (r.left()) {
      const uint64_t d = r.varint();
      if (d >= dialects_.size()) r.fail("op-name group of an unknown dialect");
      const uint64_t k = r.count();
      for (uint64_t i = 0; i < k; ++i) {
        bool registered = false;
        const uint64_t s = version_ >= 5 ? r.varint_flag(&registered) : r.varint();
        ops_.emplace_back((size_t)d, str(s));
      }
    }
  }

  void read_offsets(Cursor off, Cursor data) {
    off.what = "attribute/type offset section";
    data.what = "attribute/type section";
    const uint64_t na = off.varint(), nt = off.varint();
    if (na > off.left() || nt > off.left() - na) off.fail("entry counts larger than the section");
    auto group = [&](std::vector<Entry>* out, uint64_t total, const char* what) {
      while (out->size() < total) {
        const uint64_t d = off.varint();
        if (d >= dialects_.size()) off.fail("entry group of an unknown dialect");
        const uint64_t k = off.varint();
        if (k == 0 || k > total - out->size()) off.fail("entry group larger than its count");
        for (uint64_t i = 0; i < k; ++i) {
          Entry e;
          e.dialect = (size_t)d;
          const uint64_t size = off.varint_flag(&e.custom);
          e.data = data.take(size, what);
          out->push_back(e);
        }
      }
    };
    group(&attr_entries_, na, "attribute entry");
    group(&type_entries_, nt, "type entry");
    if (off.left()) off.fail("trailing bytes");
    attrs_.resize(na);
    types_.resize(nt);
    attr_busy_.assign(na, 0);
    type_busy_.assign(nt, 0);
  }

  // ---- attributes and types ----------------------------------------------

  struct Nest {
    int& d;
    explicit Nest(int& x) : d(x) {
      if (++d > kMaxNesting) {
        --d;
        malformed("attributes / types nested too deeply");
      }
    }
    ~Nest() { --d; }
  };

  const TypeInfo* type(uint64_t i) {
    if (i >= type_entries_.size()) malformed("type index " + std::to_string(i) + " out of range");
    if (types_[i]) return types_[i].get();
    if (type_busy_[i]) malformed("type entry " + std::to_string(i) + " refers to itself");
    type_busy_[i] = 1;
    Nest n(entry_depth_);
    Entry e = type_entries_[i];
    e.data.what = "type entry";
    std::unique_ptr<TypeInfo> t(new TypeInfo);
    const std::string& dialect = dialects_[e.dialect];
    if (!e.custom) {
      set_scalar(t.get(), text_entry(e));
    } else if (dialect == "builtin") {
      builtin_type(e.data, t.get());
    } else if (dialect == "vhlo") {
      vhlo_type(e.data, t.get());
    } else {
      unsupported("type of dialect '" + dialect + "' in its binary encoding");
    }
    if (e.custom && e.data.left()) e.data.fail("trailing bytes");
    type_busy_[i] = 0;
    types_[i] = std::move(t);
    return types_[i].get();
  }

  const AttrInfo* attr(uint64_t i) {
    if (i >= attr_entries_.size()) malformed("attribute index " + std::to_string(i) + " out of range");
    if (attrs_[i]) return attrs_[i].get();
    if (attr_busy_[i]) malformed("attribute entry " + std::to_string(i) + " refers to itself");
    attr_busy_[i] = 1;
    Nest n(entry_depth_);
    Entry e = attr_entries_[i];
    e.data.what = "attribute entry";
    std::unique_ptr<AttrInfo> a(new AttrInfo);
    const std::string& dialect = dialects_[e.dialect];
    if (!e.custom) {
      a->kind = AttrInfo::TEXT;
      a->str = text_entry(e);
    } else if (dialect == "builtin") {
      builtin_attr(e.data, a.get());
    } else if (dialect == "vhlo") {
      vhlo_attr(e.data, a.get());
    } else {
      unsupported("attribute of dialect '" + dialect + "' in its binary encoding");
    }
    if (e.custom && e.data.left()) e.data.fail("trailing bytes");
    attr_busy_[i] = 0;
    attrs_[i] = std::move(a);
    return attrs_[i].get();
  }

  static std::string text_entry(const Entry& e) {
    if (e.data.left() == 0 || e.data.end[-1] != 0) e.data.fail("text entry without its NUL");
    return std::string((const char*)e.data.p, e.data.left() - 1);
  }

  // A scalar type given by its text ("f32", "ui8", ...), with its width.
  static void set_scalar(TypeInfo* t, const std::string& s) {
    t->text = s;
    t->elem = s;
    if (s == "bf16" || s == "f16") t->bits = 16, t->is_float = true;
    else if (s == "f32") t->bits = 32, t->is_float = true;
    else if (s == "f64") t->bits = 64, t->is_float = true;
    else if (s == "f8E4M3FN" || s == "f8E5M2") t->bits = 8, t->is_float = true;
    else if (s == "index") t->bits = 64;
    else if (s.size() > 1 && s[0] == 'i' && isdigit((unsigned char)s[1])) t->bits = atoi(s.c_str() + 1);
    else if (s.size() > 2 && s[0] == 'u' && s[1] == 'i' && isdigit((unsigned char)s[2]))
      t->bits = atoi(s.c_str() + 2), t->is_unsigned = true;
    else if (s.size() > 2 && s[0] == 's' && s[1] == 'i' && isdigit((unsigned char)s[2])) t->bits = atoi(s.c_str() + 2);
    if (t->bits < 0 || t->bits > 4096) t->bits = 0;
  }

  std::vector<const TypeInfo*> type_list(Cursor& r) {
    const uint64_t n = r.count();
    std::vector<const TypeInfo*> v;
    for (uint64_t i = 0; i < n; ++i) v.push_back(type(r.varint()));
    return v;
  }

  void set_function(TypeInfo* t, Cursor& r) {
    t->is_func = true;
    t->inputs = type_list(r);
    t->results = type_list(r);
    std::string s = "(";
    for (size_t i = 0; i < t->inputs.size(); ++i) s += (i ? ", " : "") + t->inputs[i]->text;
    s += ") -> ";
    if (t->results.size() == 1 && !t->results[0]->is_func) {
      s += t->results[0]->text;
    } else {
      s += "(";
      for (size_t i = 0; i < t->results.size(); ++i) s += (i ? ", " : "") + t->results[i]->text;
      s += ")";
    }
    t->text = s;
  }

  void set_tensor(TypeInfo* t, Cursor& r, bool with_encoding) {
    if (with_encoding) (void)attr(r.varint());  // layout encoding: not used by the plan
    const uint64_t rank = r.count();
    std::string s = "tensor<";
    for (uint64_t i = 0; i < rank; ++i) {
      const int64_t d = r.svarint();
      t->shape.push_back(d);
      s += d < 0 ? std::string("?") : std::to_string(d);
      s += "x";
    }
    const TypeInfo* e = type(r.varint());
    if (e->tensor || e->is_func || e->text.compare(0, 6, "tensor") == 0) r.fail("tensor of a non-scalar element");
    t->tensor = true;
    t->elem = e->text;
    t->bits = e->bits;
    t->is_float = e->is_float;
    t->is_unsigned = e->is_unsigned;
    t->text = s + e->text + ">";
  }

  void set_tuple(TypeInfo* t, Cursor& r) {
    t->inputs = type_list(r);
    std::string s = "tuple<";
    for (size_t i = 0; i < t->inputs.size(); ++i) s += (i ? ", " : "") + t->inputs[i]->text;
    t->text = s + ">";
  }

  void set_unranked(TypeInfo* t, Cursor& r) {
    const TypeInfo* e = type(r.varint());
    t->text = "tensor<*x" + e->text + ">";
  }

  void builtin_type(Cursor& r, TypeInfo* t) {
    const uint64_t code = r.varint();
    switch (code) {
      case 0: {
        const uint64_t ws = r.varint();
        const uint64_t width = ws >> 2, sign = ws & 3;
        if (width == 0 || width > 4096 || sign == 3) r.fail("bad integer type");
        set_scalar(t, std::string(sign == 0 ? "i" : sign == 1 ? "si" : "ui") + std::to_string(width));
        return;
      }
      case 1: set_scalar(t, "index"); return;
      case 2: set_function(t, r); return;
      case 3: set_scalar(t, "bf16"); return;
      case 4: set_scalar(t, "f16"); return;
      case 5: set_scalar(t, "f32"); return;
      case 6: set_scalar(t, "f64"); return;
      case 12: set_scalar(t, "none"); return;
      case 13: set_tensor(t, r, false); return;
      case 14: set_tensor(t, r, true); return;
      case 15: set_tuple(t, r); return;
      case 18: set_unranked(t, r); return;
      default: unsupported("builtin type kind " + std::to_string(code));
    }
  }

  void vhlo_type(Cursor& r, TypeInfo* t) {
    static const char* const kScalar[] = {"i1",  nullptr, "bf16", "f16", "f32", "f64", "f8E4M3FN",
                                          "f8E5M2", nullptr, "index", "i4", "i8", "i16", "i32",
                                          "i64", "ui4", "ui8", "ui16", "ui32", "ui64"};
    const uint64_t code = r.varint();
    if (code < sizeof(kScalar) / sizeof(kScalar[0]) && kScalar[code]) {
      set_scalar(t, kScalar[code]);
      return;
    }
    switch (code) {
      case 1: {
        const TypeInfo* e = type(r.varint());
        t->text = "complex<" + e->text + ">";
        return;
      }
      case 8: set_function(t, r); return;
      case 20: set_tensor(t, r, false); return;
      case 21: set_tensor(t, r, true); return;
      case 22: t->text = "!stablehlo.token"; return;
      case 23: set_tuple(t, r); return;
      case 25: set_unranked(t, r); return;
      default: unsupported("vhlo type kind " + std::to_string(code));
    }
  }

  // APInt / APFloat bits of a known width.
  static uint64_t known_width_bits(Cursor& r, int bits) {
    if (bits <= 0) r.fail("integer or float attribute of a non-number type");
    if (bits <= 8) return r.byte();
    if (bits <= 64) {
      const uint64_t v = r.varint();
      return (v >> 1) ^ (~(v & 1) + 1);
    }
    unsupported("integer attributes wider than 64 bits");
  }

  void set_number(AttrInfo* a, Cursor& r, bool is_float) {
    a->type = type(r.varint());
    if (a->type->tensor || a->type->is_func) r.fail("number attribute of a non-scalar type");
    if (is_float != a->type->is_float) r.fail("number attribute of the wrong type class");
    a->kind = is_float ? AttrInfo::FLOAT : AttrInfo::INTEGER;
    a->bits = known_width_bits(r, a->type->bits);
    if (a->type->bits < 64) a->bits &= (1ull << a->type->bits) - 1;
  }

  static void set_elements(AttrInfo* a, Cursor& r, const TypeInfo* t) {
    a->kind = AttrInfo::ELEMENTS;
    a->type = t;
    const uint64_t n = r.varint();
    Cursor d = r.take(n, "elements data");
    a->data.assign(d.p, d.end);
  }

  std::vector<const AttrInfo*> attr_list(Cursor& r) {
    const uint64_t n = r.count();
    std::vector<const AttrInfo*> v;
    for (uint64_t i = 0; i < n; ++i) v.push_back(attr(r.varint()));
    return v;
  }

  void set_dict(AttrInfo* a, Cursor& r) {
    a->kind = AttrInfo::DICT;
    const uint64_t n = r.count();
    for (uint64_t i = 0; i < n; ++i) {
      const AttrInfo* k = attr(r.varint());
      const AttrInfo* v = attr(r.varint());
      if (k->kind != AttrInfo::STRING) r.fail("dictionary key that is not a string");
      a->dict.emplace_back(k->str, v);
    }
  }

  const AttrInfo* string_attr(Cursor& r) {
    const AttrInfo* s = attr(r.varint());
    if (s->kind != AttrInfo::STRING) r.fail("symbol reference without a string");
    return s;
  }

  void builtin_attr(Cursor& r, AttrInfo* a) {
    const uint64_t code = r.varint();
    switch (code) {
      case 0: a->kind = AttrInfo::ARRAY; a->elems = attr_list(r); return;
      case 1: set_dict(a, r); return;
      case 2: a->kind = AttrInfo::STRING; a->str = str(r.varint()); return;
      case 3:
        a->kind = AttrInfo::STRING;
        a->str = str(r.varint());
        (void)type(r.varint());
        return;
      case 4:
        a->kind = AttrInfo::SYMBOL;
        a->str = string_attr(r)->str;
        return;
      case 5: {
        a->kind = AttrInfo::SYMBOL;
        a->str = string_attr(r)->str;
        for (const AttrInfo* n : attr_list(r)) {
          if (n->kind != AttrInfo::SYMBOL) r.fail("nested symbol reference that is not flat");
          a->str += "::@" + n->str;
        }
        return;
      }
      case 6: a->kind = AttrInfo::TYPE; a->type = type(r.varint()); return;
      case 7: a->kind = AttrInfo::UNIT; return;
      case 8: set_number(a, r, false); return;
      case 9: set_number(a, r, true); return;
      case 10: case 11: case 12: case 13: case 14: case 15:
        a->kind = AttrInfo::LOCATION;  // locations are never rendered
        r.p = r.end;
        return;
      case 17: {
        const TypeInfo* e = type(r.varint());
        const uint64_t n = r.varint();
        if (e->bits <= 0 || e->tensor || e->is_func) r.fail("dense array of a non-number type");
        if (n > ((uint64_t)1 << 40)) r.fail("dense array too long");
        std::unique_ptr<TypeInfo> t(new TypeInfo(*e));
        t->tensor = true;
        t->shape = {(int64_t)n};
        t->text = "tensor<" + std::to_string(n) + "x" + e->text + ">";
        extra_types_.push_back(std::move(t));
        set_elements(a, r, extra_types_.back().get());
        return;
      }
      case 18: {
        const TypeInfo* t = type(r.varint());
        if (!t->tensor) r.fail("dense elements of a non-tensor type");
        set_elements(a, r, t);
        return;
      }
      default: unsupported("builtin attribute kind " + std::to_string(code));
    }
  }

  static void set_enum(AttrInfo* a, Cursor& r, const char* kind, std::initializer_list<const char*> names) {
    const uint64_t v = r.varint();
    if (v >= names.size()) r.fail(std::string("bad ") + kind + " value");
    a->kind = AttrInfo::ENUM;
    a->str = std::string("#stablehlo<") + kind + " " + names.begin()[v] + ">";
  }

  void vhlo_attr(Cursor& r, AttrInfo* a) {
    const uint64_t code = r.varint();
    switch (code) {
      case 0: a->kind = AttrInfo::ARRAY; a->elems = attr_list(r); return;
      case 1: {
        const uint64_t v = r.varint();
        if (v > 1) r.fail("bad boolean");
        a->kind = AttrInfo::BOOL;
        a->bits = v;
        return;
      }
      case 2: set_enum(a, r, "comparison_direction", {"EQ", "NE", "GE", "GT", "LE", "LT"}); return;
      case 3: set_enum(a, r, "comparison_type", {"NOTYPE", "FLOAT", "TOTALORDER", "SIGNED", "UNSIGNED"}); return;
      case 4:
        set_enum(a, r, "custom_call_api_version",
                 {"API_VERSION_UNSPECIFIED", "API_VERSION_ORIGINAL", "API_VERSION_STATUS_RETURNING",
                  "API_VERSION_STATUS_RETURNING_UNIFIED", "API_VERSION_TYPED_FFI"});
        return;
      case 5: set_dict(a, r); return;
      case 6: set_enum(a, r, "fft_type", {"FFT", "IFFT", "RFFT", "IRFFT"}); return;
      case 7: set_number(a, r, true); return;
      case 8: set_number(a, r, false); return;
      case 10: set_enum(a, r, "precision", {"DEFAULT", "HIGH", "HIGHEST"}); return;
      case 11: set_enum(a, r, "rng_algorithm", {"DEFAULT", "THREE_FRY", "PHILOX"}); return;
      case 12: set_enum(a, r, "rng_distribution", {"UNSPECIFIED", "UNIFORM", "NORMAL"}); return;
      case 13: a->kind = AttrInfo::STRING; a->str = str(r.varint()); return;
      case 14: {
        const TypeInfo* t = type(r.varint());
        if (!t->tensor) r.fail("tensor attribute of a non-tensor type");
        set_elements(a, r, t);
        return;
      }
      case 15: set_enum(a, r, "transpose", {"TRANSPOSE_INVALID", "NO_TRANSPOSE", "TRANSPOSE", "ADJOINT"}); return;
      case 16: a->kind = AttrInfo::TYPE; a->type = type(r.varint()); return;
      case 17: {
        const uint64_t n = r.count();
        std::string s = "#stablehlo.type_extensions<bounds = [";
        for (uint64_t i = 0; i < n; ++i) {
          const int64_t b = r.svarint();
          s += (i ? ", " : "") + (b < 0 ? std::string("?") : std::to_string(b));
        }
        a->kind = AttrInfo::TEXT;
        a->str = s + "]>";
        return;
      }
      default: unsupported("vhlo attribute kind " + std::to_string(code));
    }
  }

  // ---- rendering ---------------------------------------------------------

  // Element count, saturated at 2^41 (only compared with byte sizes); -1
  // for a dynamic dimension.
  static int64_t numel(const TypeInfo* t) {
    const int64_t kCap = (int64_t)1 << 41;
    int64_t n = 1;
    for (int64_t d : t->shape) {
      if (d < 0) return -1;
      n = (d != 0 && n > kCap / d) ? kCap : n * d;
    }
    return n;
  }

  std::string render_elements(const AttrInfo* a, bool as_array) {
    const TypeInfo* t = a->type;
    const int64_t n = numel(t);
    if (n < 0) malformed("elements of a dynamically shaped type " + t->text);
    if (t->bits <= 0) unsupported("elements of type " + t->text);
    const size_t eb = (size_t)(t->bits + 7) / 8;
    std::vector<uint8_t> d = a->data;
    if (t->bits == 1 && n > 1 && d.size() != (size_t)n && d.size() == (size_t)(n + 7) / 8) {
      // Bit-packed booleans (lowest bit first): one byte per element here.
      std::vector<uint8_t> u((size_t)n);
      for (int64_t i = 0; i < n; ++i) u[(size_t)i] = (d[(size_t)i / 8] >> (i % 8)) & 1;
      d.swap(u);
    } else if (t->bits == 1) {
      for (uint8_t& b : d) b = b ? 1 : 0;
    }
    const bool splat = n > 1 && d.size() == eb;
    if (!splat && (uint64_t)d.size() != (uint64_t)n * eb)
      malformed("elements data of " + std::to_string(d.size()) + " bytes for " + t->text);
    if (as_array && t->shape.size() == 1 && !t->is_float && eb <= 8 && n <= kMaxArrayElems) {
      std::string s = "array<" + t->elem;
      for (int64_t i = 0; i < n; ++i) {
        uint64_t bits = 0;
        memcpy(&bits, d.data() + (splat ? 0 : (size_t)i * eb), eb);
        if (!t->is_unsigned && eb < 8 && ((bits >> (8 * eb - 1)) & 1)) bits |= ~0ull << (8 * eb);
        s += (i ? ", " : ": ") + (t->is_unsigned ? std::to_string(bits) : std::to_string((int64_t)bits));
      }
      return s + ">";
    }
    if (n == 0) return "dense<> : " + t->text;
    return "dense<\"" + hex_bytes(d.data(), d.size()) + "\"> : " + t->text;
  }

  static std::string render_number(const AttrInfo* a) {
    const TypeInfo* t = a->type;
    if (a->kind == AttrInfo::FLOAT) {
      char b[40];
      snprintf(b, sizeof(b), "0x%0*llX", (t->bits + 3) / 4, (unsigned long long)a->bits);
      return std::string(b) + " : " + t->text;
    }
    if (t->bits == 1) return a->bits ? "true" : "false";
    if (t->is_unsigned) return std::to_string(a->bits) + " : " + t->text;
    uint64_t v = a->bits;
    if (t->bits < 64 && ((v >> (t->bits - 1)) & 1)) v |= ~0ull << t->bits;
    return std::to_string((int64_t)v) + " : " + t->text;
  }

  std::string render(const AttrInfo* a, const std::string& key) {
    switch (a->kind) {
      case AttrInfo::STRING: return key == "callee" ? "@" + a->str : quoted(a->str);
      case AttrInfo::INTEGER:
      case AttrInfo::FLOAT: return render_number(a);
      case AttrInfo::BOOL: return a->bits ? "true" : "false";
      case AttrInfo::ELEMENTS: return render_elements(a, key != "value");
      case AttrInfo::ARRAY: {
        std::string s = "[";
        for (size_t i = 0; i < a->elems.size(); ++i) s += (i ? ", " : "") + render(a->elems[i], "");
        return s + "]";
      }
      case AttrInfo::DICT: return "{" + render_dict(a) + "}";
      case AttrInfo::TYPE: return a->type->text;
      case AttrInfo::ENUM:
      case AttrInfo::TEXT: return a->str;
      case AttrInfo::SYMBOL: return "@" + a->str;
      case AttrInfo::UNIT: return "unit";
      case AttrInfo::LOCATION: return "loc(unknown)";
    }
    return "";
  }

  std::string render_dict(const AttrInfo* a) {
    std::string s;
    for (size_t i = 0; i < a->dict.size(); ++i) {
      const std::string& k = a->dict[i].first;
      s += (i ? ", " : "") + (bare_identifier(k) ? k : quoted(k));
      if (a->dict[i].second->kind != AttrInfo::UNIT) s += " = " + render(a->dict[i].second, k);
    }
    return s;
  }

  // ---- IR ----------------------------------------------------------------

  Scope& scope() { return scopes_.back(); }

  void open_region(uint64_t num_values, const Cursor& r) {
    if (num_values > r.left()) r.fail("region declares more values than it has bytes");
    Scope& s = scope();
    s.base.push_back(s.names.size());
    s.next.push_back(s.names.size());
    s.names.resize(s.names.size() + num_values);
    s.types.resize(s.names.size());
  }

  void close_region() {
    Scope& s = scope();
    s.names.resize(s.base.back());
    s.types.resize(s.base.back());
    s.base.pop_back();
    s.next.pop_back();
  }

  std::string define(const std::string& type_text, const Cursor& r) {
    Scope& s = scope();
    if (s.next.empty() || s.next.back() >= s.names.size()) r.fail("more values defined than the region declares");
    const std::string name = "%v" + std::to_string(next_name_++);
    s.names[s.next.back()] = name;
    s.types[s.next.back()] = type_text;
    ++s.next.back();
    return name;
  }

  static void skip_use_lists(Cursor& r, uint64_t num_values) {
    const uint64_t n = num_values > 1 ? r.count() : 1;
    for (uint64_t i = 0; i < n; ++i) {
      if (num_values > 1 && r.varint() >= num_values) r.fail("use-list order of a value out of range");
      bool pairs = false;
      const uint64_t k = r.varint_flag(&pairs);
      if (k > r.left()) r.fail("use-list order longer than the section");
      for (uint64_t j = 0; j < k; ++j) (void)r.varint();
    }
  }

  std::string op_name(uint64_t i, const std::string& parent) const {
    if (i >= ops_.size()) malformed("op name index " + std::to_string(i) + " out of range");
    const std::string& dialect = dialects_[ops_[i].first];
    const std::string& name = ops_[i].second;
    if (dialect != "vhlo") return dialect + "." + name;
    std::string n = name;
    const size_t v = n.rfind("_v");
    if (v != std::string::npos && v + 2 < n.size() && isdigit((unsigned char)n[v + 2])) n = n.substr(0, v);
    if (n == "func") return "func.func";
    if (n == "call") return "func.call";
    if (n == "return") return parent == "func.func" ? "func.return" : "stablehlo.return";
    return "stablehlo." + n;
  }

  struct RegionText {
    std::vector<std::pair<std::string, std::string>> args;  // (name, type)
    std::string body;
    bool empty = true;
  };

  RegionText read_region(Cursor& r, int depth, const std::string& parent) {
    RegionText rt;
    const uint64_t nblocks = r.varint();
    if (nblocks == 0) return rt;
    if (nblocks != 1) unsupported("regions of more than one block (" + parent + ")");
    rt.empty = false;
    const uint64_t nvalues = r.varint();
    open_region(nvalues, r);
    bool has_args = false;
    const uint64_t nops = r.varint_flag(&has_args);
    if (nops > r.left()) r.fail("op count larger than the section");
    if (has_args) {
      const uint64_t n = r.count();
      for (uint64_t i = 0; i < n; ++i) {
        bool has_loc = true;
        const uint64_t t = version_ >= 4 ? r.varint_flag(&has_loc) : r.varint();
        if (has_loc) (void)r.varint();
        const std::string tt = type(t)->text;
        rt.args.emplace_back(define(tt, r), tt);
      }
      if (version_ >= 3 && r.byte()) skip_use_lists(r, n);
    }
    for (uint64_t i = 0; i < nops; ++i) read_op(r, &rt.body, depth, parent);
    close_region();
    return rt;
  }

  std::vector<RegionText> read_regions(Cursor& r, int depth, const std::string& name) {
    if (depth >= kMaxNesting) r.fail("regions nested too deeply");
    bool isolated = false;
    const uint64_t n = r.varint_flag(&isolated);
    if (n > r.left() + 1) r.fail("region count larger than the section");
    std::vector<RegionText> out;
    Cursor inner;
    Cursor* src = &r;
    if (isolated && version_ >= 2) {
      if (r.section(&inner) != kIR) r.fail("regions of an isolated op outside an IR section");
      inner.what = "region section";
      src = &inner;
    }
    if (isolated) scopes_.emplace_back();
    for (uint64_t k = 0; k < n; ++k) out.push_back(read_region(*src, depth + 1, name));
    if (isolated) scopes_.pop_back();
    if (src == &inner && inner.left()) inner.fail("trailing bytes after the regions");
    return out;
  }

  static std::string get_str(const AttrInfo* dict, const char* key) {
    if (!dict) return "";
    for (const auto& kv : dict->dict)
      if (kv.first == key && (kv.second->kind == AttrInfo::STRING || kv.second->kind == AttrInfo::SYMBOL))
        return kv.second->str;
    return "";
  }

  static const TypeInfo* get_type(const AttrInfo* dict, const char* key) {
    if (!dict) return nullptr;
    for (const auto& kv : dict->dict)
      if (kv.first == key && kv.second->kind == AttrInfo::TYPE) return kv.second->type;
    return nullptr;
  }

  void read_op(Cursor& r, std::string* out, int depth, const std::string& parent) {
    const std::string name = op_name(r.varint(), parent);
    const uint8_t mask = r.byte();
    if (mask & 0x80) r.fail("unknown op encoding bit");
    (void)r.varint();  // location
    const AttrInfo* attrs = nullptr;
    if (mask & 0x01) {
      attrs = attr(r.varint());
      if (attrs->kind != AttrInfo::DICT) r.fail("op attributes that are not a dictionary");
    }
    if (mask & 0x40) {
      if (version_ < 5) r.fail("op properties before bytecode version 5");
      unsupported("op properties (" + name + ")");
    }
    std::vector<std::string> rtypes;
    if (mask & 0x02) {
      const uint64_t n = r.count();
      for (uint64_t i = 0; i < n; ++i) rtypes.push_back(type(r.varint())->text);
    }
    std::vector<std::string> operands, otypes;
    if (mask & 0x04) {
      const uint64_t n = r.count();
      const Scope& s = scope();
      for (uint64_t i = 0; i < n; ++i) {
        const uint64_t v = r.varint();
        if (v >= s.names.size() || s.names[v].empty()) r.fail("operand refers to a value not defined before it");
        operands.push_back(s.names[v]);
        otypes.push_back(s.types[v]);
      }
    }
    if (mask & 0x08) unsupported("successors (" + name + ")");
    if (mask & 0x20) {
      if (version_ < 3) r.fail("use-list orders before bytecode version 3");
      skip_use_lists(r, rtypes.size());
    }

    std::vector<std::string> results;
    for (const std::string& t : rtypes) results.push_back(define(t, r));
    if (results.size() > 1) {
      // "%vN:k = ...", members "%vN#i".
      Scope& s = scope();
      const size_t first = s.next.back() - results.size();
      for (size_t i = 0; i < results.size(); ++i) s.names[first + i] = results[0] + "#" + std::to_string(i);
    }
    std::vector<RegionText> regions;
    if (mask & 0x10) regions = read_regions(r, depth, name);

    if (name == "builtin.module") {
      if (regions.size() != 1) r.fail("module without its region");
      const std::string sym = get_str(attrs, "sym_name");
      *out += "module" + (sym.empty() ? std::string() : " @" + sym) + " {\n" + regions[0].body + "}\n";
      return;
    }
    if (name == "func.func") {
      const std::string sym = get_str(attrs, "sym_name");
      const TypeInfo* fty = get_type(attrs, "function_type");
      if (sym.empty() || !fty || !fty->is_func) r.fail("func without sym_name / function_type");
      if (regions.size() != 1 || regions[0].empty) unsupported("function declarations without a body (@" + sym + ")");
      const RegionText& body = regions[0];
      if (body.args.size() != fty->inputs.size()) r.fail("function arguments differ from its type (@" + sym + ")");
      const std::string vis = get_str(attrs, "sym_visibility");
      std::string h = "func.func " + (vis.empty() ? std::string("public") : vis) + " @" + sym + "(";
      for (size_t i = 0; i < body.args.size(); ++i) h += (i ? ", " : "") + body.args[i].first + ": " + body.args[i].second;
      h += ") -> (";
      for (size_t i = 0; i < fty->results.size(); ++i) h += (i ? ", " : "") + fty->results[i]->text;
      *out += h + ") {\n" + body.body + "}\n";
      return;
    }

    std::string line;
    if (results.size() == 1) line = results[0] + " = ";
    else if (results.size() > 1) line = results[0] + ":" + std::to_string(results.size()) + " = ";
    line += "\"" + name + "\"(";
    for (size_t i = 0; i < operands.size(); ++i) line += (i ? ", " : "") + operands[i];
    line += ")";
    if (!regions.empty()) {
      line += " (";
      for (size_t k = 0; k < regions.size(); ++k) {
        line += k ? ", {\n" : "{\n";
        const RegionText& rt = regions[k];
        if (!rt.args.empty()) {
          line += "^bb0(";
          for (size_t i = 0; i < rt.args.size(); ++i) line += (i ? ", " : "") + rt.args[i].first + ": " + rt.args[i].second;
          line += "):\n";
        }
        line += rt.body + "}";
      }
      line += ")";
    }
    if (attrs && !attrs->dict.empty()) line += " {" + render_dict(attrs) + "}";
    line += " : (";
    for (size_t i = 0; i < otypes.size(); ++i) line += (i ? ", " : "") + otypes[i];
    line += ") -> ";
    if (rtypes.size() == 1) {
      line += rtypes[0];
    } else {
      line += "(";
      for (size_t i = 0; i < rtypes.size(); ++i) line += (i ? ", " : "") + rtypes[i];
      line += ")";
    }
    *out += line + "\n";
  }
};

}  // namespace

bool is_mlir_bytecode(const char* data, size_t size) { return size >= 4 && memcmp(data, "ML\xefR", 4) == 0; }

std::string mlir_bytecode_to_text(const char* data, size_t size) {
  Decoder d(reinterpret_cast<const uint8_t*>(data), size);
  return d.run();
}

}  // namespace mkrt
