"""MLIR bytecode writer for the tests (test infrastructure, not product code).

It turns the StableHLO text that ``mi355x.programs`` prints (the pretty forms
of ``jax.jit(f).lower(...).as_text()``) into MLIR bytecode. The plugin's
reader (csrc/runtime/mlir_bytecode.cpp) must turn that bytecode back into a
program that plans exactly like the text. Two flavours:

* ``"vhlo"``: a StableHLO portable artifact, as jaxlib's PJRT client sends to
  PJRT_Client_Compile (/root/reference/src/pjrt_plugin/api/pjrt_client.cc:178-244;
  deserialized there by core/stablehlo_parser.mm:568-586). Ops are
  ``vhlo.<op>_v1``. Attributes and types use the vhlo dialect's binary
  encoding. Op attribute dictionaries, their string keys and locations use
  the builtin dialect's encoding.
* ``"builtin"``: the same module in the stablehlo / func dialects. Types,
  integers, strings, dense elements and dense arrays use the builtin
  encoding; stablehlo enum attributes are text entries (a dialect without a
  binary encoding).

The container follows MLIR's published bytecode format, versions 0-6. The
vhlo codes follow StableHLO's VhloBytecode.cpp. StableHLO is pinned by the
reference at 7b1b157 (scripts/setup_deps.sh:38-40); it is absent here, so
the codes are restated, not checked against it. jax is not installed either,
so nothing here is checked against jax's own emitter: the round trip pins
the reader against this writer, and the hand-assembled files in
tests/test_bytecode_cpu.py pin both against the format as written down.
"""

import re
import struct

import numpy as np

# ---------------------------------------------------------------- encoding


def varint(v, width=None):
    """MLIR prefix varint: n bytes carry 7n value bits, with n-1 trailing
    zero bits and a one bit marking the length; a zero first byte is followed
    by the 8-byte value. `width` forces a (possibly longer) encoding."""
    if not 0 <= v < 1 << 64:
        raise ValueError(v)
    if width is None:
        width = next((n for n in range(1, 9) if v < 1 << (7 * n)), 9)
    if width == 9:
        return b"\x00" + v.to_bytes(8, "little")
    if v >= 1 << (7 * width):
        raise ValueError(f"{v} does not fit a {width}-byte varint")
    return ((v << width) | (1 << (width - 1))).to_bytes(width, "little")


def zigzag(v):
    if not -(1 << 63) <= v < 1 << 63:
        raise ValueError(v)
    return ((v << 1) ^ (v >> 63)) & ((1 << 64) - 1)


def varint_flag(v, flag, width=None):
    return varint((v << 1) | int(bool(flag)), width)


# ------------------------------------------------------------------ types
#
# A type is ("tensor", shape, elem), ("scalar", elem) or ("func", ins, outs).

_ELEM_BITS = {"i1": 1, "i4": 4, "i8": 8, "i16": 16, "i32": 32, "i64": 64, "ui4": 4, "ui8": 8, "ui16": 16,
              "ui32": 32, "ui64": 64, "bf16": 16, "f16": 16, "f32": 32, "f64": 64, "index": 64}


def parse_type(s):
    s = s.strip()
    m = re.fullmatch(r"tensor<(.*)>", s)
    if not m:
        return ("scalar", s)
    parts = m.group(1).split("x")
    return ("tensor", tuple(int(d) for d in parts[:-1]), parts[-1])


def type_text(t):
    if t[0] == "tensor":
        return "tensor<" + "".join(f"{d}x" for d in t[1]) + t[2] + ">"
    if t[0] == "func":
        outs = ", ".join(type_text(o) for o in t[2])
        return "(" + ", ".join(type_text(i) for i in t[1]) + ") -> " + (outs if len(t[2]) == 1 else f"({outs})")
    return t[1]


# ------------------------------------------------------------- attributes
#
# ("str", s) ("int", value, elem) ("float", bits, elem) ("bool", b)
# ("elements", tensor_type, raw_bytes) ("dims", [ints]) ("array", [attrs])
# ("dict", [(key, attr)]) ("type", type) ("enum", kind, index) ("unit",)

ENUMS = {
    "comparison_direction": ["EQ", "NE", "GE", "GT", "LE", "LT"],
    "comparison_type": ["NOTYPE", "FLOAT", "TOTALORDER", "SIGNED", "UNSIGNED"],
    "precision": ["DEFAULT", "HIGH", "HIGHEST"],
}


def _bf16_bits(x):
    u = int(np.array(x, dtype=np.float32).view(np.uint32))
    if (u & 0x7F800000) == 0x7F800000 and (u & 0x7FFFFF):
        return 0x7FC0
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF


def element_bytes(tok, elem):
    """Little-endian bytes of one dense<> element written as `tok`."""
    tok = tok.strip()
    bits = _ELEM_BITS[elem]
    nbytes = max(1, (bits + 7) // 8)
    if tok in ("true", "false"):
        return bytes([tok == "true"])
    if tok.startswith("0x") and elem in ("bf16", "f16", "f32", "f64"):
        return int(tok, 16).to_bytes(nbytes, "little")
    if elem in ("f32", "f64", "f16", "bf16"):
        v = float(tok)
        if elem == "f32":
            return struct.pack("<f", v)
        if elem == "f64":
            return struct.pack("<d", v)
        if elem == "f16":
            return np.array(v, dtype=np.float16).tobytes()
        return _bf16_bits(v).to_bytes(2, "little")
    v = int(tok, 0)
    return (v & ((1 << (8 * nbytes)) - 1)).to_bytes(nbytes, "little")


def dense(payload, t):
    """("elements", t, raw) from the text inside dense<...>: one value (a
    splat, stored as one element) or a flat / nested list."""
    payload = payload.strip()
    if payload.startswith("["):
        toks = [x for x in re.split(r"[\[\],\s]+", payload) if x]
        raw = b"".join(element_bytes(x, t[2]) for x in toks)
    else:
        raw = element_bytes(payload, t[2])
    return ("elements", t, raw)


# ---------------------------------------------------------------- op tree


class Value:
    __slots__ = ("type",)

    def __init__(self, t):
        self.type = t


class Op:
    def __init__(self, name, operands=(), results=(), attrs=(), regions=(), isolated=False):
        self.name = name
        self.operands = list(operands)
        self.results = list(results)
        self.attrs = list(attrs)
        self.regions = list(regions)  # each region: list of blocks; block: (args, ops)
        self.isolated = isolated


def _list(s):
    return [int(x) for x in re.findall(r"-?\d+", s)]


def _top_colon(s):
    depth, last = 0, -1
    for i, c in enumerate(s):
        if c in "([{<":
            depth += 1
        elif c in ")]}" or (c == ">" and s[i - 1] != "-"):
            depth -= 1
        elif c == ":" and depth == 0 and s[i - 1:i] == " " and s[i + 1:i + 2] == " ":
            last = i
    return last


def _types(s):
    """(operand types, result types) of a trailing type signature."""
    s = s.strip()
    if "->" in s:
        ins, outs = s.split("->", 1)
        ins = ins.strip()[1:-1]
        outs = outs.strip()
        if outs.startswith("("):
            outs = outs[1:-1]
        return [parse_type(x) for x in re.findall(r"tensor<[^>]*>", ins)], \
               [parse_type(x) for x in re.findall(r"tensor<[^>]*>", outs)]
    ts = [parse_type(x) for x in re.findall(r"tensor<[^>]*>", s)]
    return ts, ts[-1:]


class _Reader:
    """The pretty StableHLO forms mi355x.programs prints."""

    def __init__(self, text):
        self.lines = [l.strip() for l in text.splitlines()]
        self.i = 0

    def module(self):
        m = re.match(r"module(?: @([\w.$]+))?", self.lines[0])
        name = m.group(1) if m else None
        funcs = []
        self.i = 1
        while self.i < len(self.lines):
            if self.lines[self.i].startswith("func.func"):
                funcs.append(self.func())
            else:
                self.i += 1
        attrs = [("sym_name", ("str", name))] if name else []
        return Op("builtin.module", attrs=attrs, regions=[[([], funcs)]], isolated=True)

    def func(self):
        head = self.lines[self.i]
        self.i += 1
        m = re.match(r"func\.func (?:(public|private) )?@([\w.$]+)\((.*?)\) -> (.*) \{$", head)
        vis, name, args, rets = m.group(1), m.group(2), m.group(3), m.group(4)
        env = {}
        block_args = []
        for an, at in re.findall(r"(%[\w.$]+): (tensor<[^>]*>)", args):
            v = Value(parse_type(at))
            env[an] = v
            block_args.append(v)
        ret_types = [parse_type(x) for x in re.findall(r"tensor<[^>]*>", rets)]
        ops = self.body(env)
        ftype = ("func", tuple(v.type for v in block_args), tuple(ret_types))
        attrs = [("sym_name", ("str", name)), ("function_type", ("type", ftype))]
        if vis == "private":
            attrs.append(("sym_visibility", ("str", "private")))
        return Op("func.func", attrs=attrs, regions=[[(block_args, ops)]], isolated=True)

    def body(self, env, end=("}",)):
        ops = []
        while True:
            line = self.lines[self.i]
            self.i += 1
            if line in end:
                return ops
            ops.append(self.stmt(line, env))

    def ref(self, env, n):
        if n not in env:
            raise ValueError(f"undefined {n}")
        return env[n]

    def stmt(self, line, env):
        m = re.match(r"(%[\w.$]+)(?::(\d+))? = (.*)$", line)
        names, rhs = ([], line) if not m else ([m.group(1)], m.group(3))
        nres = int(m.group(2)) if m and m.group(2) else (1 if m else 0)
        tc = _top_colon(rhs)
        body, sig = (rhs[:tc], rhs[tc + 1:]) if tc >= 0 else (rhs, "")
        ins, outs = _types(sig) if sig else ([], [])
        opname = body.split(None, 1)[0].split("(")[0]
        rest = body[len(opname):]
        refs = re.findall(r"%[\w.$#]+", rest)
        attrs, regions, operands = [], [], None
        short = opname.split(".", 1)[1] if "." in opname else opname

        if opname in ("return", "func.return", "stablehlo.return"):
            name = "stablehlo.return" if opname == "stablehlo.return" else "func.return"
            return Op(name, [self.ref(env, r) for r in refs])
        if short == "constant":
            t = outs[0]
            attrs = [("value", dense(re.search(r"dense<(.*)>", body).group(1), t))]
            refs = []
        elif short in ("broadcast_in_dim", "transpose"):
            key = "broadcast_dimensions" if short == "broadcast_in_dim" else "permutation"
            attrs = [(key, ("dims", _list(re.search(r"dims = \[(.*?)\]", body).group(1))))]
        elif short == "concatenate":
            attrs = [("dimension", ("int", int(re.search(r"dim = (\d+)", body).group(1)), "i64"))]
        elif short == "iota":
            attrs = [("iota_dimension", ("int", int(re.search(r"dim = (\d+)", body).group(1)), "i64"))]
        elif short == "dot_general":
            b = re.search(r"batching_dims = \[(.*?)\] x \[(.*?)\]", body)
            c = re.search(r"contracting_dims = \[(.*?)\] x \[(.*?)\]", body)
            attrs = [("lhs_batching_dimensions", ("dims", _list(b.group(1)) if b else [])),
                     ("rhs_batching_dimensions", ("dims", _list(b.group(2)) if b else [])),
                     ("lhs_contracting_dimensions", ("dims", _list(c.group(1)))),
                     ("rhs_contracting_dimensions", ("dims", _list(c.group(2))))]
            p = re.search(r"precision = \[(.*?)\]", body)
            if p:
                attrs.append(("precision_config", ("array", [("enum", "precision", ENUMS["precision"].index(x.strip()))
                                                             for x in p.group(1).split(",")])))
        elif short == "compare":
            d = re.search(r"compare\s+(\w+),", body).group(1)
            attrs = [("comparison_direction", ("enum", "comparison_direction", ENUMS["comparison_direction"].index(d)))]
            k = re.search(r",\s+(FLOAT|SIGNED|UNSIGNED|TOTALORDER|NOTYPE)\s*$", body)
            if k:
                attrs.append(("compare_type", ("enum", "comparison_type", ENUMS["comparison_type"].index(k.group(1)))))
        elif short == "reduce":
            pairs = re.findall(r"\((%[\w.$#]+) init: (%[\w.$#]+)\)", body)
            operands = [self.ref(env, a) for a, _ in pairs] + [self.ref(env, c) for _, c in pairs]
            attrs = [("dimensions", ("dims", _list(re.search(r"dimensions = \[(.*?)\]", body).group(1))))]
            inits = [v.type for v in operands[len(pairs):]]
            ap = re.search(r"applies ([\w.]+)", body)
            if ap:
                s = inits[0]
                a, b = Value(s), Value(s)
                r = Value(s)
                regions = [[([a, b], [Op(ap.group(1), [a, b], [r]), Op("stablehlo.return", [r])])]]
            else:
                head = self.lines[self.i]
                self.i += 1
                groups = re.findall(r"\(([^()]*)\)", head[len("reducer"):])
                renv = dict(env)
                lhs, rhs_args = [], []
                for g in groups:
                    (n0, t0), (n1, t1) = re.findall(r"(%[\w.$]+): (tensor<[^>]*>)", g)
                    v0, v1 = Value(parse_type(t0)), Value(parse_type(t1))
                    renv[n0], renv[n1] = v0, v1
                    lhs.append(v0)
                    rhs_args.append(v1)
                regions = [[(lhs + rhs_args, self.body(renv))]]
        elif short == "while":
            # "stablehlo.while(%iterArg = %a, ...) : types", then "cond {" ...
            # "} do {" ... "}": two regions over the loop-carried values.
            pairs = re.findall(r"(%[\w.$]+) = (%[\w.$#]+)", rest.split(")")[0])
            operands = [self.ref(env, b) for _, b in pairs]
            outs = [v.type for v in operands]
            regions = []
            for end in (("} do {",), ("}",)):
                head = self.lines[self.i]
                self.i += 1
                assert head in ("cond {", "} do {") or head.startswith("cond"), head
                renv = dict(env)
                args = [Value(v.type) for v in operands]
                for (a, _), v in zip(pairs, args):
                    renv[a] = v
                regions.append([(args, self.body(renv, end))])
                if end == ("} do {",):
                    self.i -= 1  # the "} do {" line opens the next region
        elif short == "slice":
            ranges = [r.split(":") for r in re.search(r"\[(.*?)\]", rest).group(1).split(",")]
            attrs = [("start_indices", ("dims", [int(r[0]) for r in ranges])),
                     ("limit_indices", ("dims", [int(r[1]) for r in ranges])),
                     ("strides", ("dims", [int(r[2]) if len(r) > 2 else 1 for r in ranges]))]
        elif short == "dynamic_slice":
            attrs = [("slice_sizes", ("dims", _list(re.search(r"sizes = \[(.*?)\]", body).group(1))))]
            refs = re.findall(r"%[\w.$#]+", rest.split("sizes")[0])
        elif short == "call":
            callee = re.search(r"@([\w.$]+)", body).group(1)
            attrs = [("callee", ("symbol", callee))]
            opname = "func.call"
        if operands is None:
            operands = [self.ref(env, r) for r in refs]
        if opname.startswith("stablehlo.") and short == "select":
            outs = outs[-1:]
        results = [Value(t) for t in outs[:nres]] if nres else []
        if nres > 1:
            for k, v in enumerate(results):
                env[f"{names[0]}#{k}"] = v
        elif nres == 1:
            env[names[0]] = results[0]
        return Op(opname, operands, results, attrs, regions)


def module_from_text(text):
    return _Reader(text).module()


# ------------------------------------------------------------------ writer


class Writer:
    """Serializes an op tree. `flavor` "vhlo" or "builtin"; `version` the
    bytecode version (0-6); `varint_width` forces every varint of the IR and
    of the attribute/type entries to that byte count (to cover the
    reader's wide forms); `align` puts the IR section behind an aligned
    section header."""

    VHLO_TYPES = {"i1": 0, "bf16": 2, "f16": 3, "f32": 4, "f64": 5, "index": 9, "i4": 10, "i8": 11, "i16": 12,
                  "i32": 13, "i64": 14, "ui4": 15, "ui8": 16, "ui16": 17, "ui32": 18, "ui64": 19}
    BUILTIN_FLOATS = {"bf16": 3, "f16": 4, "f32": 5, "f64": 6}

    def __init__(self, flavor="vhlo", version=1, varint_width=None, align=None, producer="StableHLO_v1.9.0"):
        assert flavor in ("vhlo", "builtin") and 0 <= version <= 6
        self.flavor, self.version, self.width, self.align, self.producer = flavor, version, varint_width, align, producer
        self.strings, self.string_ids = [], {}
        self.dialects, self.dialect_ids = [], {}
        self.opnames, self.opname_ids = [], {}
        self.attrs, self.attr_ids = [], {}  # entries: (dialect, custom, bytes)
        self.types, self.type_ids = [], {}

    # -- tables
    def v(self, x):
        if self.width is None:
            return varint(x)
        minimal = len(varint(x))
        return varint(x, 9 if self.width == 9 or minimal == 9 else max(self.width, minimal))

    def vf(self, x, flag):
        return self.v((x << 1) | int(bool(flag)))

    def sv(self, x):
        return self.v(zigzag(x))

    def string(self, s):
        if s not in self.string_ids:
            self.string_ids[s] = len(self.strings)
            self.strings.append(s)
        return self.string_ids[s]

    def dialect(self, d):
        if d not in self.dialect_ids:
            self.dialect_ids[d] = len(self.dialects)
            self.dialects.append(d)
            self.string(d)
        return self.dialect_ids[d]

    def opname(self, name):
        if self.flavor == "vhlo":
            if name == "func.func":
                name = "vhlo.func_v1"
            elif name == "func.call":
                name = "vhlo.call_v1"
            elif name in ("func.return", "stablehlo.return"):
                name = "vhlo.return_v1"
            elif name.startswith("stablehlo."):
                name = "vhlo." + name[len("stablehlo."):] + "_v1"
        d, n = name.split(".", 1)
        key = (d, n)
        if key not in self.opname_ids:
            self.opname_ids[key] = len(self.opnames)
            self.opnames.append(key)
            self.dialect(d)
            self.string(n)
        return self.opname_ids[key]

    def _entry(self, table, ids, key, dialect, build):
        if key in ids:
            return ids[key]
        idx = len(table)
        ids[key] = idx
        table.append(None)
        custom, data = build()
        table[idx] = (self.dialect(dialect), custom, data)
        return idx

    # -- types
    def type(self, t):
        return self._entry(self.types, self.type_ids, t, "vhlo" if self.flavor == "vhlo" else "builtin",
                           lambda: (True, self._type_bytes(t)))

    def _type_list(self, ts):
        return self.v(len(ts)) + b"".join(self.v(self.type(x)) for x in ts)

    def _type_bytes(self, t):
        if self.flavor == "vhlo":
            if t[0] == "scalar":
                return self.v(self.VHLO_TYPES[t[1]])
            if t[0] == "func":
                return self.v(8) + self._type_list(t[1]) + self._type_list(t[2])
            return self.v(20) + self.v(len(t[1])) + b"".join(self.sv(d) for d in t[1]) + self.v(self.type(("scalar", t[2])))
        if t[0] == "scalar":
            e = t[1]
            if e in self.BUILTIN_FLOATS:
                return self.v(self.BUILTIN_FLOATS[e])
            if e == "index":
                return self.v(1)
            sign, w = (2, int(e[2:])) if e.startswith("ui") else (0, int(e[1:]))
            return self.v(0) + self.v((w << 2) | sign)
        if t[0] == "func":
            return self.v(2) + self._type_list(t[1]) + self._type_list(t[2])
        return self.v(13) + self.v(len(t[1])) + b"".join(self.sv(d) for d in t[1]) + self.v(self.type(("scalar", t[2])))

    # -- attributes
    def builtin_string(self, s):
        return self._entry(self.attrs, self.attr_ids, ("bstr", s), "builtin",
                           lambda: (True, self.v(2) + self.v(self.string(s))))

    def unknown_loc(self):
        return self._entry(self.attrs, self.attr_ids, ("loc",), "builtin", lambda: (True, self.v(15)))

    def op_dict(self, attrs):
        key = ("opdict", repr(attrs))
        return self._entry(self.attrs, self.attr_ids, key, "builtin", lambda: (True, self.v(1) + self.v(len(attrs)) + b"".join(
            self.v(self.builtin_string(k)) + self.v(self.attr(a, k)) for k, a in attrs)))

    def _apint(self, value, bits):
        u = value & ((1 << bits) - 1)
        if bits <= 8:
            return bytes([u])
        s = u - (1 << 64) if u >= 1 << 63 else u
        return self.v(zigzag(s))

    def attr(self, a, key=""):
        dialect = "vhlo" if self.flavor == "vhlo" else ("stablehlo" if a[0] == "enum" else "builtin")
        return self._entry(self.attrs, self.attr_ids, (dialect, repr(a)), dialect, lambda: self._attr_bytes(a))

    def _attr_bytes(self, a):
        k = a[0]
        if self.flavor == "vhlo":
            if k == "str":
                return True, self.v(13) + self.v(self.string(a[1]))
            if k == "symbol":
                return True, self.v(13) + self.v(self.string(a[1]))
            if k == "int":
                return True, self.v(8) + self.v(self.type(("scalar", a[2]))) + self._apint(a[1], _ELEM_BITS[a[2]])
            if k == "float":
                return True, self.v(7) + self.v(self.type(("scalar", a[2]))) + self._apint(a[1], _ELEM_BITS[a[2]])
            if k == "bool":
                return True, self.v(1) + self.v(int(a[1]))
            if k == "elements":
                return True, self.v(14) + self.v(self.type(a[1])) + self.v(len(a[2])) + a[2]
            if k == "dims":
                t = ("tensor", (len(a[1]),), "i64")
                raw = b"".join(struct.pack("<q", d) for d in a[1])
                return True, self.v(14) + self.v(self.type(t)) + self.v(len(raw)) + raw
            if k == "array":
                return True, self.v(0) + self.v(len(a[1])) + b"".join(self.v(self.attr(x)) for x in a[1])
            if k == "type":
                return True, self.v(16) + self.v(self.type(a[1]))
            if k == "enum":
                code = {"comparison_direction": 2, "comparison_type": 3, "precision": 10}[a[1]]
                return True, self.v(code) + self.v(a[2])
            raise ValueError(a)
        if k == "str":
            return True, self.v(2) + self.v(self.string(a[1]))
        if k == "symbol":
            return True, self.v(4) + self.v(self.builtin_string(a[1]))
        if k == "int":
            return True, self.v(8) + self.v(self.type(("scalar", a[2]))) + self._apint(a[1], _ELEM_BITS[a[2]])
        if k == "float":
            return True, self.v(9) + self.v(self.type(("scalar", a[2]))) + self._apint(a[1], _ELEM_BITS[a[2]])
        if k == "elements":
            return True, self.v(18) + self.v(self.type(a[1])) + self.v(len(a[2])) + a[2]
        if k == "dims":
            raw = b"".join(struct.pack("<q", d) for d in a[1])
            return True, self.v(17) + self.v(self.type(("scalar", "i64"))) + self.v(len(a[1])) + self.v(len(raw)) + raw
        if k == "array":
            return True, self.v(0) + self.v(len(a[1])) + b"".join(self.v(self.attr(x)) for x in a[1])
        if k == "type":
            return True, self.v(6) + self.v(self.type(a[1]))
        if k == "enum":
            return False, f"#stablehlo<{a[1]} {ENUMS[a[1]][a[2]]}>".encode() + b"\x00"
        raise ValueError(a)

    # -- IR
    def _number(self, op, ids):
        """MLIR's value numbering: per isolated op from 0; a region's block
        arguments and op results in order, nested regions after its range."""
        def region(blocks, first):
            n = first
            for args, ops in blocks:
                for a in args:
                    ids[a] = n
                    n += 1
                for o in ops:
                    for r in o.results:
                        ids[r] = n
                        n += 1
            counts[id(blocks)] = n - first
            for _, ops in blocks:
                for o in ops:
                    for reg in o.regions:
                        region(reg, 0 if o.isolated else n)
        counts = {}
        for reg in op.regions:
            region(reg, 0)
        return counts

    def _op(self, op, ids, counts):
        name = op.name
        if self.flavor == "vhlo" and op.name == "func.func":
            attrs = list(op.attrs)
            if not any(k == "sym_visibility" for k, _ in attrs):
                attrs.append(("sym_visibility", ("str", "")))
            attrs += [("arg_attrs", ("array", [])), ("res_attrs", ("array", []))]
        elif op.name == "builtin.module":
            attrs = []
        else:
            attrs = op.attrs
        out = self.v(self.opname(name))
        mask = 0
        body = self.v(self.unknown_loc())
        if op.name == "builtin.module" and op.attrs:
            key = ("moddict", repr(op.attrs))
            idx = self._entry(self.attrs, self.attr_ids, key, "builtin", lambda: (True, self.v(1) + self.v(1) + self.v(
                self.builtin_string("sym_name")) + self.v(self.builtin_string(op.attrs[0][1][1]))))
            mask |= 1
            body += self.v(idx)
        elif attrs:
            mask |= 1
            body += self.v(self.op_dict(attrs))
        if op.results:
            mask |= 2
            body += self.v(len(op.results)) + b"".join(self.v(self.type(r.type)) for r in op.results)
        if op.operands:
            mask |= 4
            body += self.v(len(op.operands)) + b"".join(self.v(ids[o]) for o in op.operands)
        if op.regions:
            mask |= 16
            inner = b"".join(self._region(reg, ids, counts) for reg in op.regions)
            body += self.vf(len(op.regions), op.isolated)
            if op.isolated and self.version >= 2:
                body += self._section(4, inner)
            else:
                body += inner
        return out + bytes([mask]) + body

    def _region(self, blocks, ids, counts):
        if not blocks:
            return self.v(0)
        out = self.v(len(blocks)) + self.v(counts[id(blocks)])
        for args, ops in blocks:
            out += self.vf(len(ops), bool(args))
            if args:
                out += self.v(len(args))
                for a in args:
                    if self.version >= 4:
                        out += self.vf(self.type(a.type), True) + self.v(self.unknown_loc())
                    else:
                        out += self.v(self.type(a.type)) + self.v(self.unknown_loc())
                if self.version >= 3:
                    out += b"\x00"
            for o in ops:
                out += self._op(o, ids, counts)
        return out

    def _section(self, sid, payload, align=None, offset=0):
        if align is None:
            return bytes([sid]) + varint(len(payload)) + payload
        head = bytes([sid | 0x80]) + varint(len(payload)) + varint(align)
        pad = (-(offset + len(head))) % align
        return head + b"\xCB" * pad + payload

    def write(self, module):
        # Op names are numbered dialect by dialect, so that each dialect's
        # names form one group of the dialect section.
        first = []
        for o in _walk(module):
            probe = Writer(self.flavor, self.version)
            probe.opname(o.name)
            if probe.opnames[0] not in first:
                first.append(probe.opnames[0])
        order = []
        for d, _ in first:
            if d not in order:
                order.append(d)
        for key in sorted(first, key=lambda k: (order.index(k[0]), first.index(k))):
            self.opname_ids[key] = len(self.opnames)
            self.opnames.append(key)
            self.dialect(key[0])
            self.string(key[1])
        ids = {}
        counts = self._number(module, ids)
        ir = self.vf(1, False) + self._op(module, ids, counts)
        # Dialect section.
        d = self.v(len(self.dialects))
        for name in self.dialects:
            if self.version >= 1:
                has_version = self.flavor == "vhlo" and name == "vhlo"
                d += self.vf(self.string_ids[name], has_version)
                if has_version:
                    d += self._section(7, varint(1) + varint(9) + varint(0))
            else:
                d += self.v(self.string_ids[name])
        if self.version >= 4:
            d += self.v(len(self.opnames))
        for di, dname in enumerate(self.dialects):
            names = [n for (dd, n) in self.opnames if dd == dname]
            if not names:
                continue
            d += self.v(di) + self.v(len(names))
            for n in names:
                s = self.string_ids[n]
                d += self.vf(s, True) if self.version >= 5 else self.v(s)
        # Attribute / type sections.
        off = self.v(len(self.attrs)) + self.v(len(self.types))
        data = b""
        for table in (self.attrs, self.types):
            i = 0
            while i < len(table):
                j = i
                while j < len(table) and table[j][0] == table[i][0]:
                    j += 1
                off += self.v(table[i][0]) + self.v(j - i)
                for di, custom, payload in table[i:j]:
                    off += self.vf(len(payload), custom)
                    data += payload
                i = j
        # String section: sizes from the last string to the first.
        s = varint(len(self.strings))
        for st in reversed(self.strings):
            s += varint(len(st.encode()) + 1)
        s += b"".join(st.encode() + b"\x00" for st in self.strings)
        out = b"ML\xefR" + varint(self.version) + self.producer.encode() + b"\x00"
        out += self._section(1, d)
        out += self._section(3, off) + self._section(2, data)
        out += self._section(4, ir, self.align, len(out))
        out += self._section(0, s)
        if self.version >= 5:
            out += self._section(8, varint(0))
        return out


def _walk(op):
    yield op
    for reg in op.regions:
        for _, ops in reg:
            for o in ops:
                yield from _walk(o)


def to_bytecode(text, flavor="vhlo", version=1, varint_width=None, align=None):
    """StableHLO text (mi355x.programs forms) -> MLIR bytecode."""
    return Writer(flavor, version, varint_width, align).write(module_from_text(text))
