"""The MLIR-bytecode front end (csrc/runtime/mlir_bytecode.cpp) on the CPU.

jaxlib's PJRT client hands PJRT_Client_Compile a StableHLO portable
artifact: MLIR bytecode of the vhlo dialect
(/root/reference/src/pjrt_plugin/api/pjrt_client.cc:178-244). The reference
reads it with StableHLO's deserializePortableArtifact
(core/stablehlo_parser.mm:568-586). This build decodes it itself.

jax is not installed and the pinned StableHLO is absent, so no artifact
written by jax's emitter is available. The checks are, in order:

* the test writer's varints against the published prefix-varint table;
* a file assembled byte by byte in this test from the format description,
  decoded to an exact expected text;
* every program the workload compiles, written by the test writer
  (tests/_bytecode.py) as a vhlo artifact and as a builtin-dialect module,
  at bytecode versions 0-6, with forced wide varints and aligned sections,
  must plan exactly as its text form;
* malformed and unsupported inputs fail with INVALID_ARGUMENT /
  UNIMPLEMENTED. Truncations and byte flips of the same files run under
  AddressSanitizer in tests/test_pjrt_cpu.py.
"""

import pytest

import _bytecode as B
from mi355x import programs as P
from mi355x import runtime as rt
from test_pjrt_cpu import _corpus

INVALID_ARGUMENT, UNIMPLEMENTED = 3, 12


# ------------------------------------------------------------------ varints


@pytest.mark.parametrize("nbytes", range(1, 10))
def test_varint_prefix_table(nbytes):
    """MLIR's table: 1-8 bytes carry 7n bits, the first byte ending in a one
    bit after n-1 zero bits; 9 bytes are a zero byte and the 64-bit value."""
    lo = 0 if nbytes == 1 else 1 << (7 * (nbytes - 1))
    hi = (1 << 64) - 1 if nbytes == 9 else (1 << (7 * nbytes)) - 1
    for v in (lo, hi, (lo + hi) // 2):
        e = B.varint(v)
        assert len(e) == nbytes
        if nbytes == 9:
            assert e[0] == 0 and int.from_bytes(e[1:], "little") == v
        else:
            assert e[0] & ((1 << nbytes) - 1) == 1 << (nbytes - 1)
            assert int.from_bytes(e, "little") >> nbytes == v


def test_varint_literals():
    assert B.varint(0) == b"\x01"
    assert B.varint(1) == b"\x03"
    assert B.varint(127) == b"\xff"
    assert B.varint(128) == b"\x02\x02"
    assert B.varint(16383) == b"\xfe\xff"
    assert B.varint(5, 3) == bytes([(5 << 3 | 4) & 0xFF, 0, 0])
    assert [B.zigzag(x) for x in (0, -1, 1, -2, 2)] == [0, 1, 2, 3, 4]
    assert B.zigzag(-(1 << 63)) == (1 << 64) - 1


# ---------------------------------------------------------- hand-assembled


def _v(x):
    return B.varint(x)


def _hand_assembled():
    """A vhlo artifact, bytecode version 1:
        module @m { vhlo.func_v1 @main(%a: tensor<4xf32>) -> tensor<4xf32> {
                      %0 = vhlo.negate_v1 %a; vhlo.return_v1 %0 } }
    Every byte is spelled out here from the format, not by the writer."""
    strings = ["builtin", "vhlo", "module", "func_v1", "negate_v1", "return_v1", "sym_name", "main",
               "function_type", "m"]
    # Dialects: 0 builtin, 1 vhlo.  Op names: 0 builtin.module, 1
    # vhlo.func_v1, 2 vhlo.negate_v1, 3 vhlo.return_v1.
    dialect = (bytes([0x05,              # 2 dialects
                      0x01,              # builtin: string 0 << 1 | no version
                      0x05,              # vhlo: string 1 << 1 | no version
                      0x01, 0x03, 0x05,  # group builtin, 1 name: "module"
                      0x03, 0x07, 0x07, 0x09, 0x0B]))  # group vhlo, 3 names: 3, 4, 5
    types = [bytes([0x09]),                    # T0 vhlo f32 (code 4)
             bytes([0x29, 0x03, 0x11, 0x01]),  # T1 vhlo ranked tensor (20): rank 1, zigzag(4), T0
             bytes([0x11, 0x03, 0x03, 0x03, 0x03])]  # T2 vhlo function (8): (T1) -> (T1)
    attrs = [bytes([0x1F]),                     # A0 builtin unknown location (15)
             bytes([0x05, 0x0D]),               # A1 builtin string (2) "sym_name"
             bytes([0x05, 0x13]),               # A2 builtin string "m"
             bytes([0x03, 0x03, 0x03, 0x05]),   # A3 builtin dictionary (1): {A1 = A2}
             bytes([0x1B, 0x0F]),               # A4 vhlo string (13) "main"
             bytes([0x05, 0x11]),               # A5 builtin string "function_type"
             bytes([0x21, 0x05]),               # A6 vhlo type attribute (16): T2
             bytes([0x03, 0x05, 0x03, 0x09, 0x0B, 0x0D])]  # A7 dictionary {A1 = A4, A5 = A6}
    groups = [(0, [0, 1, 2, 3]), (1, [4]), (0, [5]), (1, [6]), (0, [7])]
    offsets = bytes([0x11, 0x07])  # 8 attributes, 3 types
    for d, idx in groups:
        offsets += _v(d) + _v(len(idx)) + b"".join(_v(len(attrs[i]) << 1 | 1) for i in idx)
    offsets += _v(1) + _v(3) + b"".join(_v(len(t) << 1 | 1) for t in types)
    data = b"".join(attrs) + b"".join(types)
    ir = bytes([
        0x05,                    # top block: 1 op, no arguments
        0x01, 0x11, 0x01, 0x07,  # builtin.module: attrs|regions, loc A0, attrs A3
        0x07,                    # 1 region << 1 | isolated
        0x03, 0x01,              # 1 block, 0 values
        0x05,                    # 1 op, no arguments
        0x03, 0x11, 0x01, 0x0F,  # vhlo.func_v1: attrs|regions, loc A0, attrs A7
        0x07,                    # 1 region << 1 | isolated (inline before version 2)
        0x03, 0x05,              # 1 block, 2 values
        0x0B, 0x03, 0x03, 0x01,  # 2 ops, arguments: 1 (type T1, loc A0)
        0x05, 0x06, 0x01, 0x03, 0x03, 0x03, 0x01,  # negate: results|operands, loc, 1 x T1, 1 x value 0
        0x07, 0x04, 0x01, 0x03, 0x03,              # return: operands, loc, 1 x value 1
    ])
    s = _v(len(strings)) + b"".join(_v(len(x) + 1) for x in reversed(strings))
    s += b"".join(x.encode() + b"\x00" for x in strings)

    def section(i, payload):
        return bytes([i]) + _v(len(payload)) + payload
    return (b"ML\xefR" + _v(1) + b"hand\x00" + section(1, dialect) + section(3, offsets) + section(2, data) +
            section(4, ir) + section(0, s))


HAND_TEXT = ('module @m {\n'
             'func.func public @main(%v0: tensor<4xf32>) -> (tensor<4xf32>) {\n'
             '%v1 = "stablehlo.negate"(%v0) : (tensor<4xf32>) -> tensor<4xf32>\n'
             '"func.return"(%v1) : (tensor<4xf32>) -> ()\n'
             '}\n'
             '}\n')


def test_hand_assembled_artifact_decodes_exactly():
    assert rt.bytecode_to_text(_hand_assembled()) == HAND_TEXT


def test_hand_assembled_artifact_plans_like_its_text():
    text = ("module @m {\n  func.func public @main(%arg0: tensor<4xf32>) -> (tensor<4xf32>) {\n"
            "    %0 = stablehlo.negate %arg0 : tensor<4xf32>\n    return %0 : tensor<4xf32>\n  }\n}\n")
    assert rt.compile_check(_hand_assembled()) == rt.compile_check(text)


def test_writer_matches_the_hand_assembled_layout():
    """The writer's output for the same module decodes to the same text."""
    text = ("module @m {\n  func.func public @main(%arg0: tensor<4xf32>) -> (tensor<4xf32>) {\n"
            "    %0 = stablehlo.negate %arg0 : tensor<4xf32>\n    return %0 : tensor<4xf32>\n  }\n}\n")
    assert rt.bytecode_to_text(B.to_bytecode(text, "vhlo", 1)) == HAND_TEXT


# ------------------------------------------------------------- round trips

CORPUS = _corpus()


@pytest.mark.parametrize("version", range(7))
@pytest.mark.parametrize("flavor", ["vhlo", "builtin"])
@pytest.mark.parametrize("name", sorted(CORPUS))
def test_corpus_plans_identically_from_bytecode(name, flavor, version):
    text = CORPUS[name]
    assert rt.compile_check(B.to_bytecode(text, flavor, version)) == rt.compile_check(text)


@pytest.mark.parametrize("width", [2, 3, 5, 8, 9])
def test_wide_varints(width):
    for name in ("argmax", "int4", "softmax_bf16", "bmm"):
        text = CORPUS[name]
        bc = B.to_bytecode(text, "vhlo", 6, varint_width=width)
        assert rt.compile_check(bc) == rt.compile_check(text), name


@pytest.mark.parametrize("align", [8, 64, 4096])
def test_aligned_ir_section(align):
    text = CORPUS["rmsnorm_bf16"]
    bc = B.to_bytecode(text, "vhlo", 2, align=align)
    assert rt.compile_check(bc) == rt.compile_check(text)


def test_full_size_workload_programs():
    """The benchmark's own shapes (dimensions need multi-byte varints)."""
    for text in (P.int4_g64_matmul(16, 4096, 14336), P.int8_pc_matmul(16, 4096, 14336),
                 P.matmul(4096, 4096, 4096), P.softmax(8192, 8192, "bf16"), P.argmax(8192, 8192),
                 P.chain6(8192, 8192), P.rmsnorm(8192, 8192)):
        assert rt.compile_check(B.to_bytecode(text)) == rt.compile_check(text)


def test_decoded_constants_are_bit_exact():
    """Constants travel as raw element bytes: the decoded text carries the
    exact f32 / bf16 / integer bit patterns."""
    t = rt.bytecode_to_text(B.to_bytecode(P.softmax(4, 8, "bf16")))
    assert 'dense<"0x80FF"> : tensor<bf16>' in t            # -inf, little-endian
    t = rt.bytecode_to_text(B.to_bytecode(P.int4_g64_matmul(16, 128, 64)))
    assert 'dense<"0x0F"> : tensor<ui8>' in t and 'dense<"0x04"> : tensor<ui8>' in t
    t = rt.bytecode_to_text(B.to_bytecode(P.chain6(4, 8)))
    assert 'dense<"0x0000C03F"> : tensor<f32>' in t          # 1.5


def test_optimized_program_of_a_bytecode_program_is_its_text():
    from mi355x import runtime as r
    bc = B.to_bytecode(CORPUS["softmax"])
    text = r.bytecode_to_text(bc)
    assert text.startswith("module @jit_softmax {") and '"stablehlo.reduce"' in text


# ------------------------------------------------------------------ errors


def _code(blob):
    with pytest.raises(rt.PluginError) as e:
        rt.compile_check(blob)
    return e.value.code


def test_truncated_files_are_invalid_argument():
    bc = _hand_assembled()
    for cut in range(4, len(bc)):
        assert _code(bc[:cut]) == INVALID_ARGUMENT, cut


def test_unknown_version_is_unimplemented():
    bc = bytearray(_hand_assembled())
    bc[4] = B.varint(7)[0]
    assert _code(bytes(bc)) == UNIMPLEMENTED


def test_other_dialects_binary_encoding_is_unimplemented():
    bc = B.to_bytecode(CORPUS["softmax"])
    assert bc.count(b"vhlo\x00") == 1
    with pytest.raises(rt.PluginError) as e:
        rt.compile_check(bc.replace(b"vhlo\x00", b"vhlx\x00"))
    assert e.value.code == UNIMPLEMENTED and "vhlx" in str(e.value)


def test_operand_past_the_defined_values_is_invalid_argument():
    bc = bytearray(_hand_assembled())
    # The return's operand (value 1, 0x03) -> value 2, one past the region.
    k = bc.rindex(bytes([0x07, 0x04, 0x01, 0x03, 0x03]))
    bc[k + 4] = 0x05
    assert _code(bytes(bc)) == INVALID_ARGUMENT


def test_self_referential_entry_is_invalid_argument():
    bc = bytearray(_hand_assembled())
    # A3 = {A1 = A2} -> {A1 = A3}: a dictionary containing itself.
    k = bc.index(bytes([0x03, 0x03, 0x03, 0x05]))
    bc[k + 3] = 0x07
    assert _code(bytes(bc)) == INVALID_ARGUMENT


def test_section_twice_is_invalid_argument():
    bc = _hand_assembled()
    assert _code(bc + bytes([0x00, 0x01, 0x01])) == INVALID_ARGUMENT
