// MLIR bytecode reader: the binary module jax's PJRT client hands to
// PJRT_Client_Compile (a StableHLO portable artifact, i.e. MLIR bytecode of
// the vhlo dialect), turned back into MLIR text for the StableHLO text
// reader.  Replaces the reference's deserializePortableArtifact + print
// (core/stablehlo_parser.mm:568-586, bytecodeToText :597).
#pragma once

#include <stddef.h>

#include <stdexcept>
#include <string>

namespace mkrt {

// MALFORMED: the bytes break the bytecode format (INVALID_ARGUMENT at
// compile).  UNSUPPORTED: well-formed content this reader does not decode
// (UNIMPLEMENTED at compile), e.g. a dialect's binary attribute encoding
// other than builtin's and vhlo's.
struct BytecodeError : std::runtime_error {
  enum Kind { MALFORMED, UNSUPPORTED };
  Kind kind;
  BytecodeError(Kind k, const std::string& m) : std::runtime_error(m), kind(k) {}
};

// True when `data` starts with the MLIR bytecode magic "ML\xefR".
bool is_mlir_bytecode(const char* data, size_t size);

// The module as MLIR text: `module`, `func.func` headers in the pretty form,
// every other op in the generic form ("stablehlo.add"(%a, %b) {attrs} :
// (types) -> type), vhlo ops under their stablehlo / func names.  Throws
// BytecodeError.
std::string mlir_bytecode_to_text(const char* data, size_t size);

}  // namespace mkrt
