// Fused elementwise emitter (ew_jit.cpp): hiprtc-compiled straight-line
// kernels for mk_ew_instr programs, cached per device and program.
#pragma once

#include <stdint.h>

#include <string>
#include <vector>

#include "../../include/mk_kernels.h"

namespace mkc {

// Generated HIP source for a program (exposed for inspection and tests).
std::string ew_jit_source(int dtype, const mk_ew_instr* prog, int n_instr, int n_inputs, int out_slot);

// Compiled kernel (hipFunction_t) for a validated program on the current
// device, compiling and loading it on first use.  Returns MK_OK or an MK_E*
// code with the message recorded for mk_last_error().
int ew_jit_get(int dtype, const mk_ew_instr* prog, int n_instr, int n_inputs, int out_slot, void** fn_out);

// Source and code object of a validated program (compiled, or taken from the
// memory or disk cache); needs no device.
int ew_jit_code(int dtype, const mk_ew_instr* prog, int n_instr, int n_inputs, int out_slot, std::string* source,
                std::vector<char>* code);

// Everything a code object depends on besides its source: the hiprtc
// version and the compile options.  A serialized executable records it, and
// its code objects are reused only when it matches.
const std::string& ew_jit_tag();

// Adds a code object for a source to the in-memory cache (a deserialized
// executable's, built under the same tag), so its first launch loads it
// instead of compiling.  A seeded object that fails to load is dropped and
// the source compiled again.
void ew_jit_seed(const std::string& source, const std::vector<char>& code);

// Process totals: hiprtc compiles, disk-cache hits, memory-cache hits.
void ew_jit_stats(int64_t* compiles, int64_t* disk_hits, int64_t* mem_hits);

// The library's on-disk cache directory (MK_CACHE_DIR, default
// $HOME/.cache/mi355x-mk, created when missing); "" when
// MK_DISABLE_CACHE_PERSIST is set or the directory is unusable.
std::string cache_directory();

}  // namespace mkc
