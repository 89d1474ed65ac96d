// Fused elementwise emitter (ew_jit.cpp): hiprtc-compiled straight-line
// kernels for mk_ew_instr programs, cached per device and program.
#pragma once

#include <string>

#include "../../include/mk_kernels.h"

namespace mkc {

// Generated HIP source for a program (exposed for inspection and tests).
std::string ew_jit_source(int dtype, const mk_ew_instr* prog, int n_instr, int n_inputs, int out_slot);

// Compiled kernel (hipFunction_t) for a validated program on the current
// device, compiling and loading it on first use.  Returns MK_OK or an MK_E*
// code with the message recorded for mk_last_error().
int ew_jit_get(int dtype, const mk_ew_instr* prog, int n_instr, int n_inputs, int out_slot, void** fn_out);

}  // namespace mkc
