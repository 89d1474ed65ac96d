// Library-wide entry points of the kernel C-ABI (include/mk_kernels.h).
#include "../../include/mk_kernels.h"
#include "capi_internal.h"

namespace mkc {

char* error_buffer() {
  static thread_local char buf[512] = {0};
  return buf;
}

}  // namespace mkc

extern "C" const char* mk_last_error(void) { return mkc::error_buffer(); }

extern "C" const char* mk_version(void) { return "mk-gfx950 0.1"; }
