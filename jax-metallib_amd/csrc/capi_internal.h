// Host-side helpers shared by the extern "C" launchers: the thread-local
// error message behind mk_last_error().
#pragma once

#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>

namespace mkc {

char* error_buffer();

inline void clear_error() { error_buffer()[0] = '\0'; }

// Record a formatted message for mk_last_error() and return `code`.
inline int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(error_buffer(), 512, fmt, ap);
  va_end(ap);
  return code;
}

}  // namespace mkc
