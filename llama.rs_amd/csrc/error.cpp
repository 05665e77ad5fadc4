// The thread-local error text behind llrs_last_error() (host only).
#include <cstdarg>
#include <cstdio>

#include "common.h"

namespace llrs {

static thread_local char g_error[1024];

int set_error(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof g_error, fmt, ap);
  va_end(ap);
  return code;
}
void clear_error() { g_error[0] = 0; }

}  // namespace llrs

extern "C" const char *llrs_last_error(void) { return llrs::g_error; }
