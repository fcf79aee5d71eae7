// Library-wide host plumbing: thread-local error string and version query.
#include "mtx_common.h"

#include <cstdarg>
#include <cstdio>

namespace mtx {

static thread_local char g_err[1024] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

}  // namespace mtx

extern "C" const char* mtx_last_error(void) { return mtx::g_err; }

extern "C" const char* mtx_version(void) { return "minitorch_amd 0.1 (gfx950)"; }
