// Host-side C ABI helpers: error reporting and version.
#include <cstdarg>
#include <cstdio>

#include "common.h"

namespace oscar {

static thread_local char g_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return code;
}

}  // namespace oscar

extern "C" const char* oscar_last_error(void) { return oscar::g_error; }
extern "C" int oscar_abi_version(void) { return OSCAR_ABI_VERSION; }
