// C-ABI plumbing shared by every q3attn entry point: per-thread error message and ABI version.
#include <stdarg.h>
#include <stdio.h>

#include "q3a_common.h"
#include "../../include/q3attn.h"

namespace {
thread_local char g_last_error[512] = {0};
}

namespace q3a {
int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}
}  // namespace q3a

extern "C" int q3a_abi_version(void) { return Q3A_ABI_VERSION; }

extern "C" const char* q3a_last_error(void) { return g_last_error; }
