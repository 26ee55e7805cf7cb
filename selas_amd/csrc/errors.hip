// Error reporting for the C ABI: a per-thread message behind selas_last_error().
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace {
thread_local char g_msg[512] = "";
}

namespace selas {

int set_error(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_msg, sizeof(g_msg), fmt, ap);
  va_end(ap);
  return code;
}

int ok() {
  g_msg[0] = '\0';
  return SELAS_OK;
}

int check_launch(const char *what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(SELAS_EHIP, "%s: launch failed: %s", what, hipGetErrorString(e));
  return ok();
}

}  // namespace selas

extern "C" const char *selas_last_error(void) { return g_msg; }

extern "C" int selas_abi_version(void) { return 6; }
