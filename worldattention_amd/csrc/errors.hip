// Error reporting shared by every entry point (wa_last_error / wa_version).
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

static thread_local char g_last_error[512] = "";

void wa_set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

int wa_fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int wa_launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return wa_fail((int)e, "%s launch failed: %s", what, hipGetErrorString(e));
  return WA_OK;
}

extern "C" int wa_version(void) { return 100; }

extern "C" const char* wa_last_error(void) { return g_last_error; }
