// Error reporting and version for the LeanSelect HIP library.
#include <stdarg.h>
#include <stdio.h>

#include "ls_common.h"

static thread_local char g_last_error[1024] = "";

int ls_fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int ls_check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return ls_fail(LS_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  return LS_OK;
}

extern "C" int ls_version(void) { return 100; }

extern "C" const char* ls_last_error(void) { return g_last_error; }
