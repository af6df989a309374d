// Library-wide C-ABI plumbing: version, the thread-local error message and launch checks.

#include <stdarg.h>
#include <stdio.h>

#include "gdn_common.h"

static thread_local char g_last_error[512] = "";

extern "C" void gdn_internal_set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

extern "C" int gdn_internal_check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    gdn_internal_set_error("%s launch failed: %s", what, hipGetErrorString(e));
    return GDN_ERR_HIP;
  }
  return GDN_OK;
}

extern "C" int gdn_abi_version(void) { return GDN_ABI_VERSION; }

extern "C" const char* gdn_last_error(void) { return g_last_error; }
