// Library-wide C-ABI plumbing: version and thread-local last error.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace mls {

static thread_local char g_last_error[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(MLS_ERR_HIP, "%s: launch failed: %s", what, hipGetErrorString(e));
  return MLS_OK;
}

}  // namespace mls

extern "C" int mls_abi_version(void) { return MLS_ABI_VERSION; }

extern "C" const char* mls_last_error(void) { return mls::g_last_error; }
