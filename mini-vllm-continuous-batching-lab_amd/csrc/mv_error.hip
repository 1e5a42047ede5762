// Thread-local last-error string and the small ABI queries.
#include <stdarg.h>
#include <stdio.h>

#include "mv_common.h"

namespace {
thread_local char g_last_error[512] = "";
}

namespace mv {

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    return fail(MV_ERR_HIP, "%s: kernel launch failed: %s", what, hipGetErrorString(err));
  }
  return MV_OK;
}

}  // namespace mv

extern "C" int mv_abi_version(void) { return MVATTN_ABI_VERSION; }

extern "C" const char* mv_last_error(void) { return g_last_error; }
