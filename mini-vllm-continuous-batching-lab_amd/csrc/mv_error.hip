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

extern "C" int mv_stream_capture_id(void* stream, uint64_t* capture_id) {
  if (!capture_id) return mv::fail(MV_ERR_INVALID_ARGUMENT, "mv_stream_capture_id: null capture_id");
  hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
  unsigned long long id = 0;
  const hipError_t err = hipStreamGetCaptureInfo(static_cast<hipStream_t>(stream), &status, &id);
  if (err != hipSuccess)
    return mv::fail(MV_ERR_HIP, "mv_stream_capture_id: %s", hipGetErrorString(err));
  *capture_id = status == hipStreamCaptureStatusActive ? static_cast<uint64_t>(id) : 0;
  return MV_OK;
}
