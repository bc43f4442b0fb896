// Error reporting of the C ABI: a thread-local message for the last failed call.
#include <cstdarg>
#include <cstdio>

#include "common.h"

namespace {
thread_local char g_msg[512] = "";
}

namespace lsh {

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_msg, sizeof(g_msg), fmt, ap);
  va_end(ap);
}

int launch_status(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return LLMSERVE_ERR_HIP;
  }
  return LLMSERVE_OK;
}

}  // namespace lsh

extern "C" const char* llmserve_last_error(void) { return g_msg; }

extern "C" int llmserve_abi_version(void) { return 1; }
