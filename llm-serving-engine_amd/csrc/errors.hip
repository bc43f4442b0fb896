// Error reporting of the C ABI: a thread-local message for the last failed call.
#include <cstdarg>
#include <cstdio>

#include "common.h"

namespace {
thread_local char g_msg[512] = "";
thread_local lsh::TimingEvents g_timing;
}

namespace lsh {

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_msg, sizeof(g_msg), fmt, ap);
  va_end(ap);
}

TimingEvents& timing_events() { return g_timing; }

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

extern "C" int llmserve_time_next_call(void* start_event, void* stop_event) {
  g_timing.start = static_cast<hipEvent_t>(start_event);
  g_timing.stop = static_cast<hipEvent_t>(stop_event);
  return LLMSERVE_OK;
}
