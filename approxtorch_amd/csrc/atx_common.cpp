// Error reporting shared by every entry point of libatx.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>

#include "../../include/atx.h"

namespace atx {

static thread_local char g_err[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return set_error(ATX_ELAUNCH, "%s: %s", what, hipGetErrorString(e));
  return ATX_OK;
}

// atx_set_timing_events: the pair recorded around the LUT GEMMs' main kernel.
static thread_local hipEvent_t g_ev_before = nullptr, g_ev_after = nullptr;

int timing_mark(bool after, hipStream_t stream) {
  const hipEvent_t ev = after ? g_ev_after : g_ev_before;
  if (ev == nullptr) return ATX_OK;
  const hipError_t e = hipEventRecord(ev, stream);
  if (e != hipSuccess)
    return set_error(ATX_ELAUNCH, "hipEventRecord (timing event): %s", hipGetErrorString(e));
  return ATX_OK;
}

}  // namespace atx

extern "C" {
const char* atx_last_error(void) { return atx::g_err; }
int atx_version(void) { return ATX_ABI_VERSION; }
int atx_set_timing_events(hipEvent_t before, hipEvent_t after) {
  if ((before == nullptr) != (after == nullptr))
    return atx::set_error(ATX_EINVAL, "atx_set_timing_events: pass both events or neither");
  atx::g_ev_before = before;
  atx::g_ev_after = after;
  return ATX_OK;
}
}
