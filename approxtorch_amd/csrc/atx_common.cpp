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

}  // namespace atx

extern "C" {
const char* atx_last_error(void) { return atx::g_err; }
int atx_version(void) { return ATX_ABI_VERSION; }
}
