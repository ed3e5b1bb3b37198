// C-ABI plumbing shared by every entry point: thread-local error text and the
// launch-status check.
#include <stdarg.h>

#include "common.h"

namespace moe {

namespace {
thread_local char g_last_error[512] = "";
}

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

int launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: kernel launch failed: %s", what, hipGetErrorString(e));
    return MOE_ERR_LAUNCH;
  }
  return MOE_OK;
}

}  // namespace moe

extern "C" const char* moe_last_error(void) { return moe::g_last_error; }

extern "C" int moe_abi_version(void) { return 1; }
