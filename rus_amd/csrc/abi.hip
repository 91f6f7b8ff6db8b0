// Error reporting shared by every C-ABI entry point (include/rus_amd.h).
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace rus {

static thread_local char g_error[1024] = {0};

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_error[0] = 0; }

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    return fail(RUS_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  }
  return RUS_OK;
}

}  // namespace rus

extern "C" const char* rus_last_error(void) { return rus::g_error; }

extern "C" int rus_abi_version(void) { return RUS_ABI_VERSION; }
