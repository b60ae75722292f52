// Error reporting shared by every C-ABI entry point.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace aspec {

static thread_local char g_last_error[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list args;
  va_start(args, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, args);
  va_end(args);
  return code;
}

int check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    return set_error(ASPEC_ERR_RUNTIME, "%s: kernel launch failed: %s", what, hipGetErrorString(err));
  }
  return ASPEC_OK;
}

}  // namespace aspec

extern "C" int aspec_abi_version(void) { return 15; }

extern "C" const char* aspec_last_error(void) { return aspec::g_last_error; }
