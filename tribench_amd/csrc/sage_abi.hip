// sage_abi.hip — version query and error reporting of the C ABI.
#include <stdarg.h>
#include <stdio.h>

#include "sage_device.h"

namespace sage {

static thread_local char g_last_error[512] = "";

int fail(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return 1;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail("%s: kernel launch failed: %s", what, hipGetErrorString(e));
  return 0;
}

}  // namespace sage

extern "C" int sage_abi_version(void) { return SAGE_ABI_VERSION; }

extern "C" const char* sage_last_error(void) { return sage::g_last_error; }
