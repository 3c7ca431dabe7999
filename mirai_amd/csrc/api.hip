// Error reporting and version of the C-ABI.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace mx {

static thread_local char g_error[1024] = "";

void set_error(const char *fmt, ...) {
  va_list args;
  va_start(args, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, args);
  va_end(args);
}

void clear_error() { g_error[0] = '\0'; }

int check_launch(const char *what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    set_error("%s: %s", what, hipGetErrorString(err));
    return MX_ERR_HIP;
  }
  return MX_OK;
}

}  // namespace mx

extern "C" const char *mx_last_error(void) { return mx::g_error; }

extern "C" int mx_abi_version(void) { return 9; }
