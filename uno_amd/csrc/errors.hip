// Thread-local error reporting for the C-ABI (see common.h for the return convention).
#include "common.h"

namespace unok {

static thread_local char g_last_error[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

const char* last_error() { return g_last_error; }

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    return set_error((int)e, "%s: launch failed: %s", what, hipGetErrorString(e));
  }
  return 0;
}

}  // namespace unok

UNOK_EXPORT const char* unok_last_error() { return unok::last_error(); }

UNOK_EXPORT int unok_abi_version() { return 1; }
