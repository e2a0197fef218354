// Error reporting shared by the C ABI entry points (see include/fa4cp.h).
#include <cstdarg>
#include <cstdio>

#include "common.h"

namespace fa4cp {

static thread_local char g_last_error[512] = {0};

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_last_error[0] = '\0'; }

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return set_error(FA4CP_ELAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return FA4CP_OK;
}

}  // namespace fa4cp

extern "C" const char* fa4cp_last_error(void) { return fa4cp::g_last_error; }

extern "C" int fa4cp_abi_version(void) { return FA4CP_ABI_VERSION; }
