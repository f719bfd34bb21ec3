// Error reporting and version entry points of the C ABI.
#include <string>

#include "common.h"

namespace dwm {

static thread_local std::string g_last_error;

void set_error(const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
}

void clear_error() { g_last_error.clear(); }

int launch_status(const char *what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: kernel launch failed: %s", what, hipGetErrorString(e));
    return DWM_ERR_HIP;
  }
  return DWM_OK;
}

}  // namespace dwm

extern "C" int dwm_version(void) { return 100; }

extern "C" const char *dwm_last_error(void) { return dwm::g_last_error.c_str(); }
