// Version, per-thread error text and launch checks of the C ABI.
#include "cab_internal.h"

namespace cab {

static thread_local std::string g_last_error;

void set_error(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
}

void clear_error() { g_last_error.clear(); }

cab_status_t launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return CAB_EHIP;
  }
  return CAB_OK;
}

}  // namespace cab

extern "C" int cab_abi_version(void) { return CAB_ABI_VERSION; }

extern "C" const char* cab_last_error(void) { return cab::g_last_error.c_str(); }
