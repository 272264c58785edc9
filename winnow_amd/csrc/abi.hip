// Version, error reporting and split planning of the C ABI.
#include <cstdarg>

#include "wn_common.h"

namespace wn {

namespace {
thread_local std::string g_last_error;
}

void set_error(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
}

void clear_error() { g_last_error.clear(); }

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: %s", what, hipGetErrorString(e));
    return WN_E_LAUNCH;
  }
  return WN_OK;
}

}  // namespace wn

extern "C" int wn_abi_version(void) { return WN_ABI_VERSION; }

extern "C" const char* wn_last_error(void) { return wn::g_last_error.c_str(); }
