// Error reporting shared by every entry point of libtai_kernels.so.
#include <stdarg.h>

#include "common.h"

namespace tai {

static thread_local char g_last_error[512] = "";

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
    return TAI_ERR_LAUNCH;
  }
  return TAI_OK;
}

}  // namespace tai

extern "C" const char* tai_last_error(void) { return tai::g_last_error; }
extern "C" int tai_abi_version(void) { return 1; }

#ifndef TAI_BUILD_ID
#define TAI_BUILD_ID "unversioned"
#endif
// Hash of the sources and flags this library was compiled from (set by the in-tree build).
extern "C" const char* tai_build_id(void) { return TAI_BUILD_ID; }
