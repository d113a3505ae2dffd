// sd_capi.cpp — error reporting and version entry points of the C ABI.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>

#include "sd_common.h"

namespace sd {

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

void clear_error() { g_last_error[0] = '\0'; }

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: kernel launch failed: %s", what, hipGetErrorString(e));
    return SD_ERR_HIP;
  }
  return SD_OK;
}

}  // namespace sd

extern "C" int sd_abi_version(void) { return SD_ABI_VERSION; }

extern "C" const char* sd_last_error(void) { return sd::g_last_error; }
