// sd_capi.cpp — error reporting and version entry points of the C ABI.
#include <hip/hip_runtime.h>

#include <atomic>
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

namespace {

// Device attributes cached per device id. Entries are atomics: concurrent
// callers on several host threads may fill the same entry, and every filler
// stores the same value, so relaxed ordering suffices.
constexpr int kMaxDevices = 64;
std::atomic<int> g_cus[kMaxDevices];
std::atomic<int> g_lds[kMaxDevices];

int cached_attr(std::atomic<int>* cache, hipDeviceAttribute_t attr, int fallback) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = 0;
  const bool cacheable = dev >= 0 && dev < kMaxDevices;
  if (cacheable) {
    const int v = cache[dev].load(std::memory_order_relaxed);
    if (v > 0) return v;
  }
  int n = 0;
  if (hipDeviceGetAttribute(&n, attr, dev) != hipSuccess || n <= 0) n = fallback;
  if (cacheable) cache[dev].store(n, std::memory_order_relaxed);
  return n;
}

}  // namespace

int device_cus() { return cached_attr(g_cus, hipDeviceAttributeMultiprocessorCount, 256); }

int device_lds_per_block() {
  return cached_attr(g_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, 65536);
}

}  // namespace sd

extern "C" int sd_abi_version(void) { return SD_ABI_VERSION; }

extern "C" const char* sd_last_error(void) { return sd::g_last_error; }
