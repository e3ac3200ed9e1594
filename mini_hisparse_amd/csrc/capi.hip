// Library-wide C-ABI entry points: error reporting and version.
#include <stdarg.h>
#include <stdio.h>

#include "hs_common.h"

namespace hs {

static thread_local char g_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list args;
  va_start(args, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, args);
  va_end(args);
}

}  // namespace hs

extern "C" const char* hs_last_error(void) { return hs::g_error; }

extern "C" int hs_version(void) { return HS_VERSION; }

extern "C" int hs_device_lds_bytes(int device, int64_t* bytes) {
  HS_CHECK_ARG(bytes != nullptr, "null output");
  int value = 0;
  hipError_t e = hipDeviceGetAttribute(&value, hipDeviceAttributeMaxSharedMemoryPerBlock, device);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    hs::set_error("hipDeviceGetAttribute failed: %s", hipGetErrorString(e));
    return HS_ERUNTIME;
  }
  *bytes = value;
  return HS_OK;
}

extern "C" int hs_host_alloc(int64_t bytes, void** host_ptr) {
  HS_CHECK_ARG(bytes >= 1 && host_ptr != nullptr, "invalid host allocation request");
  void* p = nullptr;
  hipError_t e = hipHostMalloc(&p, static_cast<size_t>(bytes), hipHostMallocDefault);
  if (e != hipSuccess || p == nullptr) {
    (void)hipGetLastError();
    hs::set_error("hipHostMalloc of %lld bytes failed: %s", static_cast<long long>(bytes), hipGetErrorString(e));
    return HS_ERUNTIME;
  }
  *host_ptr = p;
  return HS_OK;
}

extern "C" int hs_host_free(void* host_ptr) {
  if (host_ptr == nullptr) return HS_OK;
  hipError_t e = hipHostFree(host_ptr);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    hs::set_error("hipHostFree failed: %s", hipGetErrorString(e));
    return HS_ERUNTIME;
  }
  return HS_OK;
}
