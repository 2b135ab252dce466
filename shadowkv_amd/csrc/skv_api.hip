// Library-wide C ABI helpers: version, per-thread error text, pinned-host address translation.
#include <cstdarg>
#include <cstdio>

#include "skv_common.h"

static thread_local char g_last_error[512] = "";

void skv_set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

int skv_check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    skv_set_error("%s: kernel launch failed: %s", what, hipGetErrorString(e));
    return SKV_ELAUNCH;
  }
  return SKV_OK;
}

extern "C" const char* skv_version(void) { return "shadowkv_amd 0.1 gfx950"; }

extern "C" const char* skv_last_error(void) { return g_last_error; }

extern "C" int skv_host_device_pointer(const void* host_ptr, void** device_ptr) {
  if (host_ptr == nullptr || device_ptr == nullptr) {
    skv_set_error("skv_host_device_pointer: null pointer");
    return SKV_EINVAL;
  }
  void* dev = nullptr;
  hipError_t e = hipHostGetDevicePointer(&dev, const_cast<void*>(host_ptr), 0);
  if (e != hipSuccess) {
    skv_set_error("skv_host_device_pointer: %s (is the buffer pinned with hipHostMalloc?)",
                  hipGetErrorString(e));
    return SKV_EINVAL;
  }
  *device_ptr = dev;
  return SKV_OK;
}
