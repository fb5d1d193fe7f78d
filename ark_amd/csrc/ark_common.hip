// ark_common.hip -- definitions of the shared host-side helpers.
#include "ark_common.hpp"

#include <stdarg.h>
#include <stdio.h>

#include <string>

namespace ark {

namespace {
thread_local std::string g_last_error;
}

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(ARK_OPT_EHIP, "%s: %s (%d)", what, hipGetErrorString(e), (int)e);
}

const char* last_error() { return g_last_error.c_str(); }

int check_buffer(const void* p, uint64_t bytes, const char* what, int idx) {
  if (bytes == 0) return ARK_OPT_OK;
  if (p == nullptr) return fail(ARK_OPT_EINVAL, "buffer %d: %s is NULL", idx, what);
  hipPointerAttribute_t attr;
  hipError_t e = hipPointerGetAttributes(&attr, p);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return fail(ARK_OPT_EINVAL, "buffer %d: %s (%p) is not memory known to HIP", idx,
                what, p);
  }
  const bool device_ok = attr.type == hipMemoryTypeDevice || attr.type == hipMemoryTypeManaged ||
                         attr.type == hipMemoryTypeArray || attr.type == hipMemoryTypeUnified ||
                         (attr.type == hipMemoryTypeHost && attr.devicePointer != nullptr);
  if (!device_ok) {
    return fail(ARK_OPT_EINVAL, "buffer %d: %s (%p) is host memory the device cannot access",
                idx, what, p);
  }
  hipDeviceptr_t base = nullptr;
  size_t size = 0;
  e = hipMemGetAddressRange(&base, &size, (hipDeviceptr_t)p);
  if (e == hipSuccess && base != nullptr) {
    const uintptr_t b = (uintptr_t)base, q = (uintptr_t)p;
    if (q < b || q - b > size || bytes > size - (q - b)) {
      return fail(ARK_OPT_EINVAL,
                  "buffer %d: %s [%p, +%llu B) exceeds its allocation [%p, +%zu B)",
                  idx, what, p, (unsigned long long)bytes, base, size);
    }
  } else {
    (void)hipGetLastError();
  }
  return ARK_OPT_OK;
}

DeviceGuard::DeviceGuard(int dev) {
  if (hipGetDevice(&prev) != hipSuccess) return;
  ok = (prev == dev) || (hipSetDevice(dev) == hipSuccess);
}

DeviceGuard::~DeviceGuard() {
  int cur = -1;
  if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
}

}  // namespace ark
