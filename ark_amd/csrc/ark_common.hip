// ark_common.hip -- definitions of the shared host-side helpers.
#include "ark_common.hpp"

#include <stdarg.h>
#include <stdio.h>

#include <algorithm>
#include <atomic>
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

namespace {

// check_buffer, also returning the allocation range when the runtime knows it
// (*size = 0 when it does not).
int check_buffer_range(const void* p, uint64_t bytes, const char* what, int idx,
                       uintptr_t* rbase, size_t* rsize) {
  *rbase = 0;
  *rsize = 0;
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
    *rbase = b;
    *rsize = size;
  } else {
    (void)hipGetLastError();
  }
  return ARK_OPT_OK;
}

}  // namespace

int current_device_for(void* stream, int* dev) {
  *dev = 0;
  hipError_t e = hipGetDevice(dev);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return hip_fail(e, "hipGetDevice");
  }
  if (!stream) return ARK_OPT_OK;
  int sdev = -1;
  e = hipStreamGetDevice((hipStream_t)stream, &sdev);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return hip_fail(e, "device of the stream");
  }
  if (sdev != *dev)
    return fail(ARK_OPT_EINVAL,
                "the stream belongs to device %d but device %d is current: make the stream's "
                "device current before creating the handle or plan",
                sdev, *dev);
  return ARK_OPT_OK;
}

int check_buffer(const void* p, uint64_t bytes, const char* what, int idx) {
  uintptr_t b;
  size_t s;
  return check_buffer_range(p, bytes, what, idx, &b, &s);
}

int BufferChecker::check(const void* p, uint64_t bytes, const char* what, int idx) {
  if (bytes == 0) return ARK_OPT_OK;
  const uintptr_t q = (uintptr_t)p;
  for (int i = 0; i < used_; ++i)
    if (p != nullptr && q >= base_[i] && q - base_[i] <= size_[i] &&
        bytes <= size_[i] - (q - base_[i]))
      return ARK_OPT_OK;
  uintptr_t b;
  size_t s;
  const int rc = check_buffer_range(p, bytes, what, idx, &b, &s);
  if (rc == ARK_OPT_OK && s != 0) {
    base_[next_] = b;
    size_[next_] = s;
    next_ = (next_ + 1) % kRanges;
    if (used_ < kRanges) ++used_;
  }
  return rc;
}

int check_disjoint(std::vector<Span> written, std::vector<Span> readonly, const char* unit,
                   const char* writer) {
  auto empty = [](const Span& x) { return x.hi <= x.lo; };
  written.erase(std::remove_if(written.begin(), written.end(), empty), written.end());
  readonly.erase(std::remove_if(readonly.begin(), readonly.end(), empty), readonly.end());
  auto by_lo = [](const Span& a, const Span& b) { return a.lo < b.lo; };
  std::sort(written.begin(), written.end(), by_lo);
  // sorted by start, no two overlap iff each starts at or past the previous
  // one's end
  for (size_t i = 1; i < written.size(); ++i) {
    const Span &a = written[i - 1], &b = written[i];
    if (b.lo < a.hi)
      return fail(ARK_OPT_EINVAL, "%s %d %s overlaps %s %d %s (both written)", unit, a.idx,
                  a.what, unit, b.idx, b.what);
  }
  // disjoint and sorted: the ends are sorted too, so the first written span
  // ending past r.lo is the only candidate for overlapping r
  for (const Span& r : readonly) {
    auto it = std::upper_bound(written.begin(), written.end(), r.lo,
                               [](uintptr_t x, const Span& s) { return x < s.hi; });
    if (it != written.end() && it->lo < r.hi)
      return fail(ARK_OPT_EINVAL, "%s %d %s overlaps %s %d %s (written by %s)", unit, r.idx,
                  r.what, unit, it->idx, it->what, writer);
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

int lds_per_cu(int device) {
  constexpr int kDevices = 64;
  static std::atomic<int> cache[kDevices];  // 0: not queried yet, -1: unknown
  if (device < 0 || device >= kDevices) return 0;
  int v = cache[device].load(std::memory_order_relaxed);
  if (v == 0) {
    int q = 0;
    if (hipDeviceGetAttribute(&q, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, device) !=
            hipSuccess ||
        q <= 0) {
      (void)hipGetLastError();
      q = -1;
    }
    cache[device].store(q, std::memory_order_relaxed);
    v = q;
  }
  return v > 0 ? v : 0;
}

uint32_t resident_lds_bytes(const void* kernel, int threads, int blocks) {
  if (blocks <= 0) return 0;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  const uint32_t lds = (uint32_t)lds_per_cu(dev);
  if (lds == 0) return 0;
  // resident blocks with `dyn` bytes reserved (0 when it cannot launch)
  auto occ = [&](uint32_t dyn, int* n) {
    *n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(n, kernel, threads, dyn) != hipSuccess) {
      (void)hipGetLastError();
      *n = 0;
      return false;
    }
    return true;
  };
  int n0 = 0;
  if (!occ(0, &n0) || n0 <= blocks) return 0;
  // smallest reservation in (0, lds] that leaves at most b blocks
  auto first_at_most = [&](int b) {
    uint32_t lo = 0, hi = lds;  // occupancy(lo) > b >= occupancy(hi)
    while (hi - lo > 1) {
      const uint32_t mid = lo + (hi - lo) / 2;
      int n = 0;
      occ(mid, &n);
      if (n <= b)
        hi = mid;
      else
        lo = mid;
    }
    return hi;
  };
  const uint32_t a = first_at_most(blocks), z = first_at_most(blocks - 1);
  return a + (z - a) / 2;
}

}  // namespace ark
