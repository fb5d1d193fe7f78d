// ark_common.hpp -- host-side helpers shared by every C-ABI entry point of
// libark_opt.so: the thread-local last-error message, HIP error mapping,
// device guard and the caller-buffer check.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <vector>

#include "ark_opt.h"

namespace ark {

// Records a printf-style message as the calling thread's last error (read
// back with ark_opt_last_error) and returns code.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// fail(ARK_OPT_EHIP, "<what>: <hip error string> (<code>)").
int hip_fail(hipError_t e, const char* what);

// The message behind ark_opt_last_error().
const char* last_error();

// Host-side bounds check of a caller buffer: it must be device-accessible
// memory and [p, p + bytes) must lie inside its allocation when the runtime
// can tell the allocation range.  Catches host pointers and short buffers
// before any kernel touches them.  what/idx name the buffer in the message.
int check_buffer(const void* p, uint64_t bytes, const char* what, int idx);

// check_buffer for many buffers that mostly share a few allocations (one
// arena per array kind): an allocation range found once is remembered, and a
// buffer inside a remembered range needs no runtime query.
class BufferChecker {
 public:
  int check(const void* p, uint64_t bytes, const char* what, int idx);

 private:
  static constexpr int kRanges = 8;
  uintptr_t base_[kRanges] = {};
  size_t size_[kRanges] = {};
  int used_ = 0, next_ = 0;
};

// The current device, into *dev; when stream is not NULL it must belong to
// that device (a handle or plan allocates on the current device and launches
// on its stream), ARK_OPT_EINVAL naming both otherwise.
int current_device_for(void* stream, int* dev);

// Restores the caller's current device on scope exit.
struct DeviceGuard {
  int prev = -1;
  bool ok = false;
  explicit DeviceGuard(int dev);
  ~DeviceGuard();
};

inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// True when [a, a + abytes) and [b, b + bbytes) share a byte.
inline bool overlaps(const void* a, uint64_t abytes, const void* b, uint64_t bbytes) {
  const uintptr_t x = (uintptr_t)a, y = (uintptr_t)b;
  return x < y + bbytes && y < x + abytes;
}

// A byte range [lo, hi) of a caller buffer, named for error messages.
struct Span {
  uintptr_t lo = 0, hi = 0;
  const char* what = "";
  int idx = 0;
};

// Fails with ARK_OPT_EINVAL, naming both buffers, when two written spans
// share a byte or a read-only span shares a byte with a written one (read-
// only spans may overlap each other).  Empty spans are ignored.  Host-only:
// compares addresses, queries nothing.  unit and writer word the message
// ("tensor 3 w overlaps tensor 5 v", "... (written by the step)").
int check_disjoint(std::vector<Span> written, std::vector<Span> readonly,
                   const char* unit = "tensor", const char* writer = "the step");

// Residency caps for streaming kernels.  A streaming kernel that fills every
// wave slot of a CU issues more loads than HBM serves best on MI355X; fewer
// resident blocks per CU run faster (the cap of each kernel is measured where
// it is set).  The cap is a dynamic-LDS reservation the kernel never touches.
//
// The device's LDS per CU (163,840 B on MI355X), queried once per device; 0
// when the runtime cannot tell.
int lds_per_cu(int device);
// The reservation that leaves `blocks` resident blocks per CU of `kernel`
// launched with `threads` threads on the current device, by the runtime's
// occupancy calculator (which counts the kernel's own LDS, including what
// library calls such as __syncthreads_or add, and the allocation granule):
// the middle of the range of reservations that give that count.  0 when
// blocks <= 0, the kernel holds no more than that anyway, or the runtime
// cannot tell.
uint32_t resident_lds_bytes(const void* kernel, int threads, int blocks);

// Every library call that writes device memory a caller passed in reports
// the byte ranges it is about to write: every optimizer handle whose norm
// units are fresh (written by the gradient hand-off's final calls for its
// next step) and whose gradients overlap one of them loses those units, so
// its next step reads the gradients.  Host-only; cheap when no handle is
// fresh (ark_opt.hip).
void opt_units_invalidate(const void* const* dst, const uint64_t* bytes, size_t count);

// Sets device dev up for ark_grad_embed_scatter_noalloc (ark_grad.hip): looks
// up the address of that device's copy of the static workspace and creates the
// event that orders the calls, once per device.  The library's set-up calls
// (ark_opt_create, ark_grad_plan_create) run it, so that a later
// no-allocation call, also one under graph capture, needs no runtime lookup.
// Repeated calls return at once.
int grad_scratch_prepare(int dev);

// Scratch device memory from the stream-ordered pool, freed in stream order
// when the owner goes out of scope (after the work queued on it).
struct StreamBuf {
  void* p = nullptr;
  hipStream_t s = nullptr;
  hipError_t alloc(size_t bytes, hipStream_t stream) {
    s = stream;
    return hipMallocAsync(&p, bytes, stream);
  }
  ~StreamBuf() {
    if (p) (void)hipFreeAsync(p, s);
  }
};

}  // namespace ark

#define ARK_HIP(call)                                       \
  do {                                                      \
    hipError_t e_ = (call);                                 \
    if (e_ != hipSuccess) return ark::hip_fail(e_, #call);  \
  } while (0)
