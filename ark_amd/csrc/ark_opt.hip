// ark_opt.hip -- C ABI (include/ark_opt.h) over the gfx950 optimizer-step
// kernels: handle creation with the device-side tensor table and segment map,
// the per-step launch sequence, state get/set, timing, and the single-tensor
// drop-in of ark_asm_adam_step_f16.
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <string>
#include <vector>

#include "ark_ckpt.h"
#include "ark_codec.h"
#include "ark_common.hpp"
#include "ark_grad.h"
#include "ark_opt_internal.hpp"
#include "ark_opt_kernels.hpp"

using ark::SegDesc;
using ark::StepScalars;

using ark::align_up;
using ark::check_buffer;
using ark::DeviceGuard;
using ark::fail;
using ark::hip_fail;

namespace {

bool finite_f(float x) { return isfinite(x) != 0; }

int check_hparams(const ark_opt_hparams* hp) {
  if (!hp) return fail(ARK_OPT_EINVAL, "hparams is NULL");
  if (!finite_f(hp->beta1) || !finite_f(hp->beta2) || !finite_f(hp->eps))
    return fail(ARK_OPT_EINVAL, "beta1, beta2 and eps must be finite");
  if (!(hp->grad_clip > 0.0f))  // config.rs:136-138
    return fail(ARK_OPT_EINVAL, "grad_clip must be > 0 (got %g)", (double)hp->grad_clip);
  if (!finite_f(hp->loss_scale_init) || !(hp->loss_scale_init > 0.0f))
    return fail(ARK_OPT_EINVAL, "loss_scale_init must be finite and > 0");
  if (!(hp->loss_scale_min > 0.0f) || !(hp->loss_scale_max > 0.0f))
    return fail(ARK_OPT_EINVAL, "loss_scale_min and loss_scale_max must be > 0");
  if (hp->grad_dtype != ARK_OPT_GRAD_F16 && hp->grad_dtype != ARK_OPT_GRAD_F32)
    return fail(ARK_OPT_EINVAL, "grad_dtype %u unknown", hp->grad_dtype);
  return ARK_OPT_OK;
}

constexpr int kTimingPool = 256;

}  // namespace

struct ark_opt_handle {
  int device = 0;
  hipStream_t stream = nullptr;
  ark_opt_hparams hp{};
  int32_t ntensors = 0;
  uint32_t nseg = 0;
  int spb = 2;
  uint32_t norm_blocks = 0;
  uint32_t nt_from = 0;  // norm blocks from here up stream past the cache
  uint32_t sumsq_lds = 0;  // dynamic LDS per norm block (residency cap)
  uint32_t adamw_lds = 0;  // dynamic LDS per AdamW block (residency cap)
  // one device allocation carved into the pieces below
  void* dev_mem = nullptr;
  SegDesc* d_segs = nullptr;
  double* d_part_sum = nullptr;  // one partial per norm block, zero-padded
  double* d_fold = nullptr;      // fold output when there are many partials
  uint32_t padded_parts = 0;     // power of two >= parts when folding
  uint32_t fin_leaves = 1;       // leaves per finalize thread
  ark_opt_state* d_state = nullptr;
  StepScalars* d_scal = nullptr;
  ark_opt_step_info* d_info = nullptr;
  ark_opt_step_info* h_info = nullptr;  // pinned
  ark_opt_state* h_state = nullptr;     // pinned
  // the norm's units (fp32-gradient handles): written by the gradient
  // producers' final kernels, consumed by the next step instead of the read
  // of every gradient
  double* d_units = nullptr;
  bool units_fresh = false;
  struct TensorInfo {
    const void* g;
    uint64_t n;
    uint64_t seg0;  // index of its first segment
    uint32_t flags;
  };
  std::vector<TensorInfo> tensors;
  // timing
  bool timing = false;
  std::vector<hipEvent_t> ev;  // 4 per pending step
  int pending = 0;
  ark_opt_timing acc{};
};

namespace {

// Handles whose units are fresh (written by the gradient hand-off's final
// calls for their next step).  The library's other gradient writers look
// here (ark::opt_units_invalidate) so that a write after the final calls
// makes that step read the gradients instead of stale units.  Usually empty
// or one handle.
std::mutex g_fresh_mu;
std::vector<ark_opt_handle*> g_fresh;

void set_fresh_locked(ark_opt_handle* h, bool fresh) {
  h->units_fresh = fresh;
  auto it = std::find(g_fresh.begin(), g_fresh.end(), h);
  if (fresh && it == g_fresh.end()) g_fresh.push_back(h);
  if (!fresh && it != g_fresh.end()) g_fresh.erase(it);
}

// Whether h's units are fresh; either way they are not afterwards (a step
// consumes them).
bool take_fresh_units(ark_opt_handle* h) {
  std::lock_guard<std::mutex> lock(g_fresh_mu);
  const bool was = h->units_fresh;
  set_fresh_locked(h, false);
  return was;
}

int fold_timing(ark_opt_handle* h) {
  if (h->pending == 0) return ARK_OPT_OK;
  ARK_HIP(hipEventSynchronize(h->ev[4 * (h->pending - 1) + 3]));
  for (int i = 0; i < h->pending; ++i) {
    hipEvent_t* e = &h->ev[4 * i];
    float a = 0, b = 0, c = 0, d = 0;
    ARK_HIP(hipEventElapsedTime(&a, e[0], e[1]));
    ARK_HIP(hipEventElapsedTime(&b, e[1], e[2]));
    ARK_HIP(hipEventElapsedTime(&c, e[2], e[3]));
    ARK_HIP(hipEventElapsedTime(&d, e[0], e[3]));
    h->acc.ms_norm += a;
    h->acc.ms_finalize += b;
    h->acc.ms_adamw += c;
    h->acc.ms_step += d;
    h->acc.steps += 1;
  }
  h->pending = 0;
  return ARK_OPT_OK;
}

void free_handle(ark_opt_handle* h) {
  if (!h) return;
  for (hipEvent_t e : h->ev) (void)hipEventDestroy(e);
  if (h->dev_mem) (void)hipFree(h->dev_mem);
  if (h->h_info) (void)hipHostFree(h->h_info);
  if (h->h_state) (void)hipHostFree(h->h_state);
  delete h;
}

}  // namespace

extern "C" {

int ark_opt_abi_version(void) { return ARK_OPT_ABI_VERSION; }

const char* ark_opt_last_error(void) { return ark::last_error(); }

int ark_opt_struct_sizes(size_t* out, int n) {
  const size_t s[9] = {sizeof(ark_opt_tensor),  sizeof(ark_opt_hparams), sizeof(ark_opt_state),
                       sizeof(ark_opt_step_info), sizeof(ark_opt_timing), sizeof(ark_codec_span),
                       sizeof(ark_ckpt_record), sizeof(ark_ckpt_info),  sizeof(ark_grad_span)};
  if (!out || n < 0) return fail(ARK_OPT_EINVAL, "out is NULL");
  int k = n < 9 ? n : 9;
  for (int i = 0; i < k; ++i) out[i] = s[i];
  return k;
}

int ark_opt_default_hparams(ark_opt_hparams* out) {
  if (!out) return fail(ARK_OPT_EINVAL, "out is NULL");
  memset(out, 0, sizeof(*out));
  out->beta1 = 0.9f;                   // optimizer.rs:58
  out->beta2 = 0.999f;                 // optimizer.rs:59
  out->eps = 1e-8f;                    // optimizer.rs:60
  out->grad_clip = 1.0f;               // optimizer.rs:62
  out->loss_scale_init = 256.0f;       // training.rs:10
  out->loss_scale_min = 1.0f;          // training.rs:12
  out->loss_scale_max = 8192.0f;       // config.rs:69
  out->scale_up_every = 2000u;         // training.rs:13
  out->max_consecutive_nonfinite = 200u;  // training.rs:235, :298
  out->grad_dtype = ARK_OPT_GRAD_F16;
  return ARK_OPT_OK;
}

int ark_opt_create(const ark_opt_tensor* tensors, int32_t n_tensors,
                   const ark_opt_hparams* hp, void* stream,
                   ark_opt_handle** out) {
  if (!out) return fail(ARK_OPT_EINVAL, "out is NULL");
  *out = nullptr;
  if (!tensors || n_tensors <= 0)
    return fail(ARK_OPT_EINVAL, "tensor table is empty or NULL (n_tensors=%d)", n_tensors);
  int rc = check_hparams(hp);
  if (rc) return rc;
  const uint64_t gsz = hp->grad_dtype == ARK_OPT_GRAD_F16 ? 2u : 4u;

  // Segment descriptors: every tensor cut into ARK_OPT_NORM_SEGMENT pieces,
  // tensors in table order, pointers offset to each segment's start.
  std::vector<SegDesc> segs;
  for (int32_t i = 0; i < n_tensors; ++i) {
    const ark_opt_tensor& t = tensors[i];
    if (t.n == 0) continue;
    if (t.n > (1ull << 48)) return fail(ARK_OPT_EINVAL, "tensor %d: n too large", i);
    if (((uintptr_t)t.w & 1u) || ((uintptr_t)t.g & (gsz - 1)) ||
        ((uintptr_t)t.m & 3u) || ((uintptr_t)t.v & 3u))
      return fail(ARK_OPT_EINVAL, "tensor %d: pointer not aligned to its element", i);
    if (!finite_f(t.weight_decay))
      return fail(ARK_OPT_EINVAL, "tensor %d: weight_decay not finite", i);
    const uint64_t ns = (t.n + ark::kSeg - 1) / ark::kSeg;
    if (segs.size() + ns > ark::kMaxSegments)
      return fail(ARK_OPT_EINVAL, "too many elements (more than %llu segments of %d)",
                  (unsigned long long)ark::kMaxSegments, ark::kSeg);
    const bool vec =
        ((((uintptr_t)t.w | (uintptr_t)t.g | (uintptr_t)t.m | (uintptr_t)t.v) & 15u) == 0);
    uint32_t flags = vec ? ark::kSegVec : 0u;
    if (t.flags & ARK_OPT_TENSOR_NO_UNSCALE) flags |= ark::kSegNoUnscale;
    for (uint64_t k = 0; k < ns; ++k) {
      const uint64_t off = k * ark::kSeg;
      SegDesc d;
      d.w = t.w + off;
      d.g = (const char*)t.g + off * gsz;
      d.m = t.m + off;
      d.v = t.v + off;
      d.n = (uint32_t)(t.n - off < (uint64_t)ark::kSeg ? t.n - off : (uint64_t)ark::kSeg);
      d.wd = t.weight_decay;
      d.flags = flags;
      d.tensor = (uint32_t)i;
      segs.push_back(d);
    }
  }
  const uint64_t nseg = segs.size();
  int spb = ark::sumsq_spb(nseg, hp->grad_dtype);
  // ARK_OPT_SUMSQ_SPB=1|2|4|8 overrides the segments per norm block (a
  // tuning knob; the canonical tree makes the result independent of it).
  if (const char* env = getenv("ARK_OPT_SUMSQ_SPB")) {
    const int v = atoi(env);
    if (v >= 1 && v <= 8 && (v & (v - 1)) == 0 && (nseg + v - 1) / v <= ark::kMaxParts)
      spb = v;
  }
  const uint64_t parts = (nseg + spb - 1) / spb;
  if (parts > ark::kMaxParts)
    return fail(ARK_OPT_EINVAL, "too many elements (%llu segments)", (unsigned long long)nseg);
  // Resident blocks per CU of the norm and AdamW passes;
  // ARK_OPT_SUMSQ_BLOCKS_PER_CU=2..8 and ARK_OPT_ADAMW_BLOCKS_PER_CU=4..32
  // override them, 0 lifts a cap (tuning knobs: results do not depend on
  // them).
  int sumsq_per_cu = hp->grad_dtype == ARK_OPT_GRAD_F16 ? ark::kSumsqBlocksPerCuF16 : 0;
  if (const char* env = getenv("ARK_OPT_SUMSQ_BLOCKS_PER_CU")) {
    const int v = atoi(env);
    if (v == 0 || (v >= 2 && v <= 8)) sumsq_per_cu = v;
  }
  int adamw_per_cu = ark::kAdamwBlocksPerCu;
  if (const char* env = getenv("ARK_OPT_ADAMW_BLOCKS_PER_CU")) {
    const int v = atoi(env);
    if (v == 0 || (v >= 4 && v <= 32)) adamw_per_cu = v;
  }

  // The reference steps distinct per-tensor fields (optimizer.rs:171,
  // memory.rs:202-255), so w, m and v can never alias.  Here a tensor listed
  // twice or overlapping buffers would have two waves rewrite the same
  // words: refuse any written span shared with another written span or with
  // a gradient.
  {
    std::vector<ark::Span> written, grads;
    written.reserve(3 * (size_t)n_tensors);
    grads.reserve((size_t)n_tensors);
    for (int32_t i = 0; i < n_tensors; ++i) {
      const ark_opt_tensor& t = tensors[i];
      if (t.n == 0) continue;
      const uintptr_t w = (uintptr_t)t.w, g = (uintptr_t)t.g, m = (uintptr_t)t.m,
                      v = (uintptr_t)t.v;
      written.push_back({w, w + t.n * 2u, "w", i});
      written.push_back({m, m + t.n * 4u, "m", i});
      written.push_back({v, v + t.n * 4u, "v", i});
      grads.push_back({g, g + t.n * gsz, "g", i});
    }
    if ((rc = ark::check_disjoint(std::move(written), std::move(grads)))) return rc;
  }

  int dev = 0;
  if ((rc = ark::current_device_for(stream, &dev))) return rc;
  // set-up of the no-allocation scatter on this device, so that its first
  // call may come under graph capture (best effort: that call retries it)
  (void)ark::grad_scratch_prepare(dev);
  ark::BufferChecker checker;
  for (int32_t i = 0; i < n_tensors; ++i) {
    const ark_opt_tensor& t = tensors[i];
    if ((rc = checker.check(t.w, t.n * 2u, "w", i))) return rc;
    if ((rc = checker.check(t.g, t.n * gsz, "g", i))) return rc;
    if ((rc = checker.check(t.m, t.n * 4u, "m", i))) return rc;
    if ((rc = checker.check(t.v, t.n * 4u, "v", i))) return rc;
  }

  ark_opt_handle* h = new ark_opt_handle();
  h->device = dev;
  h->stream = (hipStream_t)stream;
  h->hp = *hp;
  h->ntensors = n_tensors;
  h->nseg = (uint32_t)nseg;
  h->spb = spb;
  h->norm_blocks = (uint32_t)parts;
  h->nt_from = ark::sumsq_nt_from(spb, gsz);
  h->sumsq_lds = ark::sumsq_lds_for(hp->grad_dtype, spb, sumsq_per_cu);
  h->adamw_lds = ark::adamw_lds_for(hp->grad_dtype, adamw_per_cu);

  // One allocation: segments | partial sums | state | scalars | info | units
  size_t off = 0;
  const size_t o_seg = off;
  off = align_up(off + sizeof(SegDesc) * (size_t)(nseg ? nseg : 1), 256);
  // Partials: up to kFinTarget go straight to the finalize (kFinThreads *
  // leaves doubles, zero past the real ones); more are first folded in
  // aligned groups of kFoldGroup from a power-of-two zero-padded buffer.
  const bool fold = parts > ark::kFinTarget;
  uint32_t padded = 0, leaves = 0;
  size_t psum_bytes = 0, fold_bytes = 0;
  if (fold) {
    padded = ark::kFoldGroup;
    while (padded < parts) padded <<= 1;
    psum_bytes = sizeof(double) * (size_t)padded;
    leaves = ark::finalize_leaves(padded / ark::kFoldGroup);
    fold_bytes = sizeof(double) * (size_t)ark::kFinThreads * leaves;
  } else {
    leaves = ark::finalize_leaves((uint32_t)parts);
    psum_bytes = sizeof(double) * (size_t)ark::kFinThreads * leaves;
  }
  const size_t o_psum = off;
  off = align_up(off + psum_bytes, 256);
  const size_t o_fold = off;
  off = align_up(off + fold_bytes, 256);
  const size_t o_state = off;
  off = align_up(off + sizeof(ark_opt_state), 256);
  const size_t o_scal = off;
  off = align_up(off + sizeof(StepScalars), 256);
  const size_t o_info = off;
  off = align_up(off + sizeof(ark_opt_step_info), 256);
  const size_t o_units = off;
  if (hp->grad_dtype == ARK_OPT_GRAD_F32)
    off = align_up(off + sizeof(double) * (size_t)nseg * ark::kUnitsPerSeg, 256);

  hipError_t e = hipMalloc(&h->dev_mem, off);
  if (e != hipSuccess) {
    free_handle(h);
    (void)hipGetLastError();
    return fail(ARK_OPT_ENOMEM, "hipMalloc(%zu) failed: %s", off, hipGetErrorString(e));
  }
  char* base = (char*)h->dev_mem;
  h->d_segs = (SegDesc*)(base + o_seg);
  h->d_part_sum = (double*)(base + o_psum);
  h->d_fold = fold ? (double*)(base + o_fold) : nullptr;
  h->padded_parts = padded;
  h->fin_leaves = leaves;
  h->d_state = (ark_opt_state*)(base + o_state);
  h->d_scal = (StepScalars*)(base + o_scal);
  h->d_info = (ark_opt_step_info*)(base + o_info);
  if (hp->grad_dtype == ARK_OPT_GRAD_F32 && nseg) h->d_units = (double*)(base + o_units);
  {
    uint64_t seg0 = 0;
    h->tensors.reserve((size_t)n_tensors);
    for (int32_t i = 0; i < n_tensors; ++i) {
      const ark_opt_tensor& t = tensors[i];
      h->tensors.push_back({t.g, t.n, seg0, t.flags});
      seg0 += (t.n + ark::kSeg - 1) / ark::kSeg;
    }
  }
  if (hipHostMalloc((void**)&h->h_info, sizeof(ark_opt_step_info), hipHostMallocDefault) != hipSuccess ||
      hipHostMalloc((void**)&h->h_state, sizeof(ark_opt_state), hipHostMallocDefault) != hipSuccess) {
    free_handle(h);
    (void)hipGetLastError();
    return fail(ARK_OPT_ENOMEM, "hipHostMalloc failed");
  }
  ark_opt_state st{};
  st.loss_scale = hp->loss_scale_init;  // training.rs:120
  StepScalars sc{};
  e = hipSuccess;
  if (nseg) e = hipMemcpy(h->d_segs, segs.data(), sizeof(SegDesc) * nseg, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemset(h->d_part_sum, 0, psum_bytes);
  if (e == hipSuccess && fold) e = hipMemset(h->d_fold, 0, fold_bytes);
  if (e == hipSuccess) e = hipMemcpy(h->d_state, &st, sizeof(st), hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemcpy(h->d_scal, &sc, sizeof(sc), hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    free_handle(h);
    return hip_fail(e, "uploading the tensor table");
  }
  *out = h;
  return ARK_OPT_OK;
}

int ark_opt_destroy(ark_opt_handle* h) {
  if (!h) return ARK_OPT_OK;
  ark::opt_units_set_fresh(h, false);
  DeviceGuard g(h->device);
  (void)hipStreamSynchronize(h->stream);
  free_handle(h);
  return ARK_OPT_OK;
}

static int finish_info(ark_opt_handle* h, ark_opt_step_info* info) {
  ARK_HIP(hipMemcpyAsync(h->h_info, h->d_info, sizeof(ark_opt_step_info),
                         hipMemcpyDeviceToHost, h->stream));
  ARK_HIP(hipStreamSynchronize(h->stream));
  *info = *h->h_info;
  return info->status;
}

namespace {

// ark_opt_step with lr given on the host (lr_dev NULL) or read by the
// finalize kernel from the device scalar lr_dev.
int step_impl(ark_opt_handle* h, float lr, const float* lr_dev, ark_opt_step_info* info) {
  DeviceGuard g(h->device);
  if (!g.ok) return fail(ARK_OPT_EHIP, "cannot select device %d", h->device);
  hipEvent_t* ev = nullptr;
  if (h->timing) {
    if (h->pending == kTimingPool) {
      int rc = fold_timing(h);
      if (rc) return rc;
    }
    ev = &h->ev[4 * h->pending];
    ARK_HIP(hipEventRecord(ev[0], h->stream));
  }
  if (h->nseg) {
    if (take_fresh_units(h)) {
      // the gradients' producers already formed the tree's first level
      ARK_HIP(ark::launch_units_reduce(h->spb, h->norm_blocks, h->d_units, h->d_segs, h->nseg,
                                       h->d_part_sum, h->stream));
    } else {
      ARK_HIP(ark::launch_sumsq(h->hp.grad_dtype, h->spb, h->norm_blocks, h->d_segs,
                                h->nseg, h->d_state, h->d_part_sum, h->nt_from, h->sumsq_lds,
                                h->stream));
    }
    if (h->d_fold)
      ARK_HIP(ark::launch_fold(h->padded_parts, h->d_part_sum, h->d_fold, h->stream));
  }
  if (ev) ARK_HIP(hipEventRecord(ev[1], h->stream));
  ARK_HIP(ark::launch_finalize(h->fin_leaves, h->d_fold ? h->d_fold : h->d_part_sum, h->hp,
                               lr, lr_dev, h->d_state, h->d_scal, h->d_info, h->stream));
  if (ev) ARK_HIP(hipEventRecord(ev[2], h->stream));
  if (h->nseg) {
    ARK_HIP(ark::launch_adamw(h->hp.grad_dtype, h->d_segs, h->nseg, h->d_scal,
                              h->hp.beta1, h->hp.beta2, h->hp.eps, h->adamw_lds, h->stream));
  }
  if (ev) {
    ARK_HIP(hipEventRecord(ev[3], h->stream));
    h->pending += 1;
  }
  if (info) return finish_info(h, info);
  return ARK_OPT_OK;
}

}  // namespace

int ark_opt_step(ark_opt_handle* h, float lr, ark_opt_step_info* info) {
  if (!h) return fail(ARK_OPT_EINVAL, "handle is NULL");
  if (!finite_f(lr)) return fail(ARK_OPT_EINVAL, "lr must be finite");
  return step_impl(h, lr, nullptr, info);
}

int ark_opt_step_lr_dev(ark_opt_handle* h, const float* lr_dev, ark_opt_step_info* info) {
  if (!h) return fail(ARK_OPT_EINVAL, "handle is NULL");
  if (!lr_dev || ((uintptr_t)lr_dev & 3u))
    return fail(ARK_OPT_EINVAL, "lr_dev is NULL or not 4-byte aligned");
  int rc;
  {
    DeviceGuard g(h->device);
    if (!g.ok) return fail(ARK_OPT_EHIP, "cannot select device %d", h->device);
    if ((rc = check_buffer(lr_dev, 4, "lr_dev", 0))) return rc;
  }
  rc = step_impl(h, 0.0f, lr_dev, info);
  if (rc == ARK_OPT_EINVAL) return fail(ARK_OPT_EINVAL, "the lr read from lr_dev is not finite");
  return rc;
}

int ark_opt_record_overflow(ark_opt_handle* h, ark_opt_step_info* info) {
  if (!h) return fail(ARK_OPT_EINVAL, "handle is NULL");
  DeviceGuard g(h->device);
  if (!g.ok) return fail(ARK_OPT_EHIP, "cannot select device %d", h->device);
  ark::opt_units_set_fresh(h, false);  // the loss scale they were unscaled by changes
  ARK_HIP(ark::launch_record_overflow(h->hp, h->d_state, h->d_info, h->stream));
  if (info) return finish_info(h, info);
  return ARK_OPT_OK;
}

int ark_opt_get_state(ark_opt_handle* h, ark_opt_state* out) {
  if (!h || !out) return fail(ARK_OPT_EINVAL, "handle or out is NULL");
  DeviceGuard g(h->device);
  if (!g.ok) return fail(ARK_OPT_EHIP, "cannot select device %d", h->device);
  ARK_HIP(hipMemcpyAsync(h->h_state, h->d_state, sizeof(ark_opt_state),
                         hipMemcpyDeviceToHost, h->stream));
  ARK_HIP(hipStreamSynchronize(h->stream));
  *out = *h->h_state;
  return ARK_OPT_OK;
}

int ark_opt_set_state(ark_opt_handle* h, const ark_opt_state* st) {
  if (!h || !st) return fail(ARK_OPT_EINVAL, "handle or state is NULL");
  if (!finite_f(st->loss_scale) || !(st->loss_scale > 0.0f))
    return fail(ARK_OPT_EINVAL, "loss_scale must be finite and > 0");
  DeviceGuard g(h->device);
  if (!g.ok) return fail(ARK_OPT_EHIP, "cannot select device %d", h->device);
  ARK_HIP(hipStreamSynchronize(h->stream));
  ark::opt_units_set_fresh(h, false);  // the loss scale they were unscaled by may change
  *h->h_state = *st;
  ARK_HIP(hipMemcpyAsync(h->d_state, h->h_state, sizeof(ark_opt_state),
                         hipMemcpyHostToDevice, h->stream));
  ARK_HIP(hipStreamSynchronize(h->stream));
  return ARK_OPT_OK;
}

int ark_opt_set_timing(ark_opt_handle* h, int enable) {
  if (!h) return fail(ARK_OPT_EINVAL, "handle is NULL");
  DeviceGuard g(h->device);
  if (!g.ok) return fail(ARK_OPT_EHIP, "cannot select device %d", h->device);
  if (enable && h->ev.empty()) {
    h->ev.resize(4 * kTimingPool);
    for (auto& e : h->ev) ARK_HIP(hipEventCreate(&e));
  }
  if (!enable) {
    int rc = fold_timing(h);
    if (rc) return rc;
  }
  h->timing = enable != 0;
  return ARK_OPT_OK;
}

int ark_opt_get_timing(ark_opt_handle* h, ark_opt_timing* out) {
  if (!h || !out) return fail(ARK_OPT_EINVAL, "handle or out is NULL");
  DeviceGuard g(h->device);
  if (!g.ok) return fail(ARK_OPT_EHIP, "cannot select device %d", h->device);
  int rc = fold_timing(h);
  if (rc) return rc;
  *out = h->acc;
  return ARK_OPT_OK;
}

int ark_hip_adam_step(float* w, const float* g, float* m, float* v, uint64_t n, float lr,
                      float beta1, float beta2, float eps, float wd, uint32_t t, void* stream) {
  if (n == 0) return ARK_OPT_OK;
  if ((((uintptr_t)w | (uintptr_t)g | (uintptr_t)m | (uintptr_t)v) & 3u))
    return fail(ARK_OPT_EINVAL, "pointer not aligned to its element");
  if (n > (1ull << 48) || (n + ark::kRow - 1) / ark::kRow * 64u >= (1ull << 32))
    return fail(ARK_OPT_EINVAL, "n too large (%llu)", (unsigned long long)n);
  int rc;
  const uintptr_t uw = (uintptr_t)w, ug = (uintptr_t)g, um = (uintptr_t)m, uv = (uintptr_t)v;
  if ((rc = ark::check_disjoint({{uw, uw + n * 4u, "w", 0}, {um, um + n * 4u, "m", 0},
                                 {uv, uv + n * 4u, "v", 0}},
                                {{ug, ug + n * 4u, "g", 0}})))
    return rc;
  if ((rc = check_buffer(w, n * 4u, "w", 0))) return rc;
  if ((rc = check_buffer(g, n * 4u, "g", 0))) return rc;
  if ((rc = check_buffer(m, n * 4u, "m", 0))) return rc;
  if ((rc = check_buffer(v, n * 4u, "v", 0))) return rc;
  {
    const void* d[3] = {w, m, v};  // any may be another handle's gradient
    const uint64_t b[3] = {n * 4u, n * 4u, n * 4u};
    ark::opt_units_invalidate(d, b, 3);
  }
  const bool vec = (((uw | ug | um | uv) & 15u) == 0);
  StepScalars sc{};
  sc.applied = 1u;
  sc.inv = 1.0f;
  sc.coef = 1.0f;
  sc.lr = lr;
  sc.lr_eff = ark::lr_eff_of(lr, beta1, beta2, t);  // opti.s:38-90
  sc.c1 = 1.0f - beta1;                              // opti.s:94-96
  sc.c2 = 1.0f - beta2;                              // opti.s:97-99
  ARK_HIP(ark::launch_adamw_single_w32(w, g, m, v, n, wd, vec, sc, beta1, beta2, eps,
                                        (hipStream_t)stream));
  return ARK_OPT_OK;
}

int ark_hip_adam_step_f16(uint16_t* w, const float* g, float* m, float* v,
                          uint64_t n, float lr, float beta1, float beta2,
                          float eps, float wd, uint32_t t, void* stream) {
  if (n == 0) return ARK_OPT_OK;
  if (((uintptr_t)w & 1u) || ((uintptr_t)g & 3u) || ((uintptr_t)m & 3u) || ((uintptr_t)v & 3u))
    return fail(ARK_OPT_EINVAL, "pointer not aligned to its element");
  if (n > (1ull << 48) || (n + ark::kRow - 1) / ark::kRow * 64u >= (1ull << 32))
    return fail(ARK_OPT_EINVAL, "n too large (%llu)", (unsigned long long)n);
  int rc;
  const uintptr_t uw = (uintptr_t)w, ug = (uintptr_t)g, um = (uintptr_t)m, uv = (uintptr_t)v;
  if ((rc = ark::check_disjoint({{uw, uw + n * 2u, "w", 0}, {um, um + n * 4u, "m", 0},
                                 {uv, uv + n * 4u, "v", 0}},
                                {{ug, ug + n * 4u, "g", 0}})))
    return rc;
  if ((rc = check_buffer(w, n * 2u, "w", 0))) return rc;
  if ((rc = check_buffer(g, n * 4u, "g", 0))) return rc;
  if ((rc = check_buffer(m, n * 4u, "m", 0))) return rc;
  if ((rc = check_buffer(v, n * 4u, "v", 0))) return rc;
  {
    const void* d[3] = {w, m, v};  // any may be another handle's gradient
    const uint64_t b[3] = {n * 2u, n * 4u, n * 4u};
    ark::opt_units_invalidate(d, b, 3);
  }
  const bool vec =
      ((((uintptr_t)w | (uintptr_t)g | (uintptr_t)m | (uintptr_t)v) & 15u) == 0);
  StepScalars sc{};
  sc.applied = 1u;
  sc.inv = 1.0f;
  sc.coef = 1.0f;
  sc.lr = lr;
  sc.lr_eff = ark::lr_eff_of(lr, beta1, beta2, t);  // opti.s:210-258
  sc.c1 = 1.0f - beta1;                              // opti.s:263-265
  sc.c2 = 1.0f - beta2;                              // opti.s:266-268
  ARK_HIP(ark::launch_adamw_single(w, g, m, v, n, wd, vec, sc, beta1, beta2, eps,
                                    (hipStream_t)stream));
  return ARK_OPT_OK;
}

int ark_hip_grad_clip(float* grads, uint64_t n, float threshold, float* norm_out,
                      void* stream) {
  if (norm_out) *norm_out = 0.0f;
  if (n == 0) return ARK_OPT_OK;  // no value: norm 0, nothing scaled (ffi.rs:208-210)
  if ((uintptr_t)grads & 3u) return fail(ARK_OPT_EINVAL, "grads not 4-byte aligned");
  if (n > ark::kClipMaxElements)
    return fail(ARK_OPT_EINVAL, "n = %llu exceeds %llu", (unsigned long long)n,
                (unsigned long long)ark::kClipMaxElements);
  int rc;
  if ((rc = check_buffer(grads, n * 4u, "grads", 0))) return rc;
  {
    const void* d = grads;  // it may be an optimizer's gradient
    const uint64_t b = n * 4u;
    ark::opt_units_invalidate(&d, &b, 1);
  }
  hipStream_t s = (hipStream_t)stream;
  const uint32_t nparts = ark::clip_parts(n);
  const uint32_t ngroups = (nparts + ark::kFoldGroup - 1) / ark::kFoldGroup;
  const size_t bytes = ark::align_up(sizeof(ark::ClipScalars), 256) +
                       ark::align_up((size_t)nparts * 8u, 256) + (size_t)ngroups * 8u;
  ark::StreamBuf ws;
  hipError_t e = ws.alloc(bytes, s);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return fail(ARK_OPT_ENOMEM, "hipMallocAsync(%zu) for the clip failed", bytes);
  }
  ark::ClipScalars* cs = (ark::ClipScalars*)ws.p;
  double* parts = (double*)((char*)ws.p + ark::align_up(sizeof(ark::ClipScalars), 256));
  double* folded = parts + ark::align_up((size_t)nparts * 8u, 256) / 8u;
  ARK_HIP(ark::launch_grad_clip(grads, n, threshold, parts, folded, cs, s));
  if (norm_out) {
    float norm = 0.0f;
    ARK_HIP(hipMemcpyAsync(&norm, &cs->norm, sizeof(float), hipMemcpyDeviceToHost, s));
    ARK_HIP(hipStreamSynchronize(s));
    *norm_out = norm;
  }
  return ARK_OPT_OK;
}

}  // extern "C"

// ---- the norm's units, for the gradient hand-off (ark_opt_internal.hpp) ----

namespace ark {

namespace {
void fill_units(ark_opt_handle* h, OptUnits* out) {
  out->units = h->d_units;
  out->segs = h->d_segs;
  out->state = h->d_state;
  out->stream = h->stream;
  out->device = h->device;
  out->nseg = h->nseg;
}
}  // namespace

int opt_units_for_spans(ark_opt_handle* h, const float* const* dst, const uint64_t* n,
                        size_t count, OptUnits* out) {
  if (!h) return fail(ARK_OPT_EINVAL, "optimizer handle is NULL");
  if (h->hp.grad_dtype != ARK_OPT_GRAD_F32)
    return fail(ARK_OPT_EINVAL, "the optimizer handle does not take fp32 gradients");
  size_t j = 0;
  for (size_t i = 0; i < h->tensors.size(); ++i) {
    const ark_opt_handle::TensorInfo& t = h->tensors[i];
    if (t.n == 0) continue;
    while (j < count && n[j] == 0) ++j;
    if (j == count)
      return fail(ARK_OPT_EINVAL, "the plan ends before tensor %zu of the optimizer table", i);
    if ((const void*)dst[j] != t.g || n[j] != t.n)
      return fail(ARK_OPT_EINVAL,
                  "plan span %zu (%p, %llu elements) is not tensor %zu's gradient (%p, %llu)", j,
                  (const void*)dst[j], (unsigned long long)n[j], i, t.g,
                  (unsigned long long)t.n);
    ++j;
  }
  while (j < count && n[j] == 0) ++j;
  if (j != count)
    return fail(ARK_OPT_EINVAL, "plan span %zu has no tensor in the optimizer table", j);
  fill_units(h, out);
  return ARK_OPT_OK;
}

int opt_units_for_tensor(ark_opt_handle* h, const void* g, uint64_t n, bool require_fresh,
                         OptUnits* out, uint64_t* unit0, uint32_t* seg_flags) {
  if (!h) return fail(ARK_OPT_EINVAL, "optimizer handle is NULL");
  if (require_fresh && !h->units_fresh)
    return fail(ARK_OPT_EINVAL,
                "the optimizer handle has no gradient units for its next step (run the plan's "
                "final accumulation first)");
  for (const ark_opt_handle::TensorInfo& t : h->tensors) {
    if (t.g == g && t.n == n) {
      fill_units(h, out);
      *unit0 = t.seg0 * (uint64_t)kUnitsPerSeg;
      *seg_flags = (t.flags & ARK_OPT_TENSOR_NO_UNSCALE) ? kSegNoUnscale : 0u;
      return ARK_OPT_OK;
    }
  }
  return fail(ARK_OPT_EINVAL, "no tensor of the optimizer table has gradient %p of %llu elements",
              g, (unsigned long long)n);
}

void opt_units_set_fresh(ark_opt_handle* h, bool fresh) {
  std::lock_guard<std::mutex> lock(g_fresh_mu);
  set_fresh_locked(h, fresh);
}

void opt_units_invalidate(const void* const* dst, const uint64_t* bytes, size_t count) {
  std::lock_guard<std::mutex> lock(g_fresh_mu);
  for (size_t k = 0; k < g_fresh.size();) {
    ark_opt_handle* h = g_fresh[k];
    bool hit = false;
    for (size_t i = 0; i < count && !hit; ++i) {
      if (bytes[i] == 0) continue;
      for (const ark_opt_handle::TensorInfo& t : h->tensors) {
        if (t.n && overlaps(t.g, t.n * 4u, dst[i], bytes[i])) {
          hit = true;
          break;
        }
      }
    }
    if (hit)
      set_fresh_locked(h, false);
    else
      ++k;
  }
}

}  // namespace ark
