// ark_codec.hip -- fp16 <-> fp32 weight codec (include/ark_codec.h).
//
// Pure streaming conversions, HBM bound at 6 bytes per element (2 B of fp16
// and 4 B of fp32, one read and one write).  A lane converts 4 consecutive
// elements per access: 8 bytes on the fp16 side, 16 on the fp32 side, all
// non-temporal (the data is touched once).  Unaligned pointers and tails
// fall back to per-element accesses.
//
// The batch kernel takes 4096-element segments from a descriptor table
// (source and destination already offset to the segment), several blocks per
// segment, so a whole model's tensors convert in a single launch.
#include <string.h>

#include <vector>

#include "ark_codec.h"
#include "ark_common.hpp"
#include "ark_device.hpp"

namespace {

using namespace ark::dev;

constexpr int kPerLane = 4;      // elements per access: 8 B of fp16, 16 B of fp32
constexpr int kQuads = 2;        // accesses per lane, kLanes * 4 elements apart
constexpr uint32_t kSeg = 4096;  // batch kernel: elements per segment

// Lanes per block by direction.  Measured on MI355X over the EKO-237M weight
// set with the Infinity Cache flushed before each launch: two quads per lane
// with 64-lane blocks dequantise at 6.45 TB/s and with 256-lane blocks
// quantise at 6.69 TB/s, where one quad per lane in 256-lane blocks reaches
// 5.5 and 6.1 TB/s, and four or more quads per lane fall back below 6.2.
template <uint32_t DIR>
struct Shape {
  static constexpr uint32_t kLanes = DIR == ARK_CODEC_F16_TO_F32 ? 64u : 256u;
  static constexpr uint32_t kSpan = kLanes * kPerLane * kQuads;  // elements per block
  static constexpr uint32_t kBlocksPerSeg = kSeg / kSpan;
  static_assert(kBlocksPerSeg * kSpan == kSeg, "segment shape");
};
constexpr uint32_t kMaxBlocksPerSeg = Shape<ARK_CODEC_F16_TO_F32>::kBlocksPerSeg;  // 8
static_assert(Shape<ARK_CODEC_F16_TO_F32>::kBlocksPerSeg * Shape<ARK_CODEC_F16_TO_F32>::kLanes ==
                  Shape<ARK_CODEC_F32_TO_F16>::kBlocksPerSeg * Shape<ARK_CODEC_F32_TO_F16>::kLanes,
              "both directions launch the same work-items per segment");
constexpr uint64_t kMaxPlanSegs =
    ((1ull << 32) - 1) / (kMaxBlocksPerSeg * Shape<ARK_CODEC_F16_TO_F32>::kLanes);

struct CodecSeg {
  const void* src;
  void* dst;
  uint32_t n;    // elements in this segment, 1..kSeg
  uint32_t vec;  // src and dst 16-byte aligned
};
static_assert(sizeof(CodecSeg) == 24, "24-byte descriptor");

// 4 consecutive elements.  Lanes of a wave take consecutive quads, so every
// load and store instruction covers one contiguous span (512 B of fp16,
// 1 KiB of fp32).
template <uint32_t DIR>
__device__ __forceinline__ void conv4(const void* src, void* dst) {
  if constexpr (DIR == ARK_CODEC_F16_TO_F32) {
    const u32x2 h = ld_nt<u32x2>(src);
    u32x4 a;
    a.x = f16_to_f32_bits(h.x & 0xFFFFu);
    a.y = f16_to_f32_bits(h.x >> 16);
    a.z = f16_to_f32_bits(h.y & 0xFFFFu);
    a.w = f16_to_f32_bits(h.y >> 16);
    st_nt<u32x4>(dst, a);
  } else {
    const u32x4 a = ld_nt<u32x4>(src);
    u32x2 h;
    h.x = f32_to_f16_bits(a.x) | (f32_to_f16_bits(a.y) << 16);
    h.y = f32_to_f16_bits(a.z) | (f32_to_f16_bits(a.w) << 16);
    st_nt<u32x2>(dst, h);
  }
}

template <uint32_t DIR>
__device__ __forceinline__ void conv1(const void* src, void* dst, uint64_t i) {
  if constexpr (DIR == ARK_CODEC_F16_TO_F32) {
    const uint32_t h = ld_g<uint16_t>((const uint16_t*)src + i);
    st_g<uint32_t>((uint32_t*)dst + i, f16_to_f32_bits(h));
  } else {
    const uint32_t x = ld_g<uint32_t>((const uint32_t*)src + i);
    st_g<uint16_t>((uint16_t*)dst + i, (uint16_t)f32_to_f16_bits(x));
  }
}

template <uint32_t DIR>
constexpr uint32_t src_size() { return DIR == ARK_CODEC_F16_TO_F32 ? 2u : 4u; }
template <uint32_t DIR>
constexpr uint32_t dst_size() { return DIR == ARK_CODEC_F16_TO_F32 ? 4u : 2u; }

// The block's span [b0, b0 + kSpan) of a range of n elements: lane l converts
// the quads at b0 + 4l and b0 + 4l + 4 * kLanes (each access instruction of a
// wave covers one contiguous stretch).  vec: both pointers 16-byte aligned.
template <uint32_t DIR>
__device__ __forceinline__ void convert_span(const void* src, void* dst, uint64_t b0, uint64_t n,
                                             uint32_t vec) {
  constexpr uint32_t L = Shape<DIR>::kLanes;
#pragma unroll
  for (int u = 0; u < kQuads; ++u) {
    const uint64_t e0 = b0 + (uint64_t)(u * L + threadIdx.x) * kPerLane;
    if (e0 >= n) return;  // the next quad lies further on
    if (vec && e0 + kPerLane <= n) {
      conv4<DIR>((const char*)src + e0 * src_size<DIR>(), (char*)dst + e0 * dst_size<DIR>());
    } else {
      for (int j = 0; j < kPerLane; ++j)
        if (e0 + j < n) conv1<DIR>(src, dst, e0 + j);
    }
  }
}

// One flat range; blocks take consecutive spans, grid-stride (one pass for
// every size up to the grid cap times the span).
template <uint32_t DIR>
__global__ __launch_bounds__(Shape<DIR>::kLanes) void codec_flat(const void* __restrict__ src,
                                                                 void* __restrict__ dst,
                                                                 uint64_t n, uint32_t vec) {
  constexpr uint64_t S = Shape<DIR>::kSpan;
  for (uint64_t b0 = (uint64_t)blockIdx.x * S; b0 < n; b0 += (uint64_t)gridDim.x * S)
    convert_span<DIR>(src, dst, b0, n, vec);
}

// Shape<DIR>::kBlocksPerSeg blocks per segment: block b converts the span
// (b % kBlocksPerSeg) of segment b / kBlocksPerSeg.
template <uint32_t DIR>
__global__ __launch_bounds__(Shape<DIR>::kLanes) void codec_batch(
    const CodecSeg* __restrict__ segs) {
  constexpr uint32_t B = Shape<DIR>::kBlocksPerSeg;
  const CodecSeg d = segs[blockIdx.x / B];
  convert_span<DIR>(d.src, d.dst, (uint64_t)(blockIdx.x % B) * Shape<DIR>::kSpan, d.n, d.vec);
}

constexpr uint64_t kMaxFlatBlocks = 1u << 20;

using ark::overlaps;

template <uint32_t DIR>
int run_flat(const void* src, void* dst, uint64_t n, void* stream) {
  if (n == 0) return ARK_OPT_OK;
  const uint64_t sb = n * src_size<DIR>(), db = n * dst_size<DIR>();
  if (n > (UINT64_MAX / 8)) return ark::fail(ARK_OPT_EINVAL, "n = %llu too large", (unsigned long long)n);
  if (((uintptr_t)src % src_size<DIR>()) || ((uintptr_t)dst % dst_size<DIR>()))
    return ark::fail(ARK_OPT_EINVAL, "src or dst not aligned to its element");
  int rc;
  if ((rc = ark::check_buffer(src, sb, "src", 0))) return rc;
  if ((rc = ark::check_buffer(dst, db, "dst", 0))) return rc;
  if (overlaps(src, sb, dst, db)) return ark::fail(ARK_OPT_EINVAL, "src and dst overlap");
  {
    const void* d = dst;
    ark::opt_units_invalidate(&d, &db, 1);  // dst may be an optimizer's gradient
  }
  const uint32_t vec = ((((uintptr_t)src | (uintptr_t)dst) & 15u) == 0) ? 1u : 0u;
  uint64_t blocks = (n + Shape<DIR>::kSpan - 1) / Shape<DIR>::kSpan;
  if (blocks > kMaxFlatBlocks) blocks = kMaxFlatBlocks;
  hipLaunchKernelGGL(codec_flat<DIR>, dim3((uint32_t)blocks), dim3(Shape<DIR>::kLanes), 0,
                     (hipStream_t)stream, src, dst, n, vec);
  ARK_HIP(hipGetLastError());
  return ARK_OPT_OK;
}

}  // namespace

struct ark_codec_plan {
  int device = 0;
  hipStream_t stream = nullptr;
  uint32_t direction = 0;
  uint32_t nseg = 0;
  CodecSeg* d_segs = nullptr;
  std::vector<const void*> span_dst;  // what a run writes, for
  std::vector<uint64_t> span_bytes;   // ark::opt_units_invalidate
};

extern "C" {

int ark_hip_dequant_f16_to_f32(const uint16_t* src, float* dst, uint64_t n, void* stream) {
  return run_flat<ARK_CODEC_F16_TO_F32>(src, dst, n, stream);
}

int ark_hip_quant_f32_to_f16(const float* src, uint16_t* dst, uint64_t n, void* stream) {
  return run_flat<ARK_CODEC_F32_TO_F16>(src, dst, n, stream);
}

int ark_codec_plan_create(const ark_codec_span* spans, int32_t n_spans, uint32_t direction,
                          void* stream, ark_codec_plan** out) {
  if (!out) return ark::fail(ARK_OPT_EINVAL, "out is NULL");
  *out = nullptr;
  if (direction != ARK_CODEC_F16_TO_F32 && direction != ARK_CODEC_F32_TO_F16)
    return ark::fail(ARK_OPT_EINVAL, "direction %u unknown", direction);
  if (n_spans < 0 || (n_spans > 0 && !spans))
    return ark::fail(ARK_OPT_EINVAL, "span table is NULL or n_spans < 0");
  const uint64_t ss = direction == ARK_CODEC_F16_TO_F32 ? 2u : 4u;
  const uint64_t ds = direction == ARK_CODEC_F16_TO_F32 ? 4u : 2u;
  std::vector<CodecSeg> segs;
  int rc;
  // One launch converts every span at once, so a dst shared with another
  // span's dst or src would race: every dst must be disjoint from every other
  // span (srcs may overlap each other).  Checked before any device query.
  {
    std::vector<ark::Span> written, readonly;
    uint64_t nseg = 0;
    for (int32_t i = 0; i < n_spans; ++i) {
      const ark_codec_span& s = spans[i];
      if (s.n == 0) continue;
      if (((uintptr_t)s.src % ss) || ((uintptr_t)s.dst % ds))
        return ark::fail(ARK_OPT_EINVAL, "span %d: src or dst not aligned to its element", i);
      if (s.n > (1ull << 48)) return ark::fail(ARK_OPT_EINVAL, "span %d: n too large", i);
      // one launch covers every segment with 512 work-items each, and a
      // launch's work-items stay below 2^32
      nseg += (s.n + kSeg - 1) / kSeg;
      if (nseg > kMaxPlanSegs)
        return ark::fail(ARK_OPT_EINVAL, "too many elements (more than %llu segments of %u)",
                         (unsigned long long)kMaxPlanSegs, kSeg);
      if (overlaps(s.src, s.n * ss, s.dst, s.n * ds))
        return ark::fail(ARK_OPT_EINVAL, "span %d: src and dst overlap", i);
      written.push_back({(uintptr_t)s.dst, (uintptr_t)s.dst + s.n * ds, "dst", i});
      readonly.push_back({(uintptr_t)s.src, (uintptr_t)s.src + s.n * ss, "src", i});
    }
    if ((rc = ark::check_disjoint(std::move(written), std::move(readonly), "span", "the plan")))
      return rc;
  }
  ark::BufferChecker checker;
  for (int32_t i = 0; i < n_spans; ++i) {
    const ark_codec_span& s = spans[i];
    if (s.n == 0) continue;
    if ((rc = checker.check(s.src, s.n * ss, "src", i))) return rc;
    if ((rc = checker.check(s.dst, s.n * ds, "dst", i))) return rc;
    const uint32_t vec = ((((uintptr_t)s.src | (uintptr_t)s.dst) & 15u) == 0) ? 1u : 0u;
    for (uint64_t off = 0; off < s.n; off += kSeg) {
      CodecSeg d;
      d.src = (const char*)s.src + off * ss;
      d.dst = (char*)s.dst + off * ds;
      d.n = (uint32_t)(s.n - off < kSeg ? s.n - off : kSeg);
      d.vec = vec;
      segs.push_back(d);
    }
  }
  int dev = 0;
  if ((rc = ark::current_device_for(stream, &dev))) return rc;
  ark_codec_plan* p = new ark_codec_plan();
  p->device = dev;
  p->stream = (hipStream_t)stream;
  p->direction = direction;
  p->nseg = (uint32_t)segs.size();
  for (int32_t i = 0; i < n_spans; ++i) {
    p->span_dst.push_back(spans[i].dst);
    p->span_bytes.push_back(spans[i].n * ds);
  }
  hipError_t e = hipSuccess;
  if (!segs.empty()) {
    e = hipMalloc(&p->d_segs, segs.size() * sizeof(CodecSeg));
    if (e == hipSuccess)
      e = hipMemcpy(p->d_segs, segs.data(), segs.size() * sizeof(CodecSeg), hipMemcpyHostToDevice);
  }
  if (e != hipSuccess) {
    if (p->d_segs) (void)hipFree(p->d_segs);
    delete p;
    return ark::hip_fail(e, "ark_codec_plan_create");
  }
  *out = p;
  return ARK_OPT_OK;
}

int ark_codec_plan_run(ark_codec_plan* p) {
  if (!p) return ark::fail(ARK_OPT_EINVAL, "plan is NULL");
  if (p->nseg == 0) return ARK_OPT_OK;
  ark::opt_units_invalidate(p->span_dst.data(), p->span_bytes.data(), p->span_dst.size());
  ark::DeviceGuard g(p->device);
  if (!g.ok) return ark::fail(ARK_OPT_EHIP, "cannot select device %d", p->device);
  if (p->direction == ARK_CODEC_F16_TO_F32) {
    typedef Shape<ARK_CODEC_F16_TO_F32> S;
    hipLaunchKernelGGL(codec_batch<ARK_CODEC_F16_TO_F32>, dim3(p->nseg * S::kBlocksPerSeg),
                       dim3(S::kLanes), 0, p->stream, p->d_segs);
  } else {
    typedef Shape<ARK_CODEC_F32_TO_F16> S;
    hipLaunchKernelGGL(codec_batch<ARK_CODEC_F32_TO_F16>, dim3(p->nseg * S::kBlocksPerSeg),
                       dim3(S::kLanes), 0, p->stream, p->d_segs);
  }
  ARK_HIP(hipGetLastError());
  return ARK_OPT_OK;
}

int ark_codec_plan_destroy(ark_codec_plan* p) {
  if (!p) return ARK_OPT_OK;
  int rc = ARK_OPT_OK;
  if (p->d_segs) {
    ark::DeviceGuard g(p->device);
    hipError_t e = hipFree(p->d_segs);
    if (e != hipSuccess) rc = ark::hip_fail(e, "hipFree");
  }
  delete p;
  return rc;
}

}  // extern "C"
