// ark_grad.hip -- gradient accumulation and the embedding scatter-add
// (include/ark_grad.h).
//
//   grad_flat / grad_batch  dst += src in fp32: 12 bytes per element (two
//       reads, one write), HBM bound.  Same shape as the weight codec: a lane
//       takes 4 consecutive elements per access, consecutive lanes
//       consecutive quads; the batch form runs each 4096-element segment of
//       a descriptor table as sixteen one-wave blocks, all tensors in one
//       launch.
//   embed scatter  the loop of bridge.m:922-928 adds row i of dx0 into the
//       embedding row of token i, in increasing i.  Atomics would add in an
//       arbitrary order and change the fp32 sums, so instead:
//         1. key = clamped token, value = position i, and a stable LSD radix
//            sort of (key, i) over the key's bits, which keeps equal keys in
//            increasing i: for up to kBlockSortMax tokens (the reference's
//            2 x 2048 batch) one block sorts them in LDS (block_sort_kernel),
//            beyond that keys_kernel and hipCUB's device radix sort;
//         3. gather_kernel: the dx0 rows copied in sorted order into a
//            workspace, so every run of equal keys is contiguous;
//         4. run_kernel: one 256-lane block per (run of equal keys,
//            256-column tile) finds the run's end by binary search, loads the
//            embedding row once, adds the run's rows in sorted (= original)
//            order and stores it once.  A run of kLongRun rows or more gives
//            each lane one column and keeps kColRows rows' loads in flight
//            (the run is a sequential fp32 chain per column, so its time is
//            load round trips); a shorter run is done by the first wave alone
//            with 16-byte accesses.
//       Every element therefore sees the same additions in the same order as
//       the CPU loop, and the result is bit-identical.
#include <string.h>

#include <hipcub/hipcub.hpp>
#include <vector>

#include "ark_common.hpp"
#include "ark_device.hpp"
#include "ark_grad.h"

namespace {

using namespace ark::dev;
using ark::fail;

constexpr int kThreads = 256;
constexpr int kPerLane = 4;
constexpr uint32_t kSeg = 4096;
constexpr int kWave = 64;
constexpr uint32_t kBlocksPerSeg = kSeg / (kWave * kPerLane);  // 16
constexpr int kTileCols = 256;  // run_kernel: columns per block
constexpr int kLongRun = 8;     // runs of at least this many rows: one column per lane
// Rows in flight per lane on a long run.  Measured on MI355X (4096 tokens,
// d 768): 60 rows with one column per lane run a single 4096-row run in 73 us
// against 400 us for 32 rows of four columns; more than 60 gain nothing, a
// wave keeping at most 63 vector loads outstanding.
constexpr int kColRows = 60;

struct GradSeg {
  float* dst;
  const float* src;
  uint32_t n;    // elements, 1..kSeg
  uint32_t vec;  // dst and src 16-byte aligned
};
static_assert(sizeof(GradSeg) == 24, "24-byte descriptor");

__device__ __forceinline__ void add4(float* dst, const float* src) {
  f32x4 a = ld_nt<f32x4>(dst);
  const f32x4 b = ld_nt<f32x4>(src);
  a.x = a.x + b.x;
  a.y = a.y + b.y;
  a.z = a.z + b.z;
  a.w = a.w + b.w;
  st_nt<f32x4>(dst, a);
}

__device__ __forceinline__ void add1(float* dst, const float* src) {
  st_g<float>(dst, ld_g<float>(dst) + ld_g<float>(src));
}

__global__ __launch_bounds__(kThreads) void grad_flat(float* __restrict__ dst,
                                                      const float* __restrict__ src, uint64_t n,
                                                      uint32_t vec) {
  const uint64_t nquad = (n + kPerLane - 1) / kPerLane;
  const uint64_t stride = (uint64_t)gridDim.x * kThreads;
  for (uint64_t q = (uint64_t)blockIdx.x * kThreads + threadIdx.x; q < nquad; q += stride) {
    const uint64_t e0 = q * kPerLane;
    if (vec && e0 + kPerLane <= n) {
      add4(dst + e0, src + e0);
    } else {
      for (int j = 0; j < kPerLane; ++j)
        if (e0 + j < n) add1(dst + e0 + j, src + e0 + j);
    }
  }
}

// Sixteen one-wave blocks per segment, one quad per lane: block b adds
// elements [(b % 16) * 256 + 4l, +4) of segment b / 16 (the shape the sweep
// measured fastest for two read streams and one write stream).
__global__ __launch_bounds__(kWave) void grad_batch(const GradSeg* __restrict__ segs) {
  const GradSeg d = segs[blockIdx.x / kBlocksPerSeg];
  const uint32_t e0 = ((blockIdx.x % kBlocksPerSeg) * kWave + threadIdx.x) * kPerLane;
  if (e0 >= d.n) return;
  if (d.vec && e0 + kPerLane <= d.n) {
    add4(d.dst + e0, d.src + e0);
  } else {
    for (int j = 0; j < kPerLane; ++j)
      if (e0 + j < d.n) add1(d.dst + e0 + j, d.src + e0 + j);
  }
}

// Up to kBlockSortMax tokens: one block loads them (key = clamped token,
// value = position, bridge.m:923), sorts the pairs over bits [0, end_bit)
// with the stable block radix sort, and writes them out.  Input and output
// are in blocked order (thread t holds positions t*kSortItems..), so the
// stable sort keeps equal keys in increasing position.  Padding past n takes
// the all-ones key: it ties with the largest real key at most and, coming
// later in the input, sorts after it.
constexpr int kSortThreads = 1024;
constexpr int kSortItems = 4;
constexpr uint32_t kBlockSortMax = kSortThreads * kSortItems;  // 4096

__global__ __launch_bounds__(kSortThreads) void block_sort_kernel(
    const uint32_t* __restrict__ tokens, uint32_t n, uint32_t vocab, int end_bit,
    uint32_t* __restrict__ skeys, uint32_t* __restrict__ svals) {
  typedef hipcub::BlockRadixSort<uint32_t, kSortThreads, kSortItems, uint32_t> Sort;
  __shared__ typename Sort::TempStorage tmp;
  uint32_t k[kSortItems], v[kSortItems];
#pragma unroll
  for (int j = 0; j < kSortItems; ++j) {
    const uint32_t i = threadIdx.x * kSortItems + j;
    uint32_t t = 0xFFFFFFFFu;
    if (i < n) {
      t = ld_g<uint32_t>(tokens + i);
      t = t < vocab ? t : 0u;
    }
    k[j] = t;
    v[j] = i;
  }
  Sort(tmp).Sort(k, v, 0, end_bit);
#pragma unroll
  for (int j = 0; j < kSortItems; ++j) {
    const uint32_t i = threadIdx.x * kSortItems + j;
    if (i < n) {
      skeys[i] = k[j];
      svals[i] = v[j];
    }
  }
}

// bridge.m:923: t = tokens[i] < vocab ? tokens[i] : 0
__global__ __launch_bounds__(kThreads) void keys_kernel(const uint32_t* __restrict__ tokens,
                                                        uint32_t n, uint32_t vocab,
                                                        uint32_t* __restrict__ keys,
                                                        uint32_t* __restrict__ vals) {
  const uint32_t i = blockIdx.x * kThreads + threadIdx.x;
  if (i >= n) return;
  const uint32_t t = ld_g<uint32_t>(tokens + i);
  keys[i] = t < vocab ? t : 0u;
  vals[i] = i;
}

// Row q of xs = row svals[q] of dx0 (d floats each); one block per row.
// vec: d % 4 == 0 and dx0 16-byte aligned (xs is 256-byte aligned).
__global__ __launch_bounds__(kThreads) void gather_kernel(const float* __restrict__ dx0,
                                                          const uint32_t* __restrict__ svals,
                                                          uint32_t d, uint32_t vec,
                                                          float* __restrict__ xs) {
  const float* src = dx0 + (uint64_t)svals[blockIdx.x] * d;
  float* dst = xs + (uint64_t)blockIdx.x * d;
  if (vec) {
    for (uint32_t c = threadIdx.x * kPerLane; c < d; c += kThreads * kPerLane)
      st_g<f32x4>(dst + c, ld_nt<f32x4>(src + c));
  } else {
    for (uint32_t c = threadIdx.x; c < d; c += kThreads) st_g<float>(dst + c, ld_g<float>(src + c));
  }
}

// Block (p, tile): if sorted position p starts a run of equal keys, add the
// run's rows (xs rows p.., in sorted order, which is increasing i) into
// columns [tile*256, tile*256 + 256) of the key's embedding row.  vec:
// d % 4 == 0 and g 16-byte aligned.
__global__ __launch_bounds__(kTileCols) void run_kernel(float* __restrict__ g, uint32_t d,
                                                        const float* __restrict__ xs,
                                                        const uint32_t* __restrict__ skeys,
                                                        uint32_t n, uint32_t vec) {
  const uint32_t p = blockIdx.x;
  const uint32_t t = skeys[p];
  if (p > 0 && skeys[p - 1] == t) return;
  // run end: the first sorted position with a larger key (binary search)
  uint32_t lo = p, hi = n;  // skeys[lo] == t; hi is past the run
  while (hi - lo > 1) {
    const uint32_t mid = lo + ((hi - lo) >> 1);
    if (skeys[mid] == t)
      lo = mid;
    else
      hi = mid;
  }
  const uint32_t len = hi - p;
  const float* x = xs + (uint64_t)p * d;  // the run's rows, contiguous
  if (len >= (uint32_t)kLongRun) {
    const uint32_t c = blockIdx.y * kTileCols + threadIdx.x;
    if (c >= d) return;
    float* gp = g + (uint64_t)t * d + c;
    float acc = ld_g<float>(gp);
    uint32_t k = 0;
    for (; k + kColRows <= len; k += kColRows) {
      float v[kColRows];
#pragma unroll
      for (int j = 0; j < kColRows; ++j) v[j] = ld_g<float>(x + (uint64_t)(k + j) * d + c);
#pragma unroll
      for (int j = 0; j < kColRows; ++j) acc = acc + v[j];
    }
    if (k < len) {  // the last len % kColRows rows, loaded together as well
      float v[kColRows];
#pragma unroll
      for (int j = 0; j < kColRows; ++j)
        if (k + j < len) v[j] = ld_g<float>(x + (uint64_t)(k + j) * d + c);
#pragma unroll
      for (int j = 0; j < kColRows; ++j)
        if (k + j < len) acc = acc + v[j];
    }
    st_g<float>(gp, acc);
    return;
  }
  if (threadIdx.x >= kWave) return;  // a short run: the first wave, four columns per lane
  const uint32_t c0 = blockIdx.y * kTileCols + threadIdx.x * kPerLane;
  if (c0 >= d) return;
  float* gp = g + (uint64_t)t * d + c0;
  if (vec) {  // c0 + 4 <= d since d % 4 == 0
    f32x4 acc = ld_g<f32x4>(gp);
    f32x4 v[kLongRun - 1];
#pragma unroll
    for (int j = 0; j < kLongRun - 1; ++j)
      if ((uint32_t)j < len) v[j] = ld_g<f32x4>(x + (uint64_t)j * d + c0);
#pragma unroll
    for (int j = 0; j < kLongRun - 1; ++j) {
      if ((uint32_t)j < len) {
        acc.x = acc.x + v[j].x;
        acc.y = acc.y + v[j].y;
        acc.z = acc.z + v[j].z;
        acc.w = acc.w + v[j].w;
      }
    }
    st_g<f32x4>(gp, acc);
  } else {
    const int nc = d - c0 < (uint32_t)kPerLane ? (int)(d - c0) : kPerLane;
    for (int c = 0; c < nc; ++c) {
      float acc = ld_g<float>(gp + c);
      for (uint32_t j = 0; j < len; ++j) acc = acc + ld_g<float>(x + (uint64_t)j * d + c0 + c);
      st_g<float>(gp + c, acc);
    }
  }
}

constexpr uint64_t kMaxFlatBlocks = 1u << 20;

using ark::overlaps;

using ark::StreamBuf;

}  // namespace

struct ark_grad_plan {
  int device = 0;
  hipStream_t stream = nullptr;
  uint32_t nseg = 0;
  GradSeg* d_segs = nullptr;
};

extern "C" {

int ark_grad_accumulate(float* dst, const float* src, uint64_t n, void* stream) {
  if (n == 0) return ARK_OPT_OK;
  if (n > (1ull << 60)) return fail(ARK_OPT_EINVAL, "n = %llu too large", (unsigned long long)n);
  if (((uintptr_t)dst & 3u) || ((uintptr_t)src & 3u))
    return fail(ARK_OPT_EINVAL, "dst or src not 4-byte aligned");
  int rc;
  if ((rc = ark::check_buffer(dst, n * 4, "dst", 0))) return rc;
  if ((rc = ark::check_buffer(src, n * 4, "src", 0))) return rc;
  if (overlaps(dst, n * 4, src, n * 4)) return fail(ARK_OPT_EINVAL, "dst and src overlap");
  const uint32_t vec = ((((uintptr_t)dst | (uintptr_t)src) & 15u) == 0) ? 1u : 0u;
  uint64_t blocks = ((n + kPerLane - 1) / kPerLane + kThreads - 1) / kThreads;
  if (blocks > kMaxFlatBlocks) blocks = kMaxFlatBlocks;
  hipLaunchKernelGGL(grad_flat, dim3((uint32_t)blocks), dim3(kThreads), 0, (hipStream_t)stream,
                     dst, src, n, vec);
  ARK_HIP(hipGetLastError());
  return ARK_OPT_OK;
}

int ark_grad_plan_create(const ark_grad_span* spans, int32_t n_spans, void* stream,
                         ark_grad_plan** out) {
  if (!out) return fail(ARK_OPT_EINVAL, "out is NULL");
  *out = nullptr;
  if (n_spans < 0 || (n_spans > 0 && !spans))
    return fail(ARK_OPT_EINVAL, "span table is NULL or n_spans < 0");
  std::vector<GradSeg> segs;
  ark::BufferChecker checker;
  int rc;
  for (int32_t i = 0; i < n_spans; ++i) {
    const ark_grad_span& s = spans[i];
    if (s.n == 0) continue;
    if (((uintptr_t)s.dst & 3u) || ((uintptr_t)s.src & 3u))
      return fail(ARK_OPT_EINVAL, "span %d: dst or src not 4-byte aligned", i);
    if (s.n > (1ull << 48)) return fail(ARK_OPT_EINVAL, "span %d: n too large", i);
    if ((rc = checker.check(s.dst, s.n * 4, "dst", i))) return rc;
    if ((rc = checker.check(s.src, s.n * 4, "src", i))) return rc;
    if (overlaps(s.dst, s.n * 4, s.src, s.n * 4))
      return fail(ARK_OPT_EINVAL, "span %d: dst and src overlap", i);
    const uint32_t vec = ((((uintptr_t)s.dst | (uintptr_t)s.src) & 15u) == 0) ? 1u : 0u;
    for (uint64_t off = 0; off < s.n; off += kSeg) {
      GradSeg d;
      d.dst = s.dst + off;
      d.src = s.src + off;
      d.n = (uint32_t)(s.n - off < kSeg ? s.n - off : kSeg);
      d.vec = vec;
      segs.push_back(d);
      if (segs.size() > 0x7FFFFFFFu / kBlocksPerSeg)
        return fail(ARK_OPT_EINVAL, "too many elements");
    }
  }
  ark_grad_plan* p = new ark_grad_plan();
  p->stream = (hipStream_t)stream;
  p->nseg = (uint32_t)segs.size();
  hipError_t e = hipGetDevice(&p->device);
  if (e == hipSuccess && !segs.empty()) {
    e = hipMalloc(&p->d_segs, segs.size() * sizeof(GradSeg));
    if (e == hipSuccess)
      e = hipMemcpy(p->d_segs, segs.data(), segs.size() * sizeof(GradSeg), hipMemcpyHostToDevice);
  }
  if (e != hipSuccess) {
    if (p->d_segs) (void)hipFree(p->d_segs);
    delete p;
    return ark::hip_fail(e, "ark_grad_plan_create");
  }
  *out = p;
  return ARK_OPT_OK;
}

int ark_grad_plan_run(ark_grad_plan* p) {
  if (!p) return fail(ARK_OPT_EINVAL, "plan is NULL");
  if (p->nseg == 0) return ARK_OPT_OK;
  ark::DeviceGuard g(p->device);
  if (!g.ok) return fail(ARK_OPT_EHIP, "cannot select device %d", p->device);
  hipLaunchKernelGGL(grad_batch, dim3(p->nseg * kBlocksPerSeg), dim3(kWave), 0, p->stream,
                     p->d_segs);
  ARK_HIP(hipGetLastError());
  return ARK_OPT_OK;
}

int ark_grad_plan_destroy(ark_grad_plan* p) {
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

int ark_grad_embed_scatter(float* embed_grad, uint32_t vocab, uint32_t d, const uint32_t* tokens,
                           const float* dx0, uint32_t batch_seq, void* stream) {
  if (batch_seq == 0 || d == 0) return ARK_OPT_OK;
  if (vocab == 0) return fail(ARK_OPT_EINVAL, "vocab is 0");
  if (batch_seq > 0x7FFFFFFFu) return fail(ARK_OPT_EINVAL, "batch_seq too large");
  if (((uint64_t)d + kTileCols - 1) / kTileCols > 65535u) return fail(ARK_OPT_EINVAL, "d too large");
  if (((uintptr_t)embed_grad & 3u) || ((uintptr_t)dx0 & 3u) || ((uintptr_t)tokens & 3u))
    return fail(ARK_OPT_EINVAL, "embed_grad, dx0 or tokens not 4-byte aligned");
  const uint64_t gbytes = (uint64_t)vocab * d * 4, xbytes = (uint64_t)batch_seq * d * 4;
  int rc;
  if ((rc = ark::check_buffer(embed_grad, gbytes, "embed_grad", 0))) return rc;
  if ((rc = ark::check_buffer(dx0, xbytes, "dx0", 0))) return rc;
  if ((rc = ark::check_buffer(tokens, (uint64_t)batch_seq * 4, "tokens", 0))) return rc;
  if (overlaps(embed_grad, gbytes, dx0, xbytes))
    return fail(ARK_OPT_EINVAL, "embed_grad and dx0 overlap");
  hipStream_t s = (hipStream_t)stream;
  int end_bit = 1;
  while (end_bit < 32 && ((vocab - 1u) >> end_bit) != 0u) ++end_bit;
  const int n = (int)batch_seq;
  const bool block_sort = batch_seq <= kBlockSortMax;
  size_t temp = 0;
  if (!block_sort)
    ARK_HIP(hipcub::DeviceRadixSort::SortPairs(nullptr, temp, (const uint32_t*)nullptr,
                                               (uint32_t*)nullptr, (const uint32_t*)nullptr,
                                               (uint32_t*)nullptr, n, 0, end_bit, s));
  const size_t arr = ark::align_up((size_t)batch_seq * 4, 256);
  const size_t rows = ark::align_up((size_t)xbytes, 256);
  const size_t ws_bytes = 4 * arr + rows + temp;
  StreamBuf ws;
  hipError_t e = ws.alloc(ws_bytes, s);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return fail(ARK_OPT_ENOMEM, "hipMallocAsync(%zu) for the scatter failed", ws_bytes);
  }
  uint32_t* keys = (uint32_t*)ws.p;
  uint32_t* vals = (uint32_t*)((char*)ws.p + arr);
  uint32_t* skeys = (uint32_t*)((char*)ws.p + 2 * arr);
  uint32_t* svals = (uint32_t*)((char*)ws.p + 3 * arr);
  float* xs = (float*)((char*)ws.p + 4 * arr);
  void* tmp = (char*)ws.p + 4 * arr + rows;
  if (block_sort) {
    hipLaunchKernelGGL(block_sort_kernel, dim3(1), dim3(kSortThreads), 0, s, tokens, batch_seq,
                       vocab, end_bit, skeys, svals);
    ARK_HIP(hipGetLastError());
  } else {
    hipLaunchKernelGGL(keys_kernel, dim3((batch_seq + kThreads - 1) / kThreads), dim3(kThreads),
                       0, s, tokens, batch_seq, vocab, keys, vals);
    ARK_HIP(hipGetLastError());
    ARK_HIP(hipcub::DeviceRadixSort::SortPairs(tmp, temp, keys, skeys, vals, svals, n, 0,
                                               end_bit, s));
  }
  const uint32_t gvec = ((d % 4u) == 0 && (((uintptr_t)dx0 & 15u) == 0)) ? 1u : 0u;
  hipLaunchKernelGGL(gather_kernel, dim3(batch_seq), dim3(kThreads), 0, s, dx0, svals, d, gvec,
                     xs);
  ARK_HIP(hipGetLastError());
  const uint32_t vec = ((d % 4u) == 0 && (((uintptr_t)embed_grad & 15u) == 0)) ? 1u : 0u;
  const dim3 grid(batch_seq, (d + kTileCols - 1) / kTileCols);
  hipLaunchKernelGGL(run_kernel, grid, dim3(kTileCols), 0, s, embed_grad, d, xs, skeys,
                     batch_seq, vec);
  ARK_HIP(hipGetLastError());
  return ARK_OPT_OK;
}

}  // extern "C"
