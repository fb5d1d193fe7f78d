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
//            increasing i: for up to kSortTile tokens (the reference's
//            2 x 2048 batch) one block sorts them in LDS (block_sort_kernel),
//            beyond that one hist/scan/scatter launch triple per 8-bit digit;
//         2. gather_kernel: the dx0 rows copied in sorted order into a
//            workspace, so every run of equal keys is contiguous;
//         3. run_kernel: one 256-lane block per (run of equal keys,
//            256-column tile) finds the run's end by binary search, loads the
//            embedding row once, adds the run's rows in sorted (= original)
//            order and stores it once.  A run of kLongRun rows or more gives
//            each lane one column and keeps kColRows rows' loads in flight
//            (the run is a sequential fp32 chain per column, so its time is
//            load round trips); a shorter run is done by the first wave alone
//            with 16-byte accesses.
//       Every element therefore sees the same additions in the same order as
//       the CPU loop, and the result is bit-identical.
#include <stdlib.h>
#include <string.h>

#include <mutex>
#include <vector>

#include "ark_common.hpp"
#include "ark_device.hpp"
#include "ark_grad.h"
#include "ark_opt_internal.hpp"

namespace {

using namespace ark::dev;
using ark::fail;

constexpr int kThreads = 256;
constexpr int kPerLane = 4;
constexpr uint32_t kSeg = 4096;
constexpr int kWave = 64;
constexpr uint32_t kBlocksPerSeg = kSeg / (kWave * kPerLane);  // 16
// Resident one-wave grad_batch blocks per CU, held by a dynamic-LDS
// reservation the kernel never touches.  On MI355X the accumulation over
// EKO-237M's 272 gradients takes 0.4270 ms with every wave slot (32 per CU),
// 0.4226-0.4237 ms at 22-28 per CU and 0.434 ms at 20.  grad_batch_units keeps
// every slot: its per-wave tree of squares shows at fewer waves (470.7
// against 443.0 us at 24 per CU, same box).
constexpr int kPlanBlocksPerCu = 24;
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

// ---- the norm's units from the kernels that finish the gradients ----------
// (ark_opt_internal.hpp).  A unit is 256 consecutive elements of an
// optimizer segment; its value is the pairwise f64 tree of the squares of the
// unscaled gradients (zero past the segment's end), NaN if one of them is inf
// or NaN.  Lane l of a wave holds elements [4l, 4l + 4) of the unit: the
// pair sums of its quad, then the lanes in lane order.

// The unit of the wave's four-per-lane values x (0 past the end), unscaled
// by inv; written by lane 0.
__device__ __forceinline__ void store_unit(const float (&x)[kPerLane], float inv, double* unit) {
  uint32_t bad = 0;
  double q[kPerLane];
#pragma unroll
  for (int j = 0; j < kPerLane; ++j) {
    bad |= (__float_as_uint(x[j]) & 0x7F800000u) == 0x7F800000u ? 1u : 0u;
    const float gu = x[j] * inv;
    q[j] = (double)gu * (double)gu;
  }
  double sum = (q[0] + q[1]) + (q[2] + q[3]);
#pragma unroll
  for (int st = 0; st < 6; ++st) sum = sum + __shfl_xor(sum, 1 << st);
  const bool any_bad = __ballot(bad) != 0ull;
  if (threadIdx.x == 0) *unit = any_bad ? __builtin_nan("") : sum;
}

// 1 / loss_scale (training.rs:244) unless the tensor keeps its scale.
__device__ __forceinline__ float unit_inv(const ark_opt_state* state, uint32_t seg_flags) {
  return (seg_flags & ark::kSegNoUnscale) ? 1.0f : 1.0f / state->loss_scale;
}

// grad_batch's add (same blocks, same accesses) plus the unit of the 256
// elements each wave finishes: the final accumulation before a step.  The
// plan's segments are the optimizer handle's, one for one.  (Writing the
// gradients the step's AdamW pass reads first with cache-allocating stores,
// last segment first, measured no faster: the pass gained nothing from them,
// unlike from the norm pass's cache-allocating loads.)
__global__ __launch_bounds__(kWave) void grad_batch_units(const GradSeg* __restrict__ segs,
                                                          const ark::SegDesc* __restrict__ osegs,
                                                          const ark_opt_state* __restrict__ state,
                                                          double* __restrict__ units) {
  const uint32_t s = blockIdx.x / kBlocksPerSeg, r = blockIdx.x % kBlocksPerSeg;
  const GradSeg d = segs[s];
  if (r * (uint32_t)(kWave * kPerLane) >= d.n) return;  // the unit lies past the end
  const uint32_t e0 = (r * kWave + threadIdx.x) * kPerLane;
  float x[kPerLane] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (d.vec && e0 + kPerLane <= d.n) {
    f32x4 a = ld_nt<f32x4>(d.dst + e0);
    const f32x4 b = ld_nt<f32x4>(d.src + e0);
    a.x = a.x + b.x;
    a.y = a.y + b.y;
    a.z = a.z + b.z;
    a.w = a.w + b.w;
    st_nt<f32x4>(d.dst + e0, a);
    x[0] = a.x;
    x[1] = a.y;
    x[2] = a.z;
    x[3] = a.w;
  } else {
#pragma unroll
    for (int j = 0; j < kPerLane; ++j) {
      if (e0 + j < d.n) {
        const float v = ld_g<float>(d.dst + e0 + j) + ld_g<float>(d.src + e0 + j);
        st_g<float>(d.dst + e0 + j, v);
        x[j] = v;
      }
    }
  }
  store_unit(x, unit_inv(state, osegs[s].flags), units + (uint64_t)s * kBlocksPerSeg + r);
}

// After the scatter's run_kernel: the unit of every (embedding row, 256-column
// tile) the scatter changed, from the row's final values.  d % 256 == 0, so a
// tile is one unit: row t, tile c is the tensor's unit t * (d / 256) + c.  One
// wave per (sorted position, tile); positions that do not start a run exit.
__global__ __launch_bounds__(kWave) void units_rows_kernel(const float* __restrict__ g, uint32_t d,
                                                           const uint32_t* __restrict__ skeys,
                                                           uint32_t vec,
                                                           const ark_opt_state* __restrict__ state,
                                                           uint32_t seg_flags,
                                                           double* __restrict__ units) {
  const uint32_t p = blockIdx.x;
  const uint32_t t = skeys[p];
  if (p > 0 && skeys[p - 1] == t) return;
  const uint32_t c0 = blockIdx.y * kTileCols + threadIdx.x * kPerLane;
  const float* gp = g + (uint64_t)t * d + c0;
  float x[kPerLane];
  if (vec) {
    const f32x4 a = ld_g<f32x4>(gp);
    x[0] = a.x;
    x[1] = a.y;
    x[2] = a.z;
    x[3] = a.w;
  } else {
#pragma unroll
    for (int j = 0; j < kPerLane; ++j) x[j] = ld_g<float>(gp + j);
  }
  store_unit(x, unit_inv(state, seg_flags),
             units + (uint64_t)t * (d / kTileCols) + blockIdx.y);
}

// ---- stable LSD radix sort of (clamped token, position) ------------------
// A block of kSortThreads threads holds a tile of kSortTile items: item j of
// lane l of wave w sits at tile position w*256 + j*64 + l, so the order
// (wave, item, lane) is the position order.  One pass sorts the tile by
// kRadixBits bits of the key:
//   rank   per item, how many items of its wave with the same digit precede
//          it, from ballots of the digit's bits and the wave's running count
//          of each digit in LDS (wave_rank), which ends as the (digit, wave)
//          count table;
//   scan   an exclusive block scan of that table gives every (digit, wave)
//          the number of tile items before it in (digit, position) order;
//   place  item -> scan[digit, wave] + rank.
// Equal digits keep their position order, so each pass is stable and the
// passes from the low bits up (LSD) leave the keys sorted with equal keys in
// increasing position: the order in which bridge.m:922-928's loop visits a
// token's rows.  Up to one tile (the reference's 2 x 2048 batch) one block
// does every pass in LDS (block_sort_kernel); past that each pass is three
// launches: per-tile digit counts (sort_hist_kernel), their exclusive scan
// in (digit, tile) order (sort_scan_kernel), and the tile-local rank plus the
// scanned count as the global destination (sort_scatter_kernel).
constexpr int kSortThreads = 1024;
constexpr int kSortWaves = kSortThreads / kWave;                // 16
constexpr int kSortItems = 4;
constexpr uint32_t kSortTile = kSortThreads * kSortItems;       // 4096
constexpr int kRadixBits = 8;
constexpr uint32_t kRadix = 1u << kRadixBits;                   // 256
constexpr uint32_t kHist = kRadix * kSortWaves;                 // 4096
constexpr uint32_t kPadKey = 0xFFFFFFFFu;
static_assert(kHist == kSortThreads * 4, "block_exclusive takes 4 entries per thread");
static_assert(kSortWaves * kSortItems * kWave == (int)kSortTile, "tile layout");

// bridge.m:923: t = tokens[i] < vocab ? tokens[i] : 0
__device__ __forceinline__ uint32_t clamp_token(uint32_t t, uint32_t vocab) {
  return t < vocab ? t : 0u;
}

__device__ __forceinline__ uint32_t tile_pos(uint32_t wave, int j, uint32_t lane) {
  return wave * (kSortItems * kWave) + (uint32_t)j * kWave + lane;
}

// The (digit, wave) table in LDS: wave w's counter of digit d at
// w * kHistStride + d; the stride of kRadix + 1 words puts the counters of
// different digits of one wave in different banks.
constexpr uint32_t kHistStride = kRadix + 1;
constexpr uint32_t kHistWords = kSortWaves * kHistStride;
__device__ __forceinline__ uint32_t hist_at(uint32_t d, uint32_t w) { return w * kHistStride + d; }

// rank[j] = the number of items of this wave with digit dig[j] that precede
// item j in (item, lane) order; on return the wave's counters hold its count
// of every digit.  Round j matches item j's digit across the lanes with
// kRadixBits ballots, adds the wave's running count of that digit, and the
// digit's last lane in the round writes the new count.  A round's reads all
// come before its writes (one wave, LDS accesses in program order), and
// different waves touch different counters.
__device__ __forceinline__ void wave_rank(const uint32_t (&dig)[kSortItems],
                                          uint32_t (&rank)[kSortItems], uint32_t* hist,
                                          uint32_t wave) {
  const uint32_t lane = __lane_id();
  const uint64_t below = (1ull << lane) - 1ull;
  const uint64_t above = ~((2ull << lane) - 1ull);  // lane 63: 2 << 63 wraps to 0
#pragma unroll
  for (int j = 0; j < kSortItems; ++j) {
    uint64_t same = ~0ull;  // lanes whose item j has digit dig[j]
#pragma unroll
    for (int b = 0; b < kRadixBits; ++b) {
      const uint32_t bit = (dig[j] >> b) & 1u;
      const uint64_t ones = __ballot(bit);
      same &= bit ? ones : ~ones;
    }
    uint32_t* c = hist + hist_at(dig[j], wave);
    const uint32_t r = *c + (uint32_t)__popcll(same & below);
    rank[j] = r;
    if ((same & above) == 0ull) *c = r + 1u;
  }
}

// Exclusive prefix over the block's kSortThreads x 4 values in thread order
// (thread t holds entries 4t .. 4t+3): e[i] becomes carry plus every entry
// before it; returns carry plus all entries.  Every thread of the block
// calls it; wsum is LDS scratch of kSortWaves words.
__device__ __forceinline__ uint32_t block_exclusive(uint32_t (&e)[4], uint32_t* wsum,
                                                    uint32_t carry) {
  const uint32_t lane = __lane_id(), wave = threadIdx.x / kWave;
  const uint32_t s = e[0] + e[1] + e[2] + e[3];
  uint32_t incl = s;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const uint32_t y = __shfl_up(incl, o, kWave);
    if (lane >= (uint32_t)o) incl += y;
  }
  if (lane == kWave - 1) wsum[wave] = incl;
  __syncthreads();
  uint32_t before = carry, total = carry;
#pragma unroll
  for (int w = 0; w < kSortWaves; ++w) {
    const uint32_t x = wsum[w];
    if ((uint32_t)w < wave) before += x;
    total += x;
  }
  uint32_t run = before + incl - s;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t x = e[i];
    e[i] = run;
    run += x;
  }
  __syncthreads();  // wsum is free for the next call
  return total;
}

// One pass of the tile in registers: zero the (digit, wave) table, rank,
// scan.  On return hist[hist_at(d, w)] holds the number of tile items
// (padding included) before (digit d, wave w) in (digit, position) order.
__device__ __forceinline__ void tile_pass(const uint32_t (&dig)[kSortItems],
                                          uint32_t (&rank)[kSortItems], uint32_t* hist,
                                          uint32_t* wsum) {
  const uint32_t t = threadIdx.x, wave = t / kWave;
  // thread t scans entries 4t .. 4t+3 of the (digit, wave) order: digit
  // t / 4, waves 4 (t % 4) .. 4 (t % 4) + 3
  const uint32_t sd = t / 4u, sw = 4u * (t % 4u);
#pragma unroll
  for (int i = 0; i < 4; ++i) hist[hist_at(sd, sw + i)] = 0u;
  __syncthreads();
  wave_rank(dig, rank, hist, wave);
  __syncthreads();
  uint32_t e[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) e[i] = hist[hist_at(sd, sw + i)];
  block_exclusive(e, wsum, 0u);
#pragma unroll
  for (int i = 0; i < 4; ++i) hist[hist_at(sd, sw + i)] = e[i];
  __syncthreads();
}

// Up to kSortTile tokens: one block sorts (key = clamped token, value =
// position) over bits [0, end_bit) in LDS and writes the first n pairs.
// Positions past n take the all-ones key: its digit is the largest in every
// pass and it comes after every real item, so it sorts after them all.
__global__ __launch_bounds__(kSortThreads) void block_sort_kernel(
    const uint32_t* __restrict__ tokens, uint32_t n, uint32_t vocab, int end_bit,
    uint32_t* __restrict__ skeys, uint32_t* __restrict__ svals) {
  __shared__ uint32_t s_keys[kSortTile], s_vals[kSortTile], s_hist[kHistWords],
      s_wsum[kSortWaves];
  const uint32_t lane = __lane_id(), wave = threadIdx.x / kWave;
  uint32_t k[kSortItems], v[kSortItems], dg[kSortItems], r[kSortItems];
#pragma unroll
  for (int j = 0; j < kSortItems; ++j) {
    const uint32_t p = tile_pos(wave, j, lane);
    k[j] = p < n ? clamp_token(ld_g<uint32_t>(tokens + p), vocab) : kPadKey;
    v[j] = p;
  }
  for (int shift = 0; shift < end_bit; shift += kRadixBits) {
#pragma unroll
    for (int j = 0; j < kSortItems; ++j) dg[j] = (k[j] >> shift) & (kRadix - 1u);
    tile_pass(dg, r, s_hist, s_wsum);
#pragma unroll
    for (int j = 0; j < kSortItems; ++j) {
      const uint32_t dst = s_hist[hist_at(dg[j], wave)] + r[j];
      s_keys[dst] = k[j];
      s_vals[dst] = v[j];
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kSortItems; ++j) {
      const uint32_t p = tile_pos(wave, j, lane);
      k[j] = s_keys[p];
      v[j] = s_vals[p];
    }
  }
#pragma unroll
  for (int j = 0; j < kSortItems; ++j) {
    const uint32_t p = tile_pos(wave, j, lane);
    if (p < n) {
      skeys[p] = k[j];
      svals[p] = v[j];
    }
  }
}

// counts[d * tiles + tile] = the items of the tile whose key has digit d at
// this pass: the waves' counters of wave_rank, summed over the waves.
// from_tokens: the keys are the clamped tokens (first pass).  Positions past
// n count as the padding digit, which sort_scatter_kernel never places, and
// are taken off again.
__global__ __launch_bounds__(kSortThreads) void sort_hist_kernel(
    const uint32_t* __restrict__ keys, uint32_t from_tokens, uint32_t n, uint32_t vocab,
    int shift, uint32_t* __restrict__ counts, uint32_t tiles) {
  __shared__ uint32_t s_hist[kHistWords];
  const uint32_t t = threadIdx.x, lane = __lane_id(), wave = t / kWave;
  const uint32_t sd = t / 4u, sw = 4u * (t % 4u);
#pragma unroll
  for (int i = 0; i < 4; ++i) s_hist[hist_at(sd, sw + i)] = 0u;
  uint32_t dg[kSortItems], r[kSortItems];
#pragma unroll
  for (int j = 0; j < kSortItems; ++j) {
    const uint32_t p = blockIdx.x * kSortTile + tile_pos(wave, j, lane);
    uint32_t key = kPadKey;
    if (p < n) {
      key = ld_g<uint32_t>(keys + p);
      if (from_tokens) key = clamp_token(key, vocab);
    }
    dg[j] = (key >> shift) & (kRadix - 1u);
  }
  __syncthreads();
  wave_rank(dg, r, s_hist, wave);
  __syncthreads();
  if (t < kRadix) {
    uint32_t c = 0;
#pragma unroll
    for (int w = 0; w < kSortWaves; ++w) c += s_hist[hist_at(t, w)];
    if (t == kRadix - 1u) {  // the padding: only the last tile has any
      const uint64_t end = (uint64_t)(blockIdx.x + 1) * kSortTile;
      c -= end > n ? (uint32_t)(end - n) : 0u;
    }
    counts[t * tiles + blockIdx.x] = c;
  }
}

// counts[0, total) <- its exclusive prefix sums: one block, kSortTile
// entries per round with the running total carried.
__global__ __launch_bounds__(kSortThreads) void sort_scan_kernel(uint32_t* __restrict__ counts,
                                                                 uint32_t total) {
  __shared__ uint32_t wsum[kSortWaves];
  uint32_t carry = 0;
  for (uint32_t base = 0; base < total; base += kSortTile) {
    uint32_t e[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t q = base + 4u * threadIdx.x + (uint32_t)i;
      e[i] = q < total ? counts[q] : 0u;
    }
    carry = block_exclusive(e, wsum, carry);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t q = base + 4u * threadIdx.x + (uint32_t)i;
      if (q < total) counts[q] = e[i];
    }
  }
}

// One pass over a tile: item -> counts[digit * tiles + tile] (the items of
// smaller digits, and of this digit in earlier tiles) + its rank among the
// tile's items of the same digit.  The last tile's positions past n carry
// the all-ones key (largest digit, last in position order), so they rank
// after every real item and are not written.
__global__ __launch_bounds__(kSortThreads) void sort_scatter_kernel(
    const uint32_t* __restrict__ keys_in, const uint32_t* __restrict__ vals_in,
    uint32_t from_tokens, uint32_t n, uint32_t vocab, int shift,
    const uint32_t* __restrict__ counts, uint32_t tiles, uint32_t* __restrict__ keys_out,
    uint32_t* __restrict__ vals_out) {
  __shared__ uint32_t s_hist[kHistWords], s_wsum[kSortWaves];
  const uint32_t lane = __lane_id(), wave = threadIdx.x / kWave, tile = blockIdx.x;
  uint32_t k[kSortItems], v[kSortItems], dg[kSortItems], r[kSortItems];
#pragma unroll
  for (int j = 0; j < kSortItems; ++j) {
    const uint32_t p = tile * kSortTile + tile_pos(wave, j, lane);
    k[j] = kPadKey;
    v[j] = 0u;
    if (p < n) {
      k[j] = ld_g<uint32_t>(keys_in + p);
      if (from_tokens) {
        k[j] = clamp_token(k[j], vocab);
        v[j] = p;
      } else {
        v[j] = ld_g<uint32_t>(vals_in + p);
      }
    }
    dg[j] = (k[j] >> shift) & (kRadix - 1u);
  }
  tile_pass(dg, r, s_hist, s_wsum);
#pragma unroll
  for (int j = 0; j < kSortItems; ++j) {
    const uint32_t p = tile * kSortTile + tile_pos(wave, j, lane);
    if (p < n) {
      const uint32_t d = dg[j];
      const uint32_t dst = counts[d * tiles + tile] +
                           (s_hist[hist_at(d, wave)] - s_hist[hist_at(d, 0)]) + r[j];
      keys_out[dst] = k[j];
      vals_out[dst] = v[j];
    }
  }
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
constexpr uint64_t kMaxPlanSegs = ((1ull << 32) - 1) / (kBlocksPerSeg * kWave);  // 4,194,303
// gather_kernel and run_kernel launch one 256-lane block per token along x,
// and a launch's work-items along one dimension must stay below 2^32.
constexpr uint32_t kMaxTokens = (uint32_t)((1ull << 32) / kThreads) - 1u;  // 16,777,215
static_assert(kTileCols == kThreads, "both per-token launches use 256-lane blocks");

using ark::overlaps;

using ark::StreamBuf;

// Byte offsets of the scatter's workspace arrays, each 256-byte aligned:
// the sorted keys and positions, for more than one tile a second pair that
// the sort passes alternate with and the (digit, tile) counts, then the
// copy of dx0 in sorted order.
struct ScatterLayout {
  uint32_t tiles = 0;  // kSortTile-item tiles; 1 = the one-block sort
  size_t skeys = 0, svals = 0, keys = 0, vals = 0, counts = 0, xs = 0, bytes = 0;
};

ScatterLayout scatter_layout(uint32_t n, uint32_t d) {
  ScatterLayout L;
  L.tiles = (n + kSortTile - 1) / kSortTile;
  const size_t arr = ark::align_up((size_t)n * 4, 256);
  size_t off = 0;
  L.skeys = off, off += arr;
  L.svals = off, off += arr;
  if (L.tiles > 1) {
    L.keys = off, off += arr;
    L.vals = off, off += arr;
    L.counts = off, off += ark::align_up((size_t)kRadix * L.tiles * 4, 256);
  }
  L.xs = off, off += ark::align_up((size_t)n * d * 4, 256);
  L.bytes = off;
  return L;
}

// Argument checks shared by the scatter's entry points; *skip is set when
// there is nothing to do.
int scatter_check(const float* embed_grad, uint32_t vocab, uint32_t d, const uint32_t* tokens,
                  const float* dx0, uint32_t batch_seq, bool* skip) {
  *skip = batch_seq == 0 || d == 0;
  if (*skip) return ARK_OPT_OK;
  if (vocab == 0) return fail(ARK_OPT_EINVAL, "vocab is 0");
  if (batch_seq > kMaxTokens)
    return fail(ARK_OPT_EINVAL, "batch_seq = %u too large (at most %u tokens per call)", batch_seq,
                kMaxTokens);
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
  return ARK_OPT_OK;
}

// A scatter not made through the final call: any optimizer handle whose
// norm units cover embed_grad loses them (its next step reads the gradients).
void invalidate_embed_units(const float* embed_grad, uint32_t vocab, uint32_t d) {
  const void* p = embed_grad;
  const uint64_t b = (uint64_t)vocab * d * 4;
  ark::opt_units_invalidate(&p, &b, 1);
}

// Queues the scatter on s with its workspace at ws (L.bytes bytes, 256-byte
// aligned): the sort, the row copy and the run adds.
int scatter_launch(float* embed_grad, uint32_t vocab, uint32_t d, const uint32_t* tokens,
                   const float* dx0, uint32_t n, char* ws, const ScatterLayout& L,
                   hipStream_t s) {
  int end_bit = 1;
  while (end_bit < 32 && ((vocab - 1u) >> end_bit) != 0u) ++end_bit;
  uint32_t* skeys = (uint32_t*)(ws + L.skeys);
  uint32_t* svals = (uint32_t*)(ws + L.svals);
  float* xs = (float*)(ws + L.xs);
  if (L.tiles == 1) {
    hipLaunchKernelGGL(block_sort_kernel, dim3(1), dim3(kSortThreads), 0, s, tokens, n, vocab,
                       end_bit, skeys, svals);
    ARK_HIP(hipGetLastError());
  } else {
    uint32_t* keys = (uint32_t*)(ws + L.keys);
    uint32_t* vals = (uint32_t*)(ws + L.vals);
    uint32_t* counts = (uint32_t*)(ws + L.counts);
    const int passes = (end_bit + kRadixBits - 1) / kRadixBits;
    const uint32_t* in_k = tokens;
    const uint32_t* in_v = nullptr;
    for (int pass = 0; pass < passes; ++pass) {
      const int shift = pass * kRadixBits;
      const uint32_t from_tokens = pass == 0 ? 1u : 0u;
      // the last pass writes skeys/svals; the ones before alternate back
      const bool to_sorted = ((passes - 1 - pass) & 1) == 0;
      uint32_t* out_k = to_sorted ? skeys : keys;
      uint32_t* out_v = to_sorted ? svals : vals;
      hipLaunchKernelGGL(sort_hist_kernel, dim3(L.tiles), dim3(kSortThreads), 0, s, in_k,
                         from_tokens, n, vocab, shift, counts, L.tiles);
      ARK_HIP(hipGetLastError());
      hipLaunchKernelGGL(sort_scan_kernel, dim3(1), dim3(kSortThreads), 0, s, counts,
                         kRadix * L.tiles);
      ARK_HIP(hipGetLastError());
      hipLaunchKernelGGL(sort_scatter_kernel, dim3(L.tiles), dim3(kSortThreads), 0, s, in_k, in_v,
                         from_tokens, n, vocab, shift, (const uint32_t*)counts, L.tiles, out_k,
                         out_v);
      ARK_HIP(hipGetLastError());
      in_k = out_k;
      in_v = out_v;
    }
  }
  const uint32_t gvec = ((d % 4u) == 0 && (((uintptr_t)dx0 & 15u) == 0)) ? 1u : 0u;
  hipLaunchKernelGGL(gather_kernel, dim3(n), dim3(kThreads), 0, s, dx0, svals, d, gvec, xs);
  ARK_HIP(hipGetLastError());
  const uint32_t vec = ((d % 4u) == 0 && (((uintptr_t)embed_grad & 15u) == 0)) ? 1u : 0u;
  const dim3 grid(n, (d + kTileCols - 1) / kTileCols);
  hipLaunchKernelGGL(run_kernel, grid, dim3(kTileCols), 0, s, embed_grad, d, xs, skeys, n, vec);
  ARK_HIP(hipGetLastError());
  return ARK_OPT_OK;
}

}  // namespace

// ---- the scatter's workspace without allocation --------------------------
// One file-scope device array.  It is part of this library's code object, so
// every GPU the library is used on holds a copy from the code object's load
// there (the library's first kernel launch or symbol lookup on that GPU) to
// the end of the process.  Host code never passes `scratch` itself to a
// kernel (on the host the name is only a stand-in for the symbol): it looks
// the array's device address up once per device with hipGetSymbolAddress,
// with that device current, and uses that address.
static __device__ __align__(256) uint8_t scratch[ARK_GRAD_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;

// Per device: the address of its copy of scratch, and an event recorded on
// the stream of each eager no-allocation call after its last launch, which
// the next eager call waits for, so calls from different streams or threads
// take the array in turn.
struct ScratchSlot {
  void* ptr = nullptr;
  hipEvent_t done = nullptr;
  bool recorded = false;
};
std::mutex g_scratch_mu;  // guards g_scratch and orders the calls' enqueues
ScratchSlot g_scratch[kMaxDevices];

// Sets device dev's slot up; the caller holds g_scratch_mu.
int scratch_setup_locked(int dev) {
  ScratchSlot& S = g_scratch[dev];
  if (S.ptr && S.done) return ARK_OPT_OK;
  ark::DeviceGuard g(dev);
  if (!g.ok) return fail(ARK_OPT_EHIP, "cannot select device %d", dev);
  if (!S.ptr) {
    void* p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      (void)hipGetLastError();
      return ark::hip_fail(e, "hipGetSymbolAddress(scratch)");
    }
    S.ptr = p;
  }
  if (!S.done) {
    hipError_t e = hipEventCreateWithFlags(&S.done, hipEventDisableTiming);
    if (e != hipSuccess) {
      S.done = nullptr;
      (void)hipGetLastError();
      return ark::hip_fail(e, "hipEventCreateWithFlags for the static scratch");
    }
  }
  return ARK_OPT_OK;
}

}  // namespace

namespace ark {

int grad_scratch_prepare(int dev) {
  if (dev < 0 || dev >= kMaxDevices)
    return fail(ARK_OPT_EINVAL, "device %d out of range for the static scratch", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  return scratch_setup_locked(dev);
}

}  // namespace ark

struct ark_grad_plan {
  int device = 0;
  hipStream_t stream = nullptr;
  uint32_t nseg = 0;
  GradSeg* d_segs = nullptr;
  uint32_t lds = 0;  // dynamic LDS per grad_batch block (residency cap)
  std::vector<const float*> span_dst;  // the spans as given, for matching an
  std::vector<uint64_t> span_n;        // optimizer table
  std::vector<uint64_t> span_bytes;    // 4 * span_n
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
  {
    const void* d = dst;
    const uint64_t b = n * 4;
    ark::opt_units_invalidate(&d, &b, 1);
  }
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
  int rc;
  // One launch runs every span at once, so a dst shared with another span's
  // dst or src would race: every dst must be disjoint from every other span
  // (srcs may overlap each other).  Checked before any device query.
  {
    std::vector<ark::Span> written, readonly;
    uint64_t nseg = 0;
    for (int32_t i = 0; i < n_spans; ++i) {
      const ark_grad_span& s = spans[i];
      if (s.n == 0) continue;
      if (((uintptr_t)s.dst & 3u) || ((uintptr_t)s.src & 3u))
        return fail(ARK_OPT_EINVAL, "span %d: dst or src not 4-byte aligned", i);
      if (s.n > (1ull << 48)) return fail(ARK_OPT_EINVAL, "span %d: n too large", i);
      // one launch covers every segment with kBlocksPerSeg waves, and a
      // launch's work-items stay below 2^32
      nseg += (s.n + kSeg - 1) / kSeg;
      if (nseg > kMaxPlanSegs)
        return fail(ARK_OPT_EINVAL, "too many elements (more than %llu segments of %u)",
                    (unsigned long long)kMaxPlanSegs, kSeg);
      if (overlaps(s.dst, s.n * 4, s.src, s.n * 4))
        return fail(ARK_OPT_EINVAL, "span %d: dst and src overlap", i);
      written.push_back({(uintptr_t)s.dst, (uintptr_t)s.dst + s.n * 4, "dst", i});
      readonly.push_back({(uintptr_t)s.src, (uintptr_t)s.src + s.n * 4, "src", i});
    }
    if ((rc = ark::check_disjoint(std::move(written), std::move(readonly), "span", "the plan")))
      return rc;
  }
  ark::BufferChecker checker;
  for (int32_t i = 0; i < n_spans; ++i) {
    const ark_grad_span& s = spans[i];
    if (s.n == 0) continue;
    if ((rc = checker.check(s.dst, s.n * 4, "dst", i))) return rc;
    if ((rc = checker.check(s.src, s.n * 4, "src", i))) return rc;
    const uint32_t vec = ((((uintptr_t)s.dst | (uintptr_t)s.src) & 15u) == 0) ? 1u : 0u;
    for (uint64_t off = 0; off < s.n; off += kSeg) {
      GradSeg d;
      d.dst = s.dst + off;
      d.src = s.src + off;
      d.n = (uint32_t)(s.n - off < kSeg ? s.n - off : kSeg);
      d.vec = vec;
      segs.push_back(d);
    }
  }
  int dev = 0;
  if ((rc = ark::current_device_for(stream, &dev))) return rc;
  ark_grad_plan* p = new ark_grad_plan();
  p->device = dev;
  p->stream = (hipStream_t)stream;
  p->nseg = (uint32_t)segs.size();
  for (int32_t i = 0; i < n_spans; ++i) {
    p->span_dst.push_back(spans[i].dst);
    p->span_n.push_back(spans[i].n);
    p->span_bytes.push_back(spans[i].n * 4u);
  }
  hipError_t e = hipSuccess;
  {
    // the no-allocation scatter's set-up on this device (best effort, as in
    // ark_opt_create)
    (void)ark::grad_scratch_prepare(p->device);
    // ARK_GRAD_BLOCKS_PER_CU=8..32 overrides the cap, 0 lifts it (a tuning
    // knob: results do not depend on it)
    int per_cu = kPlanBlocksPerCu;
    if (const char* env = getenv("ARK_GRAD_BLOCKS_PER_CU")) {
      const int v = atoi(env);
      if (v == 0 || (v >= 8 && v <= 32)) per_cu = v;
    }
    p->lds = ark::resident_lds_bytes((const void*)grad_batch, kWave, per_cu);
  }
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
  ark::opt_units_invalidate(reinterpret_cast<const void* const*>(p->span_dst.data()),
                            p->span_bytes.data(), p->span_dst.size());
  ark::DeviceGuard g(p->device);
  if (!g.ok) return fail(ARK_OPT_EHIP, "cannot select device %d", p->device);
  hipLaunchKernelGGL(grad_batch, dim3(p->nseg * kBlocksPerSeg), dim3(kWave), p->lds, p->stream,
                     p->d_segs);
  ARK_HIP(hipGetLastError());
  return ARK_OPT_OK;
}

int ark_grad_plan_run_final(ark_grad_plan* p, ark_opt_handle* opt) {
  if (!p) return fail(ARK_OPT_EINVAL, "plan is NULL");
  ark::OptUnits U;
  int rc = ark::opt_units_for_spans(opt, p->span_dst.data(), p->span_n.data(),
                                    p->span_n.size(), &U);
  if (rc) return rc;
  if (U.stream != p->stream || U.device != p->device)
    return fail(ARK_OPT_EINVAL, "the plan and the optimizer handle must share a stream");
  if (U.nseg != p->nseg)
    return fail(ARK_OPT_EINVAL, "plan and optimizer table differ in segments (%u, %u)", p->nseg,
                U.nseg);
  if (p->nseg) {
    ark::DeviceGuard g(p->device);
    if (!g.ok) return fail(ARK_OPT_EHIP, "cannot select device %d", p->device);
    hipLaunchKernelGGL(grad_batch_units, dim3(p->nseg * kBlocksPerSeg), dim3(kWave), 0,
                       p->stream, p->d_segs, U.segs, U.state, U.units);
    ARK_HIP(hipGetLastError());
  }
  ark::opt_units_set_fresh(opt, true);
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
  bool skip = false;
  int rc = scatter_check(embed_grad, vocab, d, tokens, dx0, batch_seq, &skip);
  if (rc || skip) return rc;
  invalidate_embed_units(embed_grad, vocab, d);
  hipStream_t s = (hipStream_t)stream;
  const ScatterLayout L = scatter_layout(batch_seq, d);
  StreamBuf ws;
  hipError_t e = ws.alloc(L.bytes, s);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return fail(ARK_OPT_ENOMEM, "hipMallocAsync(%zu) for the scatter failed", L.bytes);
  }
  return scatter_launch(embed_grad, vocab, d, tokens, dx0, batch_seq, (char*)ws.p, L, s);
}

int ark_grad_embed_scatter_final(float* embed_grad, uint32_t vocab, uint32_t d,
                                 const uint32_t* tokens, const float* dx0, uint32_t batch_seq,
                                 ark_opt_handle* opt) {
  ark::OptUnits U;
  uint64_t unit0 = 0;
  uint32_t seg_flags = 0;
  // rows are whole units only when d is a multiple of 256; otherwise the
  // scatter is done and the step reads the gradients (no units needed here)
  const bool rows_are_units = d % (uint32_t)kTileCols == 0;
  int rc = ark::opt_units_for_tensor(opt, embed_grad, (uint64_t)vocab * d, rows_are_units, &U,
                                     &unit0, &seg_flags);
  if (rc) return rc;
  bool skip = false;
  if ((rc = scatter_check(embed_grad, vocab, d, tokens, dx0, batch_seq, &skip))) return rc;
  if (skip) return ARK_OPT_OK;  // nothing changes; the units stay valid
  ark::DeviceGuard g(U.device);
  if (!g.ok) return fail(ARK_OPT_EHIP, "cannot select device %d", U.device);
  const ScatterLayout L = scatter_layout(batch_seq, d);
  StreamBuf ws;
  hipError_t e = ws.alloc(L.bytes, U.stream);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return fail(ARK_OPT_ENOMEM, "hipMallocAsync(%zu) for the scatter failed", L.bytes);
  }
  // the units of the rows it changes are stale from here until rewritten
  ark::opt_units_set_fresh(opt, false);
  rc = scatter_launch(embed_grad, vocab, d, tokens, dx0, batch_seq, (char*)ws.p, L, U.stream);
  if (rc) return rc;
  if (!rows_are_units) return ARK_OPT_OK;  // units straddle rows: the step re-reads
  const uint32_t vec = ((d % 4u) == 0 && (((uintptr_t)embed_grad & 15u) == 0)) ? 1u : 0u;
  hipLaunchKernelGGL(units_rows_kernel, dim3(batch_seq, d / kTileCols), dim3(kWave), 0, U.stream,
                     embed_grad, d, (const uint32_t*)((char*)ws.p + L.skeys), vec, U.state,
                     seg_flags, U.units + unit0);
  ARK_HIP(hipGetLastError());
  ark::opt_units_set_fresh(opt, true);
  return ARK_OPT_OK;
}

int ark_grad_embed_scatter_noalloc(float* embed_grad, uint32_t vocab, uint32_t d,
                                   const uint32_t* tokens, const float* dx0, uint32_t batch_seq,
                                   void* stream) {
  bool skip = false;
  int rc = scatter_check(embed_grad, vocab, d, tokens, dx0, batch_seq, &skip);
  if (rc || skip) return rc;
  const ScatterLayout L = scatter_layout(batch_seq, d);
  if (L.bytes > (size_t)ARK_GRAD_SCRATCH_BYTES)
    return fail(ARK_OPT_EINVAL,
                "scatter of %u tokens x %u columns needs %zu bytes of workspace; the static "
                "scratch holds %llu (ark_grad_embed_scatter allocates instead)",
                batch_seq, d, L.bytes, (unsigned long long)ARK_GRAD_SCRATCH_BYTES);
  hipStream_t s = (hipStream_t)stream;
  int dev = -1;
  hipError_t e = s ? hipStreamGetDevice(s, &dev) : hipGetDevice(&dev);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return ark::hip_fail(e, "device of the stream");
  }
  if (dev < 0 || dev >= kMaxDevices)
    return fail(ARK_OPT_EINVAL, "device %d out of range for the static scratch", dev);
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  e = hipStreamIsCapturing(s, &cap);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return ark::hip_fail(e, "hipStreamIsCapturing");
  }
  const bool captured = cap != hipStreamCaptureStatusNone;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  ScratchSlot& S = g_scratch[dev];
  if (!S.ptr || !S.done) {
    // the one-time lookup may load the code object; it is no stream work
    // and cannot be captured
    if (captured)
      return fail(ARK_OPT_EINVAL,
                  "the static scratch of device %d is not set up yet and the stream is "
                  "capturing: make one ark_grad_embed_scatter_noalloc call, or create an "
                  "optimizer handle or a gradient plan, on that device before capturing",
                  dev);
    if ((rc = scratch_setup_locked(dev))) return rc;
  }
  invalidate_embed_units(embed_grad, vocab, d);
  if (captured)  // a graph node: its replays are ordered by the caller
    return scatter_launch(embed_grad, vocab, d, tokens, dx0, batch_seq, (char*)S.ptr, L, s);
  if (S.recorded) ARK_HIP(hipStreamWaitEvent(s, S.done, 0));
  rc = scatter_launch(embed_grad, vocab, d, tokens, dx0, batch_seq, (char*)S.ptr, L, s);
  // recorded even after a failed launch, which may have queued part of its work
  e = hipEventRecord(S.done, s);
  if (e == hipSuccess) S.recorded = true;
  if (rc) return rc;
  if (e != hipSuccess) return ark::hip_fail(e, "hipEventRecord for the static scratch");
  return ARK_OPT_OK;
}

}  // extern "C"
