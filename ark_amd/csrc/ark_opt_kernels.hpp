// ark_opt_kernels.hpp -- gfx950 kernels of the optimizer step.
//
// Three stream-ordered kernels per step, no host round trip:
//   1. sumsq_kernel   : reads every gradient once (2 B/param for fp16), forms
//                       the f64 sum of squares of the unscaled gradients along
//                       the canonical pairwise tree and the inf/NaN flag, one
//                       partial per block of SPB segments.
//   2. finalize_kernel: one block; finishes the tree, runs the AMP skip /
//                       growth state machine, the clip decision and the bias
//                       corrections, and writes the step scalars.
//   3. adamw_kernel   : the fused streaming update (22 B/param): unscale, clip
//                       coefficient, AdamW with decoupled weight decay, fp16
//                       weight requantisation; exits at once on a skipped step.
//
// Every tensor is cut into ARK_OPT_NORM_SEGMENT-element segments, listed in
// table order, each with a 48-byte descriptor holding its four pointers
// already offset to the segment start, so a block finds its data with one
// scalar load and no dependent lookups.
//
// sumsq_kernel: a 256-lane block covers a segment as two halves of 256 x 8
// elements, lane l owning elements [h*2048 + 8l, h*2048 + 8l + 8) of half h
// (one 16-byte load per half).  That layout is what the canonical tree needs:
// lane groups of 8 in index order.
// adamw_kernel: one wave per 256-element row, lane l owning elements
// [4l, 4l + 4): every load and store instruction of every array covers one
// contiguous span (512 B of fp16, 1 KiB of fp32).  One-wave blocks over a
// grid of ~a million rows measured fastest on MI355X for this mix of four
// read streams and three write streams.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ark_opt.h"

namespace ark {

constexpr int kSeg = ARK_OPT_NORM_SEGMENT;  // elements per segment
constexpr int kBlock = 256;                 // lanes per sumsq block (4 waves)
constexpr int kVec = 8;                     // sumsq elements per lane group
constexpr int kHalfSeg = kBlock * kVec;     // 2048
static_assert(kSeg == 2 * kHalfSeg, "segment = two halves of 256 x 8");
constexpr int kRow = 256;                   // adamw elements per wave
constexpr int kRowsPerSeg = kSeg / kRow;    // 16
constexpr int kFinThreads = 1024;           // finalize block

// Segment descriptor flags.
constexpr uint32_t kSegNoUnscale = 1u;  // ARK_OPT_TENSOR_NO_UNSCALE
constexpr uint32_t kSegVec = 2u;        // w, g, m, v all 16-byte aligned

struct SegDesc {
  uint16_t* w;      // pointers to the segment's first element
  const void* g;
  float* m;
  float* v;
  uint32_t n;       // valid elements in this segment, 1..kSeg
  float wd;         // weight decay of the tensor
  uint32_t flags;   // kSeg*
  uint32_t tensor;  // index in the caller's table
};
static_assert(sizeof(SegDesc) == 48, "48-byte descriptor");

// Scalars of one step, written by finalize_kernel, read by adamw_kernel.
struct StepScalars {
  uint32_t applied;
  uint32_t clipped;
  float inv;     // 1 / loss_scale
  float coef;    // clip coefficient (1 when not clipped)
  float lr;
  float lr_eff;  // sqrtf(bc2) / bc1 * lr
  float c1;      // 1 - beta1
  float c2;      // 1 - beta2
};

// beta^t by binary exponentiation, then lr_eff = (sqrt(bc2) / bc1) * lr, one
// IEEE binary32 operation per step as in opti.s:223-258.  Compiled for host
// and device; both round every operation to nearest even.
__host__ __device__ inline float pow_binary(float beta, uint32_t t) {
  float res = 1.0f;
  float base = beta;
  while (t != 0u) {
    if (t & 1u) res = res * base;
    base = base * base;
    t >>= 1;
  }
  return res;
}

__host__ __device__ inline float lr_eff_of(float lr, float beta1, float beta2,
                                           uint32_t t) {
  if (t == 0u) t = 1u;  // opti.s:211-212
  const float bc1 = 1.0f - pow_binary(beta1, t);
  const float bc2 = 1.0f - pow_binary(beta2, t);
  float r = sqrtf(bc2);
  r = r / bc1;
  return r * lr;
}

// Segments per norm block: 2 for fp16 gradients, 8 for fp32 (4 or 8 past
// kMaxParts partials); halved while fewer than 512 blocks would cover the
// table.
int sumsq_spb(uint64_t nseg, uint32_t grad_dtype);
// Partial-buffer capacity: past kFinTarget the partials are folded by
// kFoldGroup, so the finalize reads at most kMaxParts / kFoldGroup = 8192.
constexpr uint32_t kMaxParts = 512u * kFinThreads;
// Above kFinTarget partials, fold_kernel first reduces aligned groups of
// kFoldGroup (one wave each) so the finalize reads at most kFinTarget values.
constexpr uint32_t kFinTarget = 8u * kFinThreads;
constexpr uint32_t kFoldGroup = 64u;

// in: padded_parts partials (a power of two, multiple of kFoldGroup, zero
// past the real ones); out: padded_parts / kFoldGroup group sums.
hipError_t launch_fold(uint32_t padded_parts, const double* in, double* out,
                       hipStream_t stream);
// adamw grid: one wave per row, 16 rows per segment; the grid must stay
// below 2^32 work-items.
constexpr uint64_t kMaxSegments = (1ull << 32) / (64ull * kRowsPerSeg) - 1;
static_assert((kMaxSegments + 7) / 8 <= kMaxParts, "8 segments per norm block cover every table");
static_assert(kMaxParts / kFoldGroup <= kFinTarget, "one fold leaves the finalize kFinTarget");

// ---------------------------------------------------------------------------
// Launch helpers (ark_opt_kernels.hip); each returns hipSuccess or the error.
// ---------------------------------------------------------------------------

// part_sum: one partial per block (NaN when the block saw a non-finite
// gradient).  A batch of segments whose segments all exist, hold kSeg
// elements and carry kSegVec takes 16-byte loads.  Blocks b >= nt_from read
// with non-temporal loads (see sumsq_nt_from).  lds_bytes of dynamic LDS per
// block (unused by the kernel) bound how many blocks a CU holds at once
// (sumsq_lds_for).
hipError_t launch_sumsq(uint32_t grad_dtype, int spb, uint32_t nblocks,
                        const SegDesc* segs, uint32_t nseg, const ark_opt_state* state,
                        double* part_sum, uint32_t nt_from, uint32_t lds_bytes,
                        hipStream_t stream);

// Resident norm blocks per CU for fp16 gradients.  Their fast path (squares
// straight from the fp16 bits under a power-of-two loss scale) has so little
// arithmetic per byte that 8 blocks per CU, the wave-slot limit, issue loads
// faster than HBM returns them: on MI355X the pass over EKO-237M's 474 MB
// takes 79.0-79.5 us at 8 blocks per CU, 77.2-77.5 at 7 and 78.9-79.1 at 6,
// and over the 1.3B set's 2.56 GB 372.6 us at 7 against 379.1 at 8.  0 = no
// cap (fp32 gradients).
constexpr int kSumsqBlocksPerCuF16 = 7;
// The dynamic LDS that holds the norm kernel for (grad_dtype, spb) at
// `blocks` per CU (resident_lds_bytes; 0 = no cap).
uint32_t sumsq_lds_for(uint32_t grad_dtype, int spb, int blocks);
// Resident one-wave AdamW blocks per CU.  32 (every wave slot) over-issue
// the pass's seven streams: on MI355X the EKO-237M pass takes 783.5 us
// unbounded, 776.6 at 26 per CU, 762.5 at 20, 760.4-760.6 at 17 and 16,
// 768 at 15 and 14 and 782 at 13; the 1.3B set's 4465-4480 us unbounded,
// 4351 at 20, 4310-4323 at 17 and 16, 4283-4285 at 15 and 14.
constexpr int kAdamwBlocksPerCu = 16;
// The dynamic LDS that holds the AdamW kernel for grad_dtype at `blocks` per
// CU (resident_lds_bytes; 0 = no cap).
uint32_t adamw_lds_for(uint32_t grad_dtype, int blocks);

// The norm pass leaves the last kNormCachedBytes it reads (its lowest
// blocks, where the AdamW pass starts) in the Infinity Cache and streams the
// rest past it.  Measured on MI355X over 128-320 MiB and all-streaming:
// 256 MiB (the cache's size) is fastest, the step 0.5 % faster at EKO-237M
// and 0.9 % at 1.3B than with every load cache-allocating.
constexpr uint64_t kNormCachedBytes = 256ull << 20;
inline uint32_t sumsq_nt_from(int spb, uint64_t grad_bytes) {
  const uint64_t per_block = (uint64_t)spb * kSeg * grad_bytes;
  const uint64_t b = kNormCachedBytes / per_block;
  return b > 0xFFFFFFFFull ? 0xFFFFFFFFu : (uint32_t)b;
}

// Leaves per finalize thread for nparts partials (a power of two <= 64); the
// partial buffer must hold kFinThreads * leaves doubles, zero past nparts.
uint32_t finalize_leaves(uint32_t nparts);

// lr_ptr: NULL, or a device scalar the kernel reads this step's lr from.
hipError_t launch_finalize(uint32_t leaves, const double* part_sum,
                           const ark_opt_hparams& hp, float lr, const float* lr_ptr,
                           ark_opt_state* state, StepScalars* scal,
                           ark_opt_step_info* info, hipStream_t stream);

// lds_bytes: dynamic LDS per block, the residency cap (adamw_lds_for).
hipError_t launch_adamw(uint32_t grad_dtype, const SegDesc* segs,
                        uint32_t nseg, const StepScalars* scal, float beta1,
                        float beta2, float eps, uint32_t lds_bytes, hipStream_t stream);

// One tensor given by value (fp32 gradients used as given, no unscale or
// clip) with host-computed scalars: the drop-in of one
// ark_asm_adam_step_f16 call.  n may exceed one segment.
hipError_t launch_adamw_single(uint16_t* w, const float* g, float* m, float* v,
                               uint64_t n, float wd, bool vec,
                               const StepScalars& sc, float beta1, float beta2,
                               float eps, hipStream_t stream);

// The same for an fp32-weight tensor: the drop-in of one ark_asm_adam_step
// call (opti.s:20-177).
hipError_t launch_adamw_single_w32(float* w, const float* g, float* m, float* v, uint64_t n,
                                   float wd, bool vec, const StepScalars& sc, float beta1,
                                   float beta2, float eps, hipStream_t stream);

// The single-tensor clip (ark_asm_grad_clip, opti.s:369-432): the
// canonical tree's sum of squares of one fp32 array (one partial per block of
// two segments, folded past kFinTarget partials), the norm and the clip
// decision on the device, then the in-place scaling when it clips.
struct ClipScalars {
  double sumsq;
  float norm;      // the pre-clip norm the call reports
  float coef;      // threshold / norm (1 when not clipped)
  uint32_t clipped;
  uint32_t pad;
};
static_assert(sizeof(ClipScalars) == 24, "24-byte clip result");
// Elements one call takes: the partials stay within what one fold and a
// 1024 x 8-leaf finalize reduce (kFinTarget * kFoldGroup = 2^19 blocks of
// 2 segments).
constexpr uint64_t kClipMaxElements = (uint64_t)kFinTarget * kFoldGroup * 2u * kSeg;
inline uint32_t clip_parts(uint64_t n) { return (uint32_t)((n + 2u * kSeg - 1) / (2u * kSeg)); }
// parts: clip_parts(n) doubles; folded: ceil(clip_parts(n) / kFoldGroup)
// doubles (used past kFinTarget partials); out: the decision.  n >= 1.
hipError_t launch_grad_clip(float* g, uint64_t n, float threshold, double* parts,
                            double* folded, ClipScalars* out, hipStream_t stream);

hipError_t launch_record_overflow(const ark_opt_hparams& hp,
                                  ark_opt_state* state,
                                  ark_opt_step_info* info, hipStream_t stream);

}  // namespace ark
