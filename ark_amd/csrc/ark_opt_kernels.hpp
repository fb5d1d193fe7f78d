// ark_opt_kernels.hpp -- gfx950 kernels of the optimizer step.
//
// Three stream-ordered kernels per step, no host round trip:
//   1. sumsq_kernel   : reads every gradient once (2 B/param for fp16), forms
//                       the f64 sum of squares of the unscaled gradients along
//                       the canonical pairwise tree and the inf/NaN flag, one
//                       partial per block.
//   2. finalize_kernel: one block; finishes the tree, runs the AMP skip /
//                       growth state machine, the clip decision and the bias
//                       corrections, and writes the step scalars.
//   3. adamw_kernel   : the fused streaming update (22 B/param): unscale, clip
//                       coefficient, AdamW with decoupled weight decay, fp16
//                       weight requantisation; exits at once on a skipped step.
//
// Tensors are cut into ARK_OPT_NORM_SEGMENT-element segments listed in table
// order; a block of 256 lanes covers a segment as two halves of 256 x 8
// elements, lane l owning elements [h*2048 + 8l, h*2048 + 8l + 8) of half h.
// Every access is a 16-byte load or store when the tensor's pointers are
// 16-byte aligned and the group of 8 lies inside the tensor.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ark_opt.h"

namespace ark {

constexpr int kSeg = ARK_OPT_NORM_SEGMENT;  // elements per segment
constexpr int kBlock = 256;                 // lanes per block (4 waves)
constexpr int kVec = 8;                     // elements per lane group
constexpr int kHalfSeg = kBlock * kVec;     // 2048
static_assert(kSeg == 2 * kHalfSeg, "segment = two halves of 256 x 8");
constexpr int kFinThreads = 1024;           // finalize block

// Device copy of one table row.
struct TensorDev {
  uint16_t* w;
  const void* g;
  float* m;
  float* v;
  uint64_t n;
  float wd;
  uint32_t flags;
  uint32_t seg0;  // global index of the tensor's first segment
  uint32_t vec;   // w, g, m, v all 16-byte aligned
};

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

// ---------------------------------------------------------------------------
// Kernel entry points (defined in ark_opt_kernels.hip).
// ---------------------------------------------------------------------------

// Launch helpers return hipSuccess or the launch error.
hipError_t launch_sumsq(uint32_t grad_dtype, int spb, uint32_t nblocks,
                        const TensorDev* tab, const uint32_t* seg_tensor,
                        uint32_t nseg, const ark_opt_state* state,
                        double* part_sum, uint32_t* part_flag,
                        hipStream_t stream);

hipError_t launch_finalize(uint32_t nparts, const double* part_sum,
                           const uint32_t* part_flag,
                           const ark_opt_hparams& hp, float lr,
                           ark_opt_state* state, StepScalars* scal,
                           ark_opt_step_info* info, hipStream_t stream);

// Blocks of adamw_kernel for nseg segments.
uint32_t adamw_blocks(uint32_t nseg);

hipError_t launch_adamw(uint32_t grad_dtype, uint32_t nblocks,
                        const TensorDev* tab, const uint32_t* seg_tensor,
                        uint32_t nseg, const StepScalars* scal, float beta1,
                        float beta2, float eps, hipStream_t stream);

// One tensor given by value with host-computed scalars (fp32 gradients, no
// unscale or clip): the drop-in of one ark_asm_adam_step_f16 call.
hipError_t launch_adamw_single(const TensorDev& t, const StepScalars& sc,
                               float beta1, float beta2, float eps,
                               hipStream_t stream);

hipError_t launch_record_overflow(const ark_opt_hparams& hp,
                                  ark_opt_state* state,
                                  ark_opt_step_info* info, hipStream_t stream);

// Largest number of block partials finalize_kernel accepts.
constexpr uint32_t kMaxParts = 64u * kFinThreads;

}  // namespace ark
