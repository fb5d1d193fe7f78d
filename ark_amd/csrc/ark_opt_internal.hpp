// ark_opt_internal.hpp -- what the gradient hand-off (ark_grad.hip) needs from
// an optimizer handle (ark_opt.hip) to hand the norm's first level to the
// step: the handle's buffer of "units".
//
// A unit is 256 consecutive elements of a segment (the AdamW row): unit r of
// segment s covers elements [r * 256, r * 256 + 256) of the segment, and its
// value is the pairwise f64 tree of the squared unscaled gradients over those
// elements (zero past the segment's end), or NaN when one of them is inf or
// NaN.  The canonical tree of the global sum is a perfect binary tree over
// the segments' elements in order, so a unit is one of its aligned subtrees
// and a norm block's partial is the pairwise tree of its units: a step whose
// units were written by the kernels that produced the final gradients needs
// no second read of them, and its sum has the same bits.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "ark_opt.h"
#include "ark_opt_kernels.hpp"

namespace ark {

constexpr int kUnit = kRow;                  // elements per unit
constexpr int kUnitsPerSeg = kSeg / kUnit;   // 16

// Device side of a handle's units: units[s * kUnitsPerSeg + r].
struct OptUnits {
  double* units = nullptr;
  const SegDesc* segs = nullptr;        // the handle's segment table
  const ark_opt_state* state = nullptr; // loss scale for the unscale
  hipStream_t stream = nullptr;
  int device = 0;
  uint32_t nseg = 0;
};

// h must take fp32 gradients and its tensors with n > 0 must be, in table
// order, exactly the count spans (dst[i], n[i]) with n[i] > 0; then *out
// describes its units.  ARK_OPT_EINVAL with a message otherwise.
int opt_units_for_spans(ark_opt_handle* h, const float* const* dst, const uint64_t* n,
                        size_t count, OptUnits* out);

// The tensor of h whose gradient is g with n elements: *unit0 = the index of
// its first unit, *seg_flags = its segments' flags.  With require_fresh it
// fails unless h's units are fresh (written since its last step).
int opt_units_for_tensor(ark_opt_handle* h, const void* g, uint64_t n, bool require_fresh,
                         OptUnits* out, uint64_t* unit0, uint32_t* seg_flags);

// Marks h's units as written for its next step (fresh) or not.
void opt_units_set_fresh(ark_opt_handle* h, bool fresh);

// (opt_units_invalidate, the other writers' side, is in ark_common.hpp.)

// units -> one partial per norm block of spb segments, exactly what
// sumsq_kernel would write for the same gradients (launch_sumsq's part_sum).
hipError_t launch_units_reduce(int spb, uint32_t nblocks, const double* units,
                               const SegDesc* segs, uint32_t nseg, double* part_sum,
                               hipStream_t stream);

}  // namespace ark
