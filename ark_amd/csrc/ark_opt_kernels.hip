// ark_opt_kernels.hip -- gfx950 kernels of the optimizer step (see the
// header for the segment layout and the kernel sequence).
//
// Arithmetic follows the reference kernel ark_asm_adam_step_f16
// (proyecto_ark/ark01/asm/opti.s:192-360) operation for operation; the build
// uses -ffp-contract=off so the only fused operations are the explicit
// __builtin_fmaf calls standing for its fmla instructions (opti.s:287, :293).
// f32 sqrt and division compile to the correctly rounded expansions, fp16
// conversion to v_cvt_f16_f32 under the default round-to-nearest-even mode,
// and fp16/fp32 denormals are preserved.
//
// Cache hints, chosen by measurement on MI355X: the AdamW pass uses
// non-temporal loads and stores for all four arrays (5-10 % faster than plain
// accesses).  The sum-of-squares pass reads the last 256 MiB of gradients it
// visits with plain, cache-allocating loads, which leaves them in the
// Infinity Cache for the AdamW pass that starts on them right after (~5 %
// faster AdamW on EKO-237M, within one step, so real training sees it too),
// and streams the rest with non-temporal loads (13 % faster reads).
#include "ark_common.hpp"
#include "ark_device.hpp"
#include "ark_opt_internal.hpp"
#include "ark_opt_kernels.hpp"

namespace ark {
namespace {

using namespace dev;

// ---- gradient access --------------------------------------------------------

template <typename GT>
struct GradIO;

template <>
struct GradIO<uint16_t> {  // fp16 bits
  typedef u32x4 Raw8;      // 8 elements, one 16-byte load
  typedef u32x2 Raw4;      // 4 elements, one 8-byte load
  template <bool NT = false>
  static __device__ __forceinline__ Raw8 load8(const uint16_t* p) {
    if constexpr (NT) return ld_nt<u32x4>(p);
    return ld_g<u32x4>(p);
  }
  static __device__ __forceinline__ Raw4 load4(const uint16_t* p) { return ld_nt<u32x2>(p); }
  static __device__ __forceinline__ void unpack8(const Raw8& r, float (&f)[8], uint32_t& bad) {
    const uint32_t x[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      bad |= ((x[i] & 0x7C00u) == 0x7C00u) | ((x[i] & 0x7C000000u) == 0x7C000000u);
      f[2 * i] = h2f(x[i] & 0xFFFFu);
      f[2 * i + 1] = h2f(x[i] >> 16);
    }
  }
  static __device__ __forceinline__ void unpack4(const Raw4& r, float (&f)[4]) {
    f[0] = h2f(r.x & 0xFFFFu);
    f[1] = h2f(r.x >> 16);
    f[2] = h2f(r.y & 0xFFFFu);
    f[3] = h2f(r.y >> 16);
  }
  static __device__ __forceinline__ float load1(const uint16_t* p, uint32_t& bad) {
    const uint32_t x = ld_g<uint16_t>(p);
    bad |= (x & 0x7C00u) == 0x7C00u;
    return h2f(x);
  }
};

template <>
struct GradIO<float> {
  struct Raw8 {
    f32x4 a, b;
  };
  typedef f32x4 Raw4;
  template <bool NT = false>
  static __device__ __forceinline__ Raw8 load8(const float* p) {
    Raw8 r;
    if constexpr (NT) {
      r.a = ld_nt<f32x4>(p);
      r.b = ld_nt<f32x4>(p + 4);
    } else {
      r.a = ld_g<f32x4>(p);
      r.b = ld_g<f32x4>(p + 4);
    }
    return r;
  }
  static __device__ __forceinline__ Raw4 load4(const float* p) { return ld_nt<f32x4>(p); }
  static __device__ __forceinline__ void unpack8(const Raw8& r, float (&f)[8], uint32_t& bad) {
    f[0] = r.a.x; f[1] = r.a.y; f[2] = r.a.z; f[3] = r.a.w;
    f[4] = r.b.x; f[5] = r.b.y; f[6] = r.b.z; f[7] = r.b.w;
#pragma unroll
    for (int i = 0; i < 8; ++i)
      bad |= (__float_as_uint(f[i]) & 0x7F800000u) == 0x7F800000u;
  }
  static __device__ __forceinline__ void unpack4(const Raw4& r, float (&f)[4]) {
    f[0] = r.x; f[1] = r.y; f[2] = r.z; f[3] = r.w;
  }
  static __device__ __forceinline__ float load1(const float* p, uint32_t& bad) {
    const float x = ld_g<float>(p);
    bad |= (__float_as_uint(x) & 0x7F800000u) == 0x7F800000u;
    return x;
  }
};

// ---- canonical tree pieces --------------------------------------------------

// Pairwise sum of 8 squares in index order.
__device__ __forceinline__ double tree8(const double (&q)[kVec]) {
  return ((q[0] + q[1]) + (q[2] + q[3])) + ((q[4] + q[5]) + (q[6] + q[7]));
}

// Squares of the unscaled gradients (vDSP_vsmul of ffi.rs:141-146, then an
// exact f64 square) and their tree8.
__device__ __forceinline__ double group_sum(const float (&f)[kVec], float inv_t) {
  double q[kVec];
#pragma unroll
  for (int j = 0; j < kVec; ++j) {
    const float gu = f[j] * inv_t;
    q[j] = (double)gu * (double)gu;
  }
  return tree8(q);
}

// The same leaves from fp16 bits when the unscale is a power of two 2^e
// (|e| <= kPow2MaxExp): f * 2^e is then exact in fp32, so the leaf
// (double)gu * (double)gu is (double)(f * f) * 2^(2e), and every f64 add of
// the tree commutes with that exact scaling (no sum of such leaves leaves
// the normal f64 range).  f * f of an 11-bit significand fits fp32's 24
// bits, so v_fma_mix_f32 (fp16 operands, fp32 result, + 0) forms it exactly
// in one instruction; the caller scales the group sums once.  An inf or NaN
// gradient squares to inf or NaN, and no finite one can make the sum
// overflow, so the block's sum alone tells whether it saw one.  3 VALU
// instructions per element against 7 for group_sum with the per-element
// finite test, which keeps the pass memory bound when the clock drops.
constexpr int kPow2MaxExp = 100;

__device__ __forceinline__ float sq_f16_lo(uint32_t x) {
  float r;
  asm("v_fma_mix_f32 %0, %1, %1, 0 op_sel_hi:[1,1,0]" : "=v"(r) : "v"(x));
  return r;
}
__device__ __forceinline__ float sq_f16_hi(uint32_t x) {
  float r;
  asm("v_fma_mix_f32 %0, %1, %1, 0 op_sel:[1,1,0] op_sel_hi:[1,1,0]" : "=v"(r) : "v"(x));
  return r;
}
__device__ __forceinline__ double group_sq_f16(const u32x4& r) {
  const uint32_t x[4] = {r.x, r.y, r.z, r.w};
  double q[kVec];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    q[2 * i] = (double)sq_f16_lo(x[i]);
    q[2 * i + 1] = (double)sq_f16_hi(x[i]);
  }
  return tree8(q);
}

// Whether the loss scale is 2^k with |k| <= kPow2MaxExp, i.e. its
// reciprocal 1 / scale is exactly 2^-k.  Tested on the scale's bits, so the
// blocks' choice of path (and their loads) need not wait for the division.
__device__ __forceinline__ bool pow2_scale(float scale) {
  const uint32_t b = __float_as_uint(scale);
  const uint32_t e = b >> 23;  // sign 0 and biased exponent
  return (b & 0x007FFFFFu) == 0u && e >= 127u - kPow2MaxExp && e <= 127u + kPow2MaxExp;
}

// Transposing butterfly over the lanes of one wave: on entry every lane holds
// W values; at step S lanes l and l^(1<<S) add the half they keep to the
// partner's copy of it, so the sum for each value index grows as a pairwise
// tree over lanes in lane order.  On exit vals[0] holds, for value index
// `idx`, the tree over the aligned group of W lanes containing this lane.
template <int W, int S>
__device__ __forceinline__ void transpose_reduce(double* vals, int lane, int& idx) {
  if constexpr (W > 1) {
    constexpr int H = W / 2;
    const bool upper = (lane >> S) & 1;
#pragma unroll
    for (int i = 0; i < H; ++i) {
      const double keep = upper ? vals[H + i] : vals[i];
      const double send = upper ? vals[i] : vals[H + i];
      vals[i] = keep + __shfl_xor(send, 1 << S);
    }
    if (upper) idx += H;
    transpose_reduce<H, S + 1>(vals, lane, idx);
  }
}

template <int kFrom>
__device__ __forceinline__ double butterfly_from(double x) {
#pragma unroll
  for (int s = kFrom; s < 6; ++s) x = x + __shfl_xor(x, 1 << s);
  return x;
}

constexpr int log2i(int v) { return v <= 1 ? 0 : 1 + log2i(v / 2); }

// ---- kernel 1: sum of squares + non-finite flag -----------------------------

// One batch of kRed full, 16-byte aligned segments (descriptors d) into
// vals[0, 2*kRed): every lane issues the loads of kLoad segments before using
// any.  NT: non-temporal loads.  SQ16: fp16 gradients under a power-of-two
// unscale, leaves from group_sq_f16 (no per-element finite test).
template <typename GT, int kRed, int kLoad, bool NT, bool SQ16>
__device__ __forceinline__ void fast_batch(const SegDesc (&dsc)[kRed], int tid, float inv,
                                           double* vals, uint32_t& bad) {
  static_assert(!SQ16 || sizeof(GT) == 2, "fp16 gradients only");
#pragma unroll
  for (int b = 0; b < kRed; b += kLoad) {
    typename GradIO<GT>::Raw8 raw[2 * kLoad];
    float inv_k[kLoad];
#pragma unroll
    for (int k = 0; k < kLoad; ++k) {
      const SegDesc& d = dsc[b + k];
      inv_k[k] = (d.flags & kSegNoUnscale) ? 1.0f : inv;
      const GT* g = static_cast<const GT*>(d.g);
      raw[2 * k] = GradIO<GT>::template load8<NT>(g + tid * kVec);
      raw[2 * k + 1] = GradIO<GT>::template load8<NT>(g + kHalfSeg + tid * kVec);
    }
#pragma unroll
    for (int i = 0; i < 2 * kLoad; ++i) {
      if constexpr (SQ16) {
        const double s = (double)inv_k[i / 2] * (double)inv_k[i / 2];  // 2^(2e), exact
        vals[2 * b + i] = group_sq_f16(raw[i]) * s;
      } else {
        float f[kVec];
        GradIO<GT>::unpack8(raw[i], f, bad);
        vals[2 * b + i] = group_sum(f, inv_k[i / 2]);
      }
    }
  }
}

// Block b covers segments [b*SPB, b*SPB + SPB) (SPB <= 8) and writes the
// pairwise tree of their 2*SPB half-segment sums: an aligned subtree of the
// global tree.  A block that saw an inf or NaN gradient writes NaN, so the
// global sum is NaN exactly when some gradient is non-finite (training.rs:291).
// Blocks from nt_from up read with non-temporal loads: they run first, and
// what they read would leave the Infinity Cache before the AdamW pass gets
// there; the blocks below (the last ~256 MiB read, where AdamW starts) keep
// cache-allocating loads.
template <typename GT, int SPB>
__global__ __launch_bounds__(kBlock) void sumsq_kernel(
    const SegDesc* __restrict__ segs, uint32_t nseg, const ark_opt_state* __restrict__ state,
    double* __restrict__ part_sum, uint32_t nt_from) {
  static_assert(SPB >= 1 && SPB <= 8 && (SPB & (SPB - 1)) == 0, "1, 2, 4 or 8 segments");
  constexpr int V = 2 * SPB;  // half-segment values per lane
  // segments whose loads are in flight together (register budget)
  constexpr int kLoadMax = sizeof(GT) == 2 ? 8 : 4;
  constexpr int kLoad = kLoadMax < SPB ? kLoadMax : SPB;
  __shared__ double lds[kBlock / 64][V];

  // Blocks run in reverse: the last block, which usually holds the ragged
  // tail of the table, starts first instead of trailing the grid.
  const uint32_t blk = gridDim.x - 1u - blockIdx.x;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const uint32_t s0 = blk * SPB;
  // The block's descriptors come first, with no other load in front of them:
  // whether it takes the vector path (every segment present, full and
  // 16-byte aligned) follows from them by scalar compares, so the data loads
  // wait for one scalar round trip.  Every field is in registers before the
  // first branch, so the loads go out together instead of the compiler
  // sinking the pointers' past the checks.
  asm volatile("" : "+s"(nt_from));
  float loss_scale = state->loss_scale;
  SegDesc dsc[SPB];
#pragma unroll
  for (int k = 0; k < SPB; ++k) dsc[k] = segs[s0 + k < nseg ? s0 + k : nseg - 1u];
#pragma unroll
  for (int k = 0; k < SPB; ++k)
    asm volatile("" : "+s"(dsc[k].g), "+s"(dsc[k].n), "+s"(dsc[k].flags));
  asm volatile("" : "+s"(loss_scale));
  const float inv = 1.0f / loss_scale;  // training.rs:244
  bool fast = s0 + SPB <= nseg;
#pragma unroll
  for (int k = 0; k < SPB; ++k)
    fast = fast && dsc[k].n == (uint32_t)kSeg && (dsc[k].flags & kSegVec) != 0u;

  bool sq16 = false;
  if constexpr (sizeof(GT) == 2) sq16 = fast && pow2_scale(loss_scale);

  uint32_t bad = 0;
  double vals[V];
  if (sq16 && blk >= nt_from) {
    if constexpr (sizeof(GT) == 2) fast_batch<GT, SPB, kLoad, true, true>(dsc, tid, inv, vals, bad);
  } else if (sq16) {
    if constexpr (sizeof(GT) == 2) fast_batch<GT, SPB, kLoad, false, true>(dsc, tid, inv, vals, bad);
  } else if (fast && blk >= nt_from) {
    fast_batch<GT, SPB, kLoad, true, false>(dsc, tid, inv, vals, bad);
  } else if (fast) {
    fast_batch<GT, SPB, kLoad, false, false>(dsc, tid, inv, vals, bad);
  } else {
    // some segment ragged, unaligned or past the end: full aligned segments
    // still take the vector loads, the rest go element by element
#pragma unroll
    for (int k = 0; k < SPB; ++k) {
      if (s0 + k >= nseg) {
        vals[2 * k] = 0.0;
        vals[2 * k + 1] = 0.0;
        continue;
      }
      const SegDesc& d = dsc[k];
      const float inv_t = (d.flags & kSegNoUnscale) ? 1.0f : inv;
      const GT* g = static_cast<const GT*>(d.g);
      if (d.n == (uint32_t)kSeg && (d.flags & kSegVec)) {
        const typename GradIO<GT>::Raw8 r0 = GradIO<GT>::load8(g + tid * kVec);
        const typename GradIO<GT>::Raw8 r1 = GradIO<GT>::load8(g + kHalfSeg + tid * kVec);
        float f[kVec];
        GradIO<GT>::unpack8(r0, f, bad);
        vals[2 * k] = group_sum(f, inv_t);
        GradIO<GT>::unpack8(r1, f, bad);
        vals[2 * k + 1] = group_sum(f, inv_t);
        continue;
      }
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint32_t e0 = h * kHalfSeg + tid * kVec;
        float f[kVec];
#pragma unroll
        for (int j = 0; j < kVec; ++j)
          f[j] = (e0 + j < d.n) ? GradIO<GT>::load1(g + e0 + j, bad) : 0.0f;
        vals[2 * k + h] = group_sum(f, inv_t);
      }
    }
  }

  int idx = 0;
  transpose_reduce<V, 0>(vals, lane, idx);
  const double wsum = butterfly_from<log2i(V)>(vals[0]);
  if (lane < V) lds[wave][idx] = wsum;
  const int any_bad = __syncthreads_or((int)bad);
  if (wave == 0) {
    double x = 0.0;
    if (lane < V) x = (lds[0][lane] + lds[1][lane]) + (lds[2][lane] + lds[3][lane]);
    // pairwise over the V half-segment sums in lane (= index) order
#pragma unroll
    for (int st = 0; st < log2i(V); ++st) x = x + __shfl_xor(x, 1 << st);
    // sq16 blocks: a non-finite sum is exactly a non-finite gradient
    const bool nonfinite = any_bad || (sq16 && !__builtin_isfinite(x));
    if (tid == 0) part_sum[blk] = nonfinite ? __builtin_nan("") : x;
  }
}

// ---- kernel 1 from units (ark_opt_internal.hpp) ----------------------------

// One wave per norm block: the block's SPB * kUnitsPerSeg units, zero past a
// segment's end and past the last segment, summed as a pairwise tree in index
// order (K consecutive units per lane, then the lanes in lane order).  That is
// the perfect binary tree sumsq_kernel forms over the block's elements, so
// the partial has the same bits; a NaN unit (a non-finite gradient) makes the
// partial NaN.
template <int SPB>
__global__ __launch_bounds__(64) void units_reduce_kernel(const double* __restrict__ units,
                                                          const SegDesc* __restrict__ segs,
                                                          uint32_t nseg,
                                                          double* __restrict__ part_sum) {
  constexpr int U = SPB * kUnitsPerSeg;     // 16 .. 128 units per block
  constexpr int K = U >= 64 ? U / 64 : 1;   // units per lane
  constexpr int L = U >= 64 ? 64 : U;       // lanes holding units
  static_assert(K <= kUnitsPerSeg, "a lane's units lie in one segment");
  const uint32_t lane = threadIdx.x;
  double x = 0.0;
  if (lane < (uint32_t)L) {
    const uint32_t u0 = lane * K;
    const uint32_t s = blockIdx.x * SPB + u0 / kUnitsPerSeg;
    double q[K];
#pragma unroll
    for (int k = 0; k < K; ++k) q[k] = 0.0;
    if (s < nseg) {
      const uint32_t n = segs[s].n;
      const double* p = units + (uint64_t)s * kUnitsPerSeg + u0 % kUnitsPerSeg;
#pragma unroll
      for (int k = 0; k < K; ++k)
        if ((u0 % kUnitsPerSeg + k) * (uint32_t)kUnit < n) q[k] = p[k];
    }
#pragma unroll
    for (int w = K / 2; w >= 1; w /= 2)
#pragma unroll
      for (int i = 0; i < w; ++i) q[i] = q[2 * i] + q[2 * i + 1];
    x = q[0];
  }
#pragma unroll
  for (int st = 0; st < log2i(L); ++st) x = x + __shfl_xor(x, 1 << st);
  if (lane == 0) part_sum[blockIdx.x] = x;
}

// ---- kernel 2: finalize ----------------------------------------------------

// Pairwise tree over p[0, L) (p 16-byte aligned, L a power of two).
template <int L>
__device__ __forceinline__ double leaf_tree(const double* __restrict__ p) {
  if constexpr (L == 1) {
    return p[0];
  } else if constexpr (L == 2) {
    typedef double f64x2 __attribute__((ext_vector_type(2)));
    const f64x2 v = *(const ARK_GLOBAL f64x2*)p;
    return v.x + v.y;
  } else {
    const double a = leaf_tree<L / 2>(p);
    const double b = leaf_tree<L / 2>(p + L / 2);
    return a + b;
  }
}

// Many partials: one wave per aligned group of kFoldGroup partials writes the
// group's pairwise tree (again an aligned subtree), so the single-block
// finalize never reads more than kFinTarget values.
__global__ __launch_bounds__(kFoldGroup) void fold_kernel(const double* __restrict__ in,
                                                          double* __restrict__ out) {
  double x = in[blockIdx.x * kFoldGroup + threadIdx.x];
  x = butterfly_from<0>(x);
  if (threadIdx.x == 0) out[blockIdx.x] = x;
}

__device__ inline uint32_t amp_skip(const ark_opt_hparams& hp, ark_opt_state& st) {
  // training.rs:294-301 (and :231-236 for the logits-gradient check)
  st.loss_scale = fmaxf(st.loss_scale * 0.5f, hp.loss_scale_min);
  st.clean_steps = 0u;
  st.skipped_steps += 1u;
  st.consecutive_nonfinite += 1u;
  if (st.consecutive_nonfinite > hp.max_consecutive_nonfinite) {
    st.early_stop = 1u;
    return ARK_OPT_EARLY_STOP;
  }
  return ARK_OPT_OK;
}

// part_sum holds kFinThreads * L partials, zero past the last block's.
// lr_ptr: when not NULL, this step's learning rate is *lr_ptr (read as the
// kernel runs) instead of lr; a non-finite one makes the step a no-op that
// reports ARK_OPT_EINVAL.
template <int L>
__global__ __launch_bounds__(kFinThreads) void finalize_kernel(
    const double* __restrict__ part_sum, ark_opt_hparams hp, float lr,
    const float* __restrict__ lr_ptr, ark_opt_state* __restrict__ state,
    StepScalars* __restrict__ scal, ark_opt_step_info* __restrict__ info) {
  __shared__ double wsum[kFinThreads / 64];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;

  double x = leaf_tree<L>(part_sum + (uint32_t)tid * L);
  x = butterfly_from<0>(x);
  if (lane == 0) wsum[wave] = x;
  __syncthreads();
  if (wave != 0) return;
  double y = lane < kFinThreads / 64 ? wsum[lane] : 0.0;
#pragma unroll
  for (int s = 0; s < log2i(kFinThreads / 64); ++s) y = y + __shfl_xor(y, 1 << s);
  if (lane != 0) return;

  if (lr_ptr) lr = *lr_ptr;
  const double sumsq = y;
  const bool any_bad = __builtin_isnan(sumsq);
  ark_opt_state st = *state;
  StepScalars sc = {};
  ark_opt_step_info out = {};
  sc.c1 = 1.0f - hp.beta1;
  sc.c2 = 1.0f - hp.beta2;
  sc.lr = lr;
  sc.coef = 1.0f;
  out.lr = lr;
  out.clip_coef = 1.0f;
  out.status = ARK_OPT_OK;
  if (st.early_stop) {
    out.status = ARK_OPT_EARLY_STOP;
    out.inv_scale = 1.0f / st.loss_scale;
  } else if (!(fabsf(lr) <= 3.402823466e38f)) {  // a non-finite lr: nothing changes
    out.status = ARK_OPT_EINVAL;
    out.inv_scale = 1.0f / st.loss_scale;
    sc.lr = 0.0f;
  } else {
    const float scale = st.loss_scale;
    const float inv = 1.0f / scale;  // training.rs:244
    sc.inv = inv;
    out.inv_scale = inv;
    out.grad_sumsq = sumsq;
    const float norm = sqrtf((float)sumsq);  // optimizer.rs:145
    out.grad_norm = norm;
    if (any_bad) {  // training.rs:293-305: no update, t unchanged
      out.nonfinite = 1;
      out.status = (int32_t)amp_skip(hp, st);
    } else {
      const bool clipped = (norm > hp.grad_clip) && (norm > 0.0f);  // :148
      const float coef = clipped ? hp.grad_clip / norm : 1.0f;     // :149
      st.t += 1u;                                                   // :172
      sc.applied = 1u;
      sc.clipped = clipped ? 1u : 0u;
      sc.coef = coef;
      sc.lr_eff = lr_eff_of(lr, hp.beta1, hp.beta2, st.t);
      out.applied = 1;
      out.clipped = clipped ? 1 : 0;
      out.clip_coef = coef;
      out.lr_eff = sc.lr_eff;
      st.clean_steps += 1u;           // training.rs:317
      st.consecutive_nonfinite = 0u;  // :318
      if (st.clean_steps >= hp.scale_up_every) {                     // :319
        const float nueva = fminf(scale * 2.0f, hp.loss_scale_max);  // :320
        if (nueva > scale) st.loss_scale = nueva;                     // :321
        st.clean_steps = 0u;                                          // :325
      }
    }
  }
  out.state = st;
  *state = st;
  *scal = sc;
  *info = out;
}

__global__ void record_overflow_kernel(ark_opt_hparams hp,
                                       ark_opt_state* __restrict__ state,
                                       ark_opt_step_info* __restrict__ info) {
  ark_opt_state st = *state;
  ark_opt_step_info out = {};
  out.nonfinite = 1;
  out.clip_coef = 1.0f;
  out.inv_scale = 1.0f / st.loss_scale;
  if (st.early_stop) {
    out.status = ARK_OPT_EARLY_STOP;
  } else {
    out.status = (int32_t)amp_skip(hp, st);
  }
  out.state = st;
  *state = st;
  *info = out;
}

// ---- kernel 3: fused AdamW -------------------------------------------------

struct ElemConsts {
  float beta1, beta2, c1, c2, eps, lr_eff, decay;
};

// One element of opti.s:278-308 (the 4-wide loop; the scalar tail :317-346
// is the same sequence).
__device__ __forceinline__ uint32_t adam_elem(uint32_t w16, float g, float& m,
                                              float& v, const ElemConsts& k) {
  float w = h2f(w16);                 // fcvtl
  float mm = m * k.beta1;             // fmul
  mm = __builtin_fmaf(k.c1, g, mm);   // fmla
  float vv = v * k.beta2;             // fmul
  const float gg = g * g;             // fmul
  vv = __builtin_fmaf(k.c2, gg, vv);  // fmla
  float d = sqrtf(vv);                // fsqrt
  d = d + k.eps;                      // fadd
  float u = mm / d;                   // fdiv
  u = u * k.lr_eff;                   // fmul
  w = w * k.decay;                    // fmul
  w = w - u;                          // fsub
  m = mm;
  v = vv;
  return f2h(w);                      // fcvtn
}

// One element of _ark_asm_adam_step (opti.s:105-131; the tail :135-160 is
// the same sequence): adam_elem's operations on an fp32 weight, without the
// fp16 widening and narrowing.
__device__ __forceinline__ float adam_elem_w32(float w, float g, float& m, float& v,
                                               const ElemConsts& k) {
  float mm = m * k.beta1;             // fmul  :114
  mm = __builtin_fmaf(k.c1, g, mm);   // fmla  :115
  float vv = v * k.beta2;             // fmul  :118
  const float gg = g * g;             // fmul  :119
  vv = __builtin_fmaf(k.c2, gg, vv);  // fmla  :120
  float d = sqrtf(vv);                // fsqrt :123
  d = d + k.eps;                      // fadd  :124
  float u = mm / d;                   // fdiv  :125
  u = u * k.lr_eff;                   // fmul  :126
  w = w * k.decay;                    // fmul  :128
  w = w - u;                          // fsub  :129
  m = mm;
  v = vv;
  return w;
}

// The elements [0, valid) of one 256-element row, one wave: lane l owns
// [4l, 4l + 4).  Full aligned rows use one coalesced access per array.
template <typename GT>
__device__ __forceinline__ void adam_row(uint16_t* w, const GT* g, float* m, float* v,
                                         uint32_t valid, bool vec, float inv_t,
                                         float coef, const ElemConsts& k) {
  const uint32_t e = threadIdx.x * 4u;
  if (vec && valid == (uint32_t)kRow) {
    const typename GradIO<GT>::Raw4 gr = GradIO<GT>::load4(g + e);
    const u32x2 wr = ld_nt<u32x2>(w + e);
    const f32x4 mr = ld_nt<f32x4>(m + e);
    const f32x4 vr = ld_nt<f32x4>(v + e);
    float gf[4];
    GradIO<GT>::unpack4(gr, gf);
    float mm[4] = {mr.x, mr.y, mr.z, mr.w};
    float vv[4] = {vr.x, vr.y, vr.z, vr.w};
    const uint32_t wi[4] = {wr.x & 0xFFFFu, wr.x >> 16, wr.y & 0xFFFFu, wr.y >> 16};
    uint32_t wo[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      // training.rs:308, then optimizer.rs:151-165 (coef is exactly 1.0f
      // when the step does not clip, and x * 1.0f == x bit for bit)
      const float gj = (gf[j] * inv_t) * coef;
      wo[j] = adam_elem(wi[j], gj, mm[j], vv[j], k);
    }
    st_nt<u32x2>(w + e, u32x2{wo[0] | (wo[1] << 16), wo[2] | (wo[3] << 16)});
    st_nt<f32x4>(m + e, f32x4{mm[0], mm[1], mm[2], mm[3]});
    st_nt<f32x4>(v + e, f32x4{vv[0], vv[1], vv[2], vv[3]});
  } else {
    uint32_t unused = 0;
    for (int j = 0; j < 4; ++j) {
      const uint32_t i = e + j;
      if (i >= valid) break;
      const float gj = (GradIO<GT>::load1(g + i, unused) * inv_t) * coef;
      float mj = ld_g<float>(m + i), vj = ld_g<float>(v + i);
      const uint32_t wj = adam_elem(ld_g<uint16_t>(w + i), gj, mj, vj, k);
      st_g<uint16_t>(w + i, (uint16_t)wj);
      st_g<float>(m + i, mj);
      st_g<float>(v + i, vj);
    }
  }
}

template <typename GT>
__global__ __launch_bounds__(64) void adamw_kernel(
    const SegDesc* __restrict__ segs, const StepScalars* __restrict__ scal,
    float beta1, float beta2, float eps) {
  SegDesc d = segs[blockIdx.x / kRowsPerSeg];
  StepScalars sc = *scal;
  // Every field used below is in registers before the first branch, so the
  // wave waits for one round trip of scalar loads rather than a chain of
  // them (left alone, the compiler loads the step scalars, branches, then
  // loads the descriptor).
  asm volatile("" : "+s"(d.w), "+s"(d.g), "+s"(d.m), "+s"(d.v), "+s"(d.n), "+s"(d.wd),
               "+s"(d.flags), "+s"(sc.applied), "+s"(sc.inv), "+s"(sc.coef), "+s"(sc.lr),
               "+s"(sc.lr_eff), "+s"(sc.c1), "+s"(sc.c2));
  if (!sc.applied) return;  // skipped step: training.rs:293-305
  const uint32_t r0 = (blockIdx.x % kRowsPerSeg) * kRow;
  if (r0 >= d.n) return;  // row past the end of a short segment
  const uint32_t valid = d.n - r0 < (uint32_t)kRow ? d.n - r0 : (uint32_t)kRow;
  ElemConsts c;
  c.beta1 = beta1;
  c.beta2 = beta2;
  c.c1 = sc.c1;
  c.c2 = sc.c2;
  c.eps = eps;
  c.lr_eff = sc.lr_eff;
  c.decay = 1.0f - sc.lr * d.wd;  // opti.s:219-221 with the tensor's wd
  const float inv_t = (d.flags & kSegNoUnscale) ? 1.0f : sc.inv;
  adam_row<GT>(d.w + r0, static_cast<const GT*>(d.g) + r0, d.m + r0, d.v + r0, valid,
               (d.flags & kSegVec) != 0, inv_t, sc.coef, c);
}

__global__ __launch_bounds__(64) void adamw_single_kernel(
    uint16_t* w, const float* g, float* m, float* v, uint64_t n, float wd,
    uint32_t vec, StepScalars sc, float beta1, float beta2, float eps) {
  const uint64_t r0 = (uint64_t)blockIdx.x * kRow;
  const uint32_t valid = n - r0 < (uint64_t)kRow ? (uint32_t)(n - r0) : (uint32_t)kRow;
  ElemConsts c;
  c.beta1 = beta1;
  c.beta2 = beta2;
  c.c1 = sc.c1;
  c.c2 = sc.c2;
  c.eps = eps;
  c.lr_eff = sc.lr_eff;
  c.decay = 1.0f - sc.lr * wd;
  adam_row<float>(w + r0, g + r0, m + r0, v + r0, valid, vec != 0, 1.0f, 1.0f, c);
}

// ark_hip_adam_step: one wave per 256-element row of an fp32-weight tensor,
// lane l on elements [4l, 4l + 4), one 16-byte access per array when the row
// is full and every pointer 16-byte aligned.
__global__ __launch_bounds__(64) void adamw_single_w32_kernel(
    float* w, const float* g, float* m, float* v, uint64_t n, float wd, uint32_t vec,
    StepScalars sc, float beta1, float beta2, float eps) {
  const uint64_t r0 = (uint64_t)blockIdx.x * kRow;
  const uint32_t valid = n - r0 < (uint64_t)kRow ? (uint32_t)(n - r0) : (uint32_t)kRow;
  ElemConsts c;
  c.beta1 = beta1;
  c.beta2 = beta2;
  c.c1 = sc.c1;
  c.c2 = sc.c2;
  c.eps = eps;
  c.lr_eff = sc.lr_eff;
  c.decay = 1.0f - sc.lr * wd;
  const uint64_t e = r0 + threadIdx.x * 4u;
  if (vec && valid == (uint32_t)kRow) {
    const f32x4 gr = ld_nt<f32x4>(g + e);
    const f32x4 wr = ld_nt<f32x4>(w + e);
    const f32x4 mr = ld_nt<f32x4>(m + e);
    const f32x4 vr = ld_nt<f32x4>(v + e);
    const float gf[4] = {gr.x, gr.y, gr.z, gr.w};
    float ww[4] = {wr.x, wr.y, wr.z, wr.w};
    float mm[4] = {mr.x, mr.y, mr.z, mr.w};
    float vv[4] = {vr.x, vr.y, vr.z, vr.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) ww[j] = adam_elem_w32(ww[j], gf[j], mm[j], vv[j], c);
    st_nt<f32x4>(w + e, f32x4{ww[0], ww[1], ww[2], ww[3]});
    st_nt<f32x4>(m + e, f32x4{mm[0], mm[1], mm[2], mm[3]});
    st_nt<f32x4>(v + e, f32x4{vv[0], vv[1], vv[2], vv[3]});
  } else {
    for (uint32_t j = 0; j < 4; ++j) {
      const uint64_t i = e + j;
      if (i >= r0 + valid) break;
      float mj = ld_g<float>(m + i), vj = ld_g<float>(v + i);
      const float wj = adam_elem_w32(ld_g<float>(w + i), ld_g<float>(g + i), mj, vj, c);
      st_g<float>(w + i, wj);
      st_g<float>(m + i, mj);
      st_g<float>(v + i, vj);
    }
  }
}

// ---- the single-tensor clip (ark_asm_grad_clip, opti.s:369-432) ----------

// Block b covers elements [b * 2 * kSeg, (b + 1) * 2 * kSeg) of one fp32
// array and writes the pairwise tree of its squares: the same lane layout and
// reduction as sumsq_kernel<float, 2> over a one-tensor table, so the partial
// is an aligned subtree of the canonical tree.  No non-finite flag: an inf
// value squares to inf and a NaN to NaN, and the f64 tree carries them (+inf
// unless a NaN is present), as the reference's fmla chain does.
// Blocks run last to first, and blocks from nt_from up read with
// non-temporal loads, so the first kNormCachedBytes of the array, read last,
// stay in the Infinity Cache for clip_scale_kernel, which starts there.
__global__ __launch_bounds__(kBlock) void clip_norm_kernel(const float* __restrict__ g,
                                                           uint64_t n, uint32_t vec,
                                                           uint32_t nt_from,
                                                           double* __restrict__ part_sum) {
  constexpr int V = 4;  // two segments, two halves each
  __shared__ double lds[kBlock / 64][V];
  const uint32_t blk = gridDim.x - 1u - blockIdx.x;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const uint64_t base = (uint64_t)blk * (2u * kSeg);
  const float* p = g + base;
  double vals[V];
  uint32_t bad = 0;  // unused: non-finite values stay in the sum
  if (vec && base + 2u * kSeg <= n) {
    GradIO<float>::Raw8 raw[V];
    if (blk >= nt_from) {
#pragma unroll
      for (int h = 0; h < V; ++h)
        raw[h] = GradIO<float>::load8<true>(p + h * kHalfSeg + tid * kVec);
    } else {
#pragma unroll
      for (int h = 0; h < V; ++h)
        raw[h] = GradIO<float>::load8<false>(p + h * kHalfSeg + tid * kVec);
    }
#pragma unroll
    for (int h = 0; h < V; ++h) {
      float f[kVec];
      GradIO<float>::unpack8(raw[h], f, bad);
      vals[h] = group_sum(f, 1.0f);
    }
  } else {
    const uint64_t left = n - base;
#pragma unroll
    for (int h = 0; h < V; ++h) {
      const uint64_t e0 = (uint64_t)h * kHalfSeg + (uint64_t)tid * kVec;
      float f[kVec];
#pragma unroll
      for (int j = 0; j < kVec; ++j) f[j] = (e0 + j < left) ? ld_g<float>(p + e0 + j) : 0.0f;
      vals[h] = group_sum(f, 1.0f);
    }
  }
  int idx = 0;
  transpose_reduce<V, 0>(vals, lane, idx);
  const double wsum = butterfly_from<log2i(V)>(vals[0]);
  if (lane < V) lds[wave][idx] = wsum;
  __syncthreads();
  if (wave == 0) {
    double x = 0.0;
    if (lane < V) x = (lds[0][lane] + lds[1][lane]) + (lds[2][lane] + lds[3][lane]);
#pragma unroll
    for (int st = 0; st < log2i(V); ++st) x = x + __shfl_xor(x, 1 << st);
    if (tid == 0) part_sum[blk] = x;
  }
}

// fold_kernel over nparts partials read as zero past the last one.
__global__ __launch_bounds__(kFoldGroup) void clip_fold_kernel(const double* __restrict__ in,
                                                               uint32_t nparts,
                                                               double* __restrict__ out) {
  const uint32_t i = blockIdx.x * kFoldGroup + threadIdx.x;
  double x = i < nparts ? in[i] : 0.0;
  x = butterfly_from<0>(x);
  if (threadIdx.x == 0) out[blockIdx.x] = x;
}

// The root of the tree over nparts leaves (zero past them, padded to
// kFinThreads * L), as finalize_kernel forms it; then the decision of
// opti.s:399-404: norm = fsqrt of the sum as fp32 (the reference's sum is
// fp32), clipped when norm > threshold (fcmp + b.le: an unordered compare
// does not clip), coefficient threshold / norm.
template <int L>
__global__ __launch_bounds__(kFinThreads) void clip_finalize_kernel(
    const double* __restrict__ leaves, uint32_t nparts, float threshold,
    ClipScalars* __restrict__ out) {
  __shared__ double wsum[kFinThreads / 64];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  double q[L];
#pragma unroll
  for (int j = 0; j < L; ++j) {
    const uint32_t i = (uint32_t)tid * L + j;
    q[j] = i < nparts ? leaves[i] : 0.0;
  }
#pragma unroll
  for (int w = L / 2; w >= 1; w /= 2)
#pragma unroll
    for (int j = 0; j < w; ++j) q[j] = q[2 * j] + q[2 * j + 1];
  double x = butterfly_from<0>(q[0]);
  if (lane == 0) wsum[wave] = x;
  __syncthreads();
  if (wave != 0) return;
  double y = lane < kFinThreads / 64 ? wsum[lane] : 0.0;
#pragma unroll
  for (int s = 0; s < log2i(kFinThreads / 64); ++s) y = y + __shfl_xor(y, 1 << s);
  if (lane != 0) return;
  ClipScalars c;
  c.sumsq = y;
  c.norm = sqrtf((float)y);
  c.clipped = c.norm > threshold ? 1u : 0u;
  c.coef = c.clipped ? threshold / c.norm : 1.0f;
  *out = c;
}

// g[i] = g[i] * coef (fmul, opti.s:409-420) when the finalize decided to
// clip; otherwise every block exits at once.  Grid-stride over 4-element
// groups.
__global__ __launch_bounds__(256) void clip_scale_kernel(float* __restrict__ g, uint64_t n,
                                                         uint32_t vec,
                                                         const ClipScalars* __restrict__ cs) {
  const uint32_t clipped = cs->clipped;
  const float coef = cs->coef;
  if (!clipped) return;
  const uint64_t stride = (uint64_t)gridDim.x * 256u * 4u;
  for (uint64_t e = ((uint64_t)blockIdx.x * 256u + threadIdx.x) * 4u; e < n; e += stride) {
    if (vec && e + 4u <= n) {
      f32x4 x = ld_nt<f32x4>(g + e);
      x.x = x.x * coef;
      x.y = x.y * coef;
      x.z = x.z * coef;
      x.w = x.w * coef;
      st_nt<f32x4>(g + e, x);
    } else {
      for (uint64_t j = e; j < e + 4u && j < n; ++j) st_g<float>(g + j, ld_g<float>(g + j) * coef);
    }
  }
}

}  // namespace

hipError_t launch_grad_clip(float* g, uint64_t n, float threshold, double* parts,
                            double* folded, ClipScalars* out, hipStream_t stream) {
  const uint32_t nparts = clip_parts(n);
  const uint32_t vec = ((uintptr_t)g & 15u) == 0 ? 1u : 0u;
  const uint32_t nt_from = (uint32_t)(kNormCachedBytes / (2u * kSeg * sizeof(float)));
  hipLaunchKernelGGL(clip_norm_kernel, dim3(nparts), dim3(kBlock), 0, stream, g, n, vec, nt_from,
                     parts);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const double* leaves = parts;
  uint32_t nleaves = nparts;
  if (nparts > kFinTarget) {
    const uint32_t groups = (nparts + kFoldGroup - 1) / kFoldGroup;
    hipLaunchKernelGGL(clip_fold_kernel, dim3(groups), dim3(kFoldGroup), 0, stream, parts,
                       nparts, folded);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    leaves = folded;
    nleaves = groups;
  }
  const dim3 one(1), fin(kFinThreads);
#define ARK_CLIP_FIN(L)                                                                         hipLaunchKernelGGL((clip_finalize_kernel<L>), one, fin, 0, stream, leaves, nleaves, threshold,                      out)
  switch (finalize_leaves(nleaves)) {
    case 1: ARK_CLIP_FIN(1); break;
    case 2: ARK_CLIP_FIN(2); break;
    case 4: ARK_CLIP_FIN(4); break;
    case 8: ARK_CLIP_FIN(8); break;
    default: return hipErrorInvalidValue;
  }
#undef ARK_CLIP_FIN
  if ((e = hipGetLastError()) != hipSuccess) return e;
  uint64_t blocks = (n + 1023u) / 1024u;
  if (blocks > 65536u) blocks = 65536u;
  hipLaunchKernelGGL(clip_scale_kernel, dim3((uint32_t)blocks), dim3(256), 0, stream, g, n, vec,
                     (const ClipScalars*)out);
  return hipGetLastError();
}

int sumsq_spb(uint64_t nseg, uint32_t grad_dtype) {
  // fp16 gradients: 2 segments (16 KiB) per block measured fastest for the
  // norm pass on MI355X, fold included: 78.9 against 80.8 us at EKO-237M with
  // 8, 15.1 against 18.0 us on an eighth of it, 55.7 against 57.3 us on an
  // eighth of the 1.3B set; 1 segment per block is slower (93 us at
  // EKO-237M: each block's descriptor load then stands alone in front of
  // its data loads), as are 16 and 32.
  // fp32 gradients: 8.  Such a handle's norm usually comes from the units
  // the gradient hand-off wrote (units_reduce_kernel: one wave per block
  // reads 16 doubles per segment), whose cost is per block, not per byte: at
  // EKO-237M 4.5 us with 8 segments per block and no fold, against 8.5 us
  // plus a 4.5 us fold with 2 (the reading pass gains 4.6 us with 2).
  // Larger blocks only when the partials would exceed kMaxParts (beyond
  // 2^31 elements); 8 covers every table kMaxSegments allows.  A small table
  // gets smaller blocks until the grid has two blocks per CU (512): the pass
  // is then latency bound, and one EKO 768x768 tensor steps in 9.9 instead
  // of 12.0 us.
  int spb = grad_dtype == ARK_OPT_GRAD_F32 ? 8 : 2;
  while (spb < 8 && (nseg + spb - 1) / spb > kMaxParts) spb *= 2;
  while (spb > 1 && (nseg + spb - 1) / spb < 512) spb /= 2;
  return spb;
}

hipError_t launch_fold(uint32_t padded_parts, const double* in, double* out,
                       hipStream_t stream) {
  if (padded_parts % kFoldGroup) return hipErrorInvalidValue;
  hipLaunchKernelGGL(fold_kernel, dim3(padded_parts / kFoldGroup), dim3(kFoldGroup), 0,
                     stream, in, out);
  return hipGetLastError();
}

hipError_t launch_sumsq(uint32_t grad_dtype, int spb, uint32_t nblocks,
                        const SegDesc* segs, uint32_t nseg, const ark_opt_state* state,
                        double* part_sum, uint32_t nt_from, uint32_t lds_bytes,
                        hipStream_t stream) {
  const dim3 grid(nblocks), block(kBlock);
#define ARK_SUMSQ(GT, SPB)                                                                \
  hipLaunchKernelGGL((sumsq_kernel<GT, SPB>), grid, block, lds_bytes, stream, segs, nseg, \
                     state, part_sum, nt_from)
  switch (spb * 2 + (grad_dtype == ARK_OPT_GRAD_F16 ? 0 : 1)) {
    case 2: ARK_SUMSQ(uint16_t, 1); break;
    case 4: ARK_SUMSQ(uint16_t, 2); break;
    case 8: ARK_SUMSQ(uint16_t, 4); break;
    case 16: ARK_SUMSQ(uint16_t, 8); break;
    case 3: ARK_SUMSQ(float, 1); break;
    case 5: ARK_SUMSQ(float, 2); break;
    case 9: ARK_SUMSQ(float, 4); break;
    case 17: ARK_SUMSQ(float, 8); break;
    default: return hipErrorInvalidValue;
  }
#undef ARK_SUMSQ
  return hipGetLastError();
}

hipError_t launch_units_reduce(int spb, uint32_t nblocks, const double* units,
                               const SegDesc* segs, uint32_t nseg, double* part_sum,
                               hipStream_t stream) {
  const dim3 grid(nblocks), block(64);
#define ARK_UNITS(SPB)                                                                     \
  hipLaunchKernelGGL((units_reduce_kernel<SPB>), grid, block, 0, stream, units, segs, nseg, \
                     part_sum)
  switch (spb) {
    case 1: ARK_UNITS(1); break;
    case 2: ARK_UNITS(2); break;
    case 4: ARK_UNITS(4); break;
    case 8: ARK_UNITS(8); break;
    default: return hipErrorInvalidValue;
  }
#undef ARK_UNITS
  return hipGetLastError();
}

uint32_t sumsq_lds_for(uint32_t grad_dtype, int spb, int blocks) {
  const bool f16 = grad_dtype == ARK_OPT_GRAD_F16;
  const void* k = nullptr;
  switch (spb) {
    case 1: k = f16 ? (const void*)sumsq_kernel<uint16_t, 1> : (const void*)sumsq_kernel<float, 1>; break;
    case 2: k = f16 ? (const void*)sumsq_kernel<uint16_t, 2> : (const void*)sumsq_kernel<float, 2>; break;
    case 4: k = f16 ? (const void*)sumsq_kernel<uint16_t, 4> : (const void*)sumsq_kernel<float, 4>; break;
    case 8: k = f16 ? (const void*)sumsq_kernel<uint16_t, 8> : (const void*)sumsq_kernel<float, 8>; break;
    default: return 0;
  }
  return resident_lds_bytes(k, kBlock, blocks);
}

uint32_t adamw_lds_for(uint32_t grad_dtype, int blocks) {
  const void* k = grad_dtype == ARK_OPT_GRAD_F16 ? (const void*)adamw_kernel<uint16_t>
                                                 : (const void*)adamw_kernel<float>;
  return resident_lds_bytes(k, 64, blocks);
}

uint32_t finalize_leaves(uint32_t nparts) {
  uint32_t L = 1;
  while ((uint64_t)L * kFinThreads < nparts) L <<= 1;
  return L;
}

hipError_t launch_finalize(uint32_t leaves, const double* part_sum,
                           const ark_opt_hparams& hp, float lr, const float* lr_ptr,
                           ark_opt_state* state, StepScalars* scal,
                           ark_opt_step_info* info, hipStream_t stream) {
  const dim3 grid(1), block(kFinThreads);
#define ARK_FIN(L)                                                                   \
  hipLaunchKernelGGL((finalize_kernel<L>), grid, block, 0, stream, part_sum, hp, lr, \
                     lr_ptr, state, scal, info)
  switch (leaves) {
    case 1: ARK_FIN(1); break;
    case 2: ARK_FIN(2); break;
    case 4: ARK_FIN(4); break;
    case 8: ARK_FIN(8); break;
    case 16: ARK_FIN(16); break;
    case 32: ARK_FIN(32); break;
    case 64: ARK_FIN(64); break;
    default: return hipErrorInvalidValue;
  }
#undef ARK_FIN
  return hipGetLastError();
}

hipError_t launch_adamw(uint32_t grad_dtype, const SegDesc* segs, uint32_t nseg,
                        const StepScalars* scal, float beta1, float beta2,
                        float eps, uint32_t lds_bytes, hipStream_t stream) {
  if ((uint64_t)nseg > kMaxSegments) return hipErrorInvalidValue;
  const dim3 grid(nseg * kRowsPerSeg), block(64);
  if (grad_dtype == ARK_OPT_GRAD_F16)
    hipLaunchKernelGGL((adamw_kernel<uint16_t>), grid, block, lds_bytes, stream, segs, scal,
                       beta1, beta2, eps);
  else
    hipLaunchKernelGGL((adamw_kernel<float>), grid, block, lds_bytes, stream, segs, scal,
                       beta1, beta2, eps);
  return hipGetLastError();
}

hipError_t launch_adamw_single(uint16_t* w, const float* g, float* m, float* v,
                               uint64_t n, float wd, bool vec,
                               const StepScalars& sc, float beta1, float beta2,
                               float eps, hipStream_t stream) {
  const uint64_t rows = (n + kRow - 1) / kRow;
  if (rows == 0) return hipSuccess;
  if (rows * 64u >= (1ull << 32)) return hipErrorInvalidValue;
  hipLaunchKernelGGL(adamw_single_kernel, dim3((uint32_t)rows), dim3(64), 0, stream, w,
                     g, m, v, n, wd, vec ? 1u : 0u, sc, beta1, beta2, eps);
  return hipGetLastError();
}

hipError_t launch_adamw_single_w32(float* w, const float* g, float* m, float* v, uint64_t n,
                                   float wd, bool vec, const StepScalars& sc, float beta1,
                                   float beta2, float eps, hipStream_t stream) {
  const uint64_t rows = (n + kRow - 1) / kRow;
  if (rows == 0) return hipSuccess;
  if (rows * 64u >= (1ull << 32)) return hipErrorInvalidValue;
  hipLaunchKernelGGL(adamw_single_w32_kernel, dim3((uint32_t)rows), dim3(64), 0, stream, w, g,
                     m, v, n, wd, vec ? 1u : 0u, sc, beta1, beta2, eps);
  return hipGetLastError();
}

hipError_t launch_record_overflow(const ark_opt_hparams& hp,
                                  ark_opt_state* state,
                                  ark_opt_step_info* info, hipStream_t stream) {
  hipLaunchKernelGGL(record_overflow_kernel, dim3(1), dim3(1), 0, stream, hp,
                     state, info);
  return hipGetLastError();
}

}  // namespace ark
