// ark_opt_kernels.hip -- gfx950 kernels of the optimizer step (see the
// header for the segment layout and the kernel sequence).
//
// Arithmetic follows the reference kernel ark_asm_adam_step_f16
// (proyecto_ark/ark01/asm/opti.s:192-360) operation for operation; the build
// uses -ffp-contract=off so the only fused operations are the explicit
// __builtin_fmaf calls standing for its fmla instructions (opti.s:287, :293).
// f32 sqrt and division compile to the correctly rounded expansions and
// fp16 conversion to v_cvt_f16_f32 under the default round-to-nearest-even
// mode with fp16/fp32 denormals preserved.
#include "ark_opt_kernels.hpp"

namespace ark {
namespace {

__device__ __forceinline__ float h2f(uint16_t b) {
  return (float)__builtin_bit_cast(_Float16, b);
}
// The empty asm makes f opaque, so the preceding fp32 arithmetic can never be
// merged with the conversion into a single-rounding mixed-precision fma: the
// reference rounds to fp32 (fsub) and then to fp16 (fcvtn).
__device__ __forceinline__ uint16_t f2h(float f) {
  asm("" : "+v"(f));
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// ---- gradient access --------------------------------------------------------

template <typename GT>
struct Grad;

template <>
struct Grad<uint16_t> {  // fp16 bits
  static __device__ __forceinline__ void load8(const void* g, uint64_t e,
                                               float (&out)[kVec],
                                               uint32_t& bad) {
    const uint4 raw = *reinterpret_cast<const uint4*>(
        static_cast<const uint16_t*>(g) + e);
    const uint32_t wv[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t x = wv[i];
      bad |= ((x & 0x7C00u) == 0x7C00u) | ((x & 0x7C000000u) == 0x7C000000u);
      out[2 * i] = h2f((uint16_t)(x & 0xFFFFu));
      out[2 * i + 1] = h2f((uint16_t)(x >> 16));
    }
  }
  static __device__ __forceinline__ float load1(const void* g, uint64_t e,
                                                uint32_t& bad) {
    const uint16_t x = static_cast<const uint16_t*>(g)[e];
    bad |= (x & 0x7C00u) == 0x7C00u;
    return h2f(x);
  }
};

template <>
struct Grad<float> {
  static __device__ __forceinline__ void load8(const void* g, uint64_t e,
                                               float (&out)[kVec],
                                               uint32_t& bad) {
    const float4* p =
        reinterpret_cast<const float4*>(static_cast<const float*>(g) + e);
    const float4 a = p[0], b = p[1];
    out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
    out[4] = b.x; out[5] = b.y; out[6] = b.z; out[7] = b.w;
#pragma unroll
    for (int i = 0; i < kVec; ++i)
      bad |= (__float_as_uint(out[i]) & 0x7F800000u) == 0x7F800000u;
  }
  static __device__ __forceinline__ float load1(const void* g, uint64_t e,
                                                uint32_t& bad) {
    const float x = static_cast<const float*>(g)[e];
    bad |= (__float_as_uint(x) & 0x7F800000u) == 0x7F800000u;
    return x;
  }
};

// ---- canonical tree pieces --------------------------------------------------

// Pairwise sum of 8 squares in index order.
__device__ __forceinline__ double tree8(const double (&q)[kVec]) {
  return ((q[0] + q[1]) + (q[2] + q[3])) + ((q[4] + q[5]) + (q[6] + q[7]));
}

// Transposing butterfly over the lanes of one wave: on entry every lane holds
// W values; at step S lanes l and l^(1<<S) add the half they keep to the
// partner's copy of it, so the sum for each value index grows as a pairwise
// tree over lanes in lane order.  On exit vals[0] holds, for value index
// `idx`, the tree over the aligned group of W lanes containing this lane.
template <int W, int S>
__device__ __forceinline__ void transpose_reduce(double* vals, int lane,
                                                 int& idx) {
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

// Block b covers segments [b*SPB, b*SPB + SPB) and writes the pairwise tree
// of their 2*SPB half-segment sums: an aligned subtree of the global tree.
template <typename GT, int SPB>
__global__ __launch_bounds__(kBlock) void sumsq_kernel(
    const TensorDev* __restrict__ tab, const uint32_t* __restrict__ seg_tensor,
    uint32_t nseg, const ark_opt_state* __restrict__ state,
    double* __restrict__ part_sum, uint32_t* __restrict__ part_flag) {
  constexpr int V = 2 * SPB;
  static_assert(V <= 64, "one value index per lane of a wave");
  __shared__ double lds[kBlock / 64][V];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const float inv = 1.0f / state->loss_scale;  // training.rs:244
  uint32_t bad = 0;
  double vals[V];

#pragma unroll
  for (int k = 0; k < SPB; ++k) {
    const uint32_t s = blockIdx.x * SPB + k;
    if (s >= nseg) {
      vals[2 * k] = 0.0;
      vals[2 * k + 1] = 0.0;
      continue;
    }
    const TensorDev& T = tab[seg_tensor[s]];
    const float inv_t = (T.flags & ARK_OPT_TENSOR_NO_UNSCALE) ? 1.0f : inv;
    const uint64_t start = (uint64_t)(s - T.seg0) * kSeg;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint64_t e0 = start + (uint64_t)h * kHalfSeg + (uint64_t)tid * kVec;
      float g[kVec];
      if (T.vec && e0 + kVec <= T.n) {
        Grad<GT>::load8(T.g, e0, g, bad);
      } else {
#pragma unroll
        for (int j = 0; j < kVec; ++j)
          g[j] = (e0 + j < T.n) ? Grad<GT>::load1(T.g, e0 + j, bad) : 0.0f;
      }
      double q[kVec];
#pragma unroll
      for (int j = 0; j < kVec; ++j) {
        const float gu = g[j] * inv_t;  // vDSP_vsmul, ffi.rs:141-146
        q[j] = (double)gu * (double)gu; // exact in f64
      }
      vals[2 * k + h] = tree8(q);
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
    for (int s = 0; s < log2i(V); ++s) x = x + __shfl_xor(x, 1 << s);
    if (lane == 0) {
      part_sum[blockIdx.x] = x;
      part_flag[blockIdx.x] = any_bad ? 1u : 0u;
    }
  }
}

// ---- kernel 2: finalize ----------------------------------------------------

template <int L>
__device__ __forceinline__ double leaf_tree(const double* __restrict__ p,
                                            uint32_t base, uint32_t n) {
  if constexpr (L == 1) {
    return base < n ? p[base] : 0.0;
  } else {
    const double a = leaf_tree<L / 2>(p, base, n);
    const double b = leaf_tree<L / 2>(p, base + L / 2, n);
    return a + b;
  }
}

__device__ inline uint32_t amp_skip(const ark_opt_hparams& hp,
                                    ark_opt_state& st) {
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

template <int L>
__global__ __launch_bounds__(kFinThreads) void finalize_kernel(
    const double* __restrict__ part_sum, const uint32_t* __restrict__ part_flag,
    uint32_t nparts, ark_opt_hparams hp, float lr,
    ark_opt_state* __restrict__ state, StepScalars* __restrict__ scal,
    ark_opt_step_info* __restrict__ info) {
  __shared__ double wsum[kFinThreads / 64];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;

  const uint32_t base = (uint32_t)tid * L;
  double x = leaf_tree<L>(part_sum, base, nparts);
  uint32_t bad = 0;
#pragma unroll
  for (int i = 0; i < L; ++i)
    if (base + i < nparts) bad |= part_flag[base + i];
  x = butterfly_from<0>(x);
  if (lane == 0) wsum[wave] = x;
  const int any_bad = __syncthreads_or((int)bad);
  if (wave != 0) return;
  double y = lane < kFinThreads / 64 ? wsum[lane] : 0.0;
#pragma unroll
  for (int s = 0; s < log2i(kFinThreads / 64); ++s) y = y + __shfl_xor(y, 1 << s);
  if (lane != 0) return;

  const double sumsq = y;
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
      st.clean_steps += 1u;              // training.rs:317
      st.consecutive_nonfinite = 0u;     // :318
      if (st.clean_steps >= hp.scale_up_every) {  // :319
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
__device__ __forceinline__ uint16_t adam_elem(uint16_t w16, float g, float& m,
                                              float& v, const ElemConsts& k) {
  float w = h2f(w16);                // fcvtl
  float mm = m * k.beta1;            // fmul
  mm = __builtin_fmaf(k.c1, g, mm);  // fmla
  float vv = v * k.beta2;            // fmul
  const float gg = g * g;            // fmul
  vv = __builtin_fmaf(k.c2, gg, vv); // fmla
  float d = sqrtf(vv);               // fsqrt
  d = d + k.eps;                     // fadd
  float u = mm / d;                  // fdiv
  u = u * k.lr_eff;                  // fmul
  w = w * k.decay;                   // fmul
  w = w - u;                         // fsub
  m = mm;
  v = vv;
  return f2h(w);                     // fcvtn
}

template <typename GT>
__device__ __forceinline__ void adam_segment(const TensorDev& T, uint64_t start,
                                             float inv_t, uint32_t clipped,
                                             float coef, const ElemConsts& k) {
  const int tid = threadIdx.x;
  uint32_t unused = 0;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint64_t e0 = start + (uint64_t)h * kHalfSeg + (uint64_t)tid * kVec;
    if (T.vec && e0 + kVec <= T.n) {
      float g[kVec];
      Grad<GT>::load8(T.g, e0, g, unused);
      const uint4 wr = *reinterpret_cast<const uint4*>(T.w + e0);
      float4* mp = reinterpret_cast<float4*>(T.m + e0);
      float4* vp = reinterpret_cast<float4*>(T.v + e0);
      const float4 m0 = mp[0], m1 = mp[1];
      const float4 v0 = vp[0], v1 = vp[1];
      float m[kVec] = {m0.x, m0.y, m0.z, m0.w, m1.x, m1.y, m1.z, m1.w};
      float v[kVec] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
      const uint32_t win[4] = {wr.x, wr.y, wr.z, wr.w};
      uint32_t wout[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float ga = g[2 * i] * inv_t;      // training.rs:308
        float gb = g[2 * i + 1] * inv_t;
        if (clipped) {                     // optimizer.rs:151-165
          ga = ga * coef;
          gb = gb * coef;
        }
        const uint16_t lo =
            adam_elem((uint16_t)(win[i] & 0xFFFFu), ga, m[2 * i], v[2 * i], k);
        const uint16_t hi =
            adam_elem((uint16_t)(win[i] >> 16), gb, m[2 * i + 1], v[2 * i + 1], k);
        wout[i] = (uint32_t)lo | ((uint32_t)hi << 16);
      }
      *reinterpret_cast<uint4*>(T.w + e0) = make_uint4(wout[0], wout[1], wout[2], wout[3]);
      mp[0] = make_float4(m[0], m[1], m[2], m[3]);
      mp[1] = make_float4(m[4], m[5], m[6], m[7]);
      vp[0] = make_float4(v[0], v[1], v[2], v[3]);
      vp[1] = make_float4(v[4], v[5], v[6], v[7]);
    } else {
      for (int j = 0; j < kVec; ++j) {
        const uint64_t e = e0 + j;
        if (e >= T.n) break;
        float g = Grad<GT>::load1(T.g, e, unused) * inv_t;
        if (clipped) g = g * coef;
        float m = T.m[e], v = T.v[e];
        T.w[e] = adam_elem(T.w[e], g, m, v, k);
        T.m[e] = m;
        T.v[e] = v;
      }
    }
  }
}

template <typename GT, int SPB>
__global__ __launch_bounds__(kBlock) void adamw_kernel(
    const TensorDev* __restrict__ tab, const uint32_t* __restrict__ seg_tensor,
    uint32_t nseg, const StepScalars* __restrict__ scal, float beta1,
    float beta2, float eps) {
  const StepScalars sc = *scal;
  if (!sc.applied) return;  // skipped step: training.rs:293-305
#pragma unroll
  for (int k = 0; k < SPB; ++k) {
    const uint32_t s = blockIdx.x * SPB + k;
    if (s >= nseg) return;
    const TensorDev& T = tab[seg_tensor[s]];
    ElemConsts c;
    c.beta1 = beta1;
    c.beta2 = beta2;
    c.c1 = sc.c1;
    c.c2 = sc.c2;
    c.eps = eps;
    c.lr_eff = sc.lr_eff;
    c.decay = 1.0f - sc.lr * T.wd;  // opti.s:219-221 (per-tensor wd)
    const float inv_t = (T.flags & ARK_OPT_TENSOR_NO_UNSCALE) ? 1.0f : sc.inv;
    adam_segment<GT>(T, (uint64_t)(s - T.seg0) * kSeg, inv_t, sc.clipped,
                     sc.coef, c);
  }
}

__global__ __launch_bounds__(kBlock) void adamw_single_kernel(
    TensorDev T, StepScalars sc, float beta1, float beta2, float eps) {
  ElemConsts c;
  c.beta1 = beta1;
  c.beta2 = beta2;
  c.c1 = sc.c1;
  c.c2 = sc.c2;
  c.eps = eps;
  c.lr_eff = sc.lr_eff;
  c.decay = 1.0f - sc.lr * T.wd;
  adam_segment<float>(T, (uint64_t)blockIdx.x * kSeg, 1.0f, 0u, 1.0f, c);
}

constexpr int kAdamSpb = 1;

}  // namespace

hipError_t launch_sumsq(uint32_t grad_dtype, int spb, uint32_t nblocks,
                        const TensorDev* tab, const uint32_t* seg_tensor,
                        uint32_t nseg, const ark_opt_state* state,
                        double* part_sum, uint32_t* part_flag,
                        hipStream_t stream) {
  const dim3 grid(nblocks), block(kBlock);
  if (grad_dtype == ARK_OPT_GRAD_F16) {
    if (spb == 8)
      hipLaunchKernelGGL((sumsq_kernel<uint16_t, 8>), grid, block, 0, stream,
                         tab, seg_tensor, nseg, state, part_sum, part_flag);
    else
      hipLaunchKernelGGL((sumsq_kernel<uint16_t, 16>), grid, block, 0, stream,
                         tab, seg_tensor, nseg, state, part_sum, part_flag);
  } else {
    if (spb == 8)
      hipLaunchKernelGGL((sumsq_kernel<float, 8>), grid, block, 0, stream, tab,
                         seg_tensor, nseg, state, part_sum, part_flag);
    else
      hipLaunchKernelGGL((sumsq_kernel<float, 16>), grid, block, 0, stream,
                         tab, seg_tensor, nseg, state, part_sum, part_flag);
  }
  return hipGetLastError();
}

hipError_t launch_finalize(uint32_t nparts, const double* part_sum,
                           const uint32_t* part_flag,
                           const ark_opt_hparams& hp, float lr,
                           ark_opt_state* state, StepScalars* scal,
                           ark_opt_step_info* info, hipStream_t stream) {
  const dim3 grid(1), block(kFinThreads);
  const uint32_t per = (nparts + kFinThreads - 1) / kFinThreads;
#define ARK_FIN(L)                                                          \
  hipLaunchKernelGGL((finalize_kernel<L>), grid, block, 0, stream, part_sum, \
                     part_flag, nparts, hp, lr, state, scal, info)
  if (per <= 1) ARK_FIN(1);
  else if (per <= 2) ARK_FIN(2);
  else if (per <= 4) ARK_FIN(4);
  else if (per <= 8) ARK_FIN(8);
  else if (per <= 16) ARK_FIN(16);
  else if (per <= 32) ARK_FIN(32);
  else if (per <= 64) ARK_FIN(64);
  else return hipErrorInvalidValue;
#undef ARK_FIN
  return hipGetLastError();
}

hipError_t launch_adamw(uint32_t grad_dtype, uint32_t nblocks,
                        const TensorDev* tab, const uint32_t* seg_tensor,
                        uint32_t nseg, const StepScalars* scal, float beta1,
                        float beta2, float eps, hipStream_t stream) {
  const dim3 grid(nblocks), block(kBlock);
  if (grad_dtype == ARK_OPT_GRAD_F16)
    hipLaunchKernelGGL((adamw_kernel<uint16_t, kAdamSpb>), grid, block, 0,
                       stream, tab, seg_tensor, nseg, scal, beta1, beta2, eps);
  else
    hipLaunchKernelGGL((adamw_kernel<float, kAdamSpb>), grid, block, 0, stream,
                       tab, seg_tensor, nseg, scal, beta1, beta2, eps);
  return hipGetLastError();
}

uint32_t adamw_blocks(uint32_t nseg) { return (nseg + kAdamSpb - 1) / kAdamSpb; }

hipError_t launch_adamw_single(const TensorDev& t, const StepScalars& sc,
                               float beta1, float beta2, float eps,
                               hipStream_t stream) {
  const uint64_t nseg = (t.n + kSeg - 1) / kSeg;
  if (nseg == 0) return hipSuccess;
  if (nseg > 0x7FFFFFFFull) return hipErrorInvalidValue;
  hipLaunchKernelGGL(adamw_single_kernel, dim3((uint32_t)nseg), dim3(kBlock),
                     0, stream, t, sc, beta1, beta2, eps);
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
