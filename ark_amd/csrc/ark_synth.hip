// ark_synth.hip -- seeded synthetic inputs on the device (include/ark_synth.h).
// Integer SplitMix64 counters plus two correctly rounded fp32 multiplies, so a
// CPU restatement reproduces every bit.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ark_common.hpp"
#include "ark_synth.h"

namespace {

constexpr uint64_t kGolden = 0x9E3779B97F4A7C15ull;

__host__ __device__ inline uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

__host__ __device__ inline uint64_t synth_base(uint64_t seed, uint32_t tensor_id,
                                               uint32_t step) {
  const uint64_t ctr = ((uint64_t)tensor_id << 32) | (uint64_t)step;
  return mix64(seed + kGolden * (ctr + 1));
}

__device__ inline float synth_z(uint64_t base, uint64_t i) {
  const uint64_t x = mix64(base + kGolden * (i + 1));
  const int32_t u = (int32_t)(x & 0xFFFFu) + (int32_t)((x >> 16) & 0xFFFFu) +
                    (int32_t)((x >> 32) & 0xFFFFu) + (int32_t)((x >> 48) & 0xFFFFu);
  const int32_t d = 2 * u - 262140;
  return (float)d * 0x1.bb67aep-17f;
}

// fp32 -> fp16 after an fp32 product: the value passes through an empty asm so
// the compiler cannot merge the multiply and the conversion into one
// single-rounding mixed-precision fma (the result must be rounded to fp32
// first, then to fp16).
__device__ inline uint16_t f32_to_f16_bits(float y) {
  asm("" : "+v"(y));
  return __builtin_bit_cast(uint16_t, (_Float16)y);
}

template <bool kHalf>
__global__ __launch_bounds__(256) void normal_kernel(void* out, uint64_t n,
                                                     uint64_t base,
                                                     float sigma_scale) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const float y = synth_z(base, i) * sigma_scale;
    if constexpr (kHalf)
      static_cast<uint16_t*>(out)[i] = f32_to_f16_bits(y);
    else
      static_cast<float*>(out)[i] = y;
  }
}

__global__ __launch_bounds__(256) void fill_kernel(uint16_t* out, uint64_t n,
                                                   uint16_t bits) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    out[i] = bits;
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void copy_kernel(u32x4* __restrict__ dst,
                                                   const u32x4* __restrict__ src,
                                                   uint64_t n) {
  const uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x;
  if (i < n)
    __builtin_nontemporal_store(
        __builtin_nontemporal_load((const __attribute__((address_space(1))) u32x4*)(src + i)),
        (__attribute__((address_space(1))) u32x4*)(dst + i));
}

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
#define ARK_G1 __attribute__((address_space(1)))

template <typename T>
__device__ __forceinline__ T ldnt(const void* p) {
  return __builtin_nontemporal_load((const ARK_G1 T*)p);
}
template <typename T>
__device__ __forceinline__ void stnt(void* p, T v) {
  __builtin_nontemporal_store(v, (ARK_G1 T*)p);
}

// The optimizer's AdamW row without its arithmetic: one wave per 256-element
// row, lane l on elements [4l, 4l + 4), non-temporal loads of g (fp16, 8 B),
// w (fp16, 8 B), m and v (fp32, 16 B each), then non-temporal stores of w, m
// and v -- the same seven streams, 12 bytes read and 10 written per element,
// in the same instructions.  Between the loads and the stores a chain of
// `spacing` dependent fp32 fma stands in for the element math; with k0 = 0,
// k1 = 1, k2 = 0 (kernel arguments, so the chain cannot be dropped) every
// stored value equals the loaded one.
__global__ __launch_bounds__(64) void stream_mix_kernel(uint16_t* __restrict__ w,
                                                        const uint16_t* __restrict__ g,
                                                        float* __restrict__ m,
                                                        float* __restrict__ v, uint32_t spacing,
                                                        float k0, float k1, float k2) {
  const uint64_t e = (uint64_t)blockIdx.x * 256u + threadIdx.x * 4u;
  const u32x2 gg = ldnt<u32x2>(g + e);
  u32x2 ww = ldnt<u32x2>(w + e);
  f32x4 mm = ldnt<f32x4>(m + e);
  f32x4 vv = ldnt<f32x4>(v + e);
  float acc = (float)((gg.x ^ gg.y) & 1u) + mm.x + vv.x + (float)(ww.x & 1u);
  for (uint32_t i = 0; i < spacing; ++i) acc = __builtin_fmaf(acc, k1, k2);
  const float z = acc * k0;  // 0 for finite acc
  ww.x += (uint32_t)z;
  mm.x += z;
  vv.x += z;
  stnt<u32x2>(w + e, ww);
  stnt<f32x4>(m + e, mm);
  stnt<f32x4>(v + e, vv);
}

uint32_t grid_for(uint64_t n) {
  uint64_t b = (n + 255) / 256;
  if (b > 65536) b = 65536;
  return (uint32_t)(b ? b : 1);
}

int status(hipError_t e) { return e == hipSuccess ? 0 : -2; }

// What a call is about to write may be an optimizer's gradient.
void written(const void* p, uint64_t bytes) { ark::opt_units_invalidate(&p, &bytes, 1); }

}  // namespace

extern "C" {

int ark_synth_normal_f16(uint16_t* out, uint64_t n, uint64_t seed,
                         uint32_t tensor_id, uint32_t step, float sigma_scale,
                         void* stream) {
  if (n == 0) return 0;
  if (!out) return -1;
  written(out, n * 2u);
  hipLaunchKernelGGL(normal_kernel<true>, dim3(grid_for(n)), dim3(256), 0,
                     (hipStream_t)stream, (void*)out, n,
                     synth_base(seed, tensor_id, step), sigma_scale);
  return status(hipGetLastError());
}

int ark_synth_normal_f32(float* out, uint64_t n, uint64_t seed,
                         uint32_t tensor_id, uint32_t step, float sigma_scale,
                         void* stream) {
  if (n == 0) return 0;
  if (!out) return -1;
  written(out, n * 4u);
  hipLaunchKernelGGL(normal_kernel<false>, dim3(grid_for(n)), dim3(256), 0,
                     (hipStream_t)stream, (void*)out, n,
                     synth_base(seed, tensor_id, step), sigma_scale);
  return status(hipGetLastError());
}

int ark_synth_copy(void* dst, const void* src, uint64_t nbytes, void* stream) {
  if (nbytes == 0) return 0;
  if (!dst || !src || (nbytes & 15u) || (((uintptr_t)dst | (uintptr_t)src) & 15u)) return -1;
  const uint64_t n = nbytes / 16u;
  const uint64_t blocks = (n + 255) / 256;
  if (blocks > 0xFFFFFFFFull / 256u) return -1;
  written(dst, nbytes);
  hipLaunchKernelGGL(copy_kernel, dim3((uint32_t)blocks), dim3(256), 0,
                     (hipStream_t)stream, (u32x4*)dst, (const u32x4*)src, n);
  return status(hipGetLastError());
}

int ark_synth_stream_mix(uint16_t* w, const uint16_t* g, float* m, float* v, uint64_t n,
                         uint32_t spacing, uint32_t blocks_per_cu, void* stream) {
  if (n == 0) return 0;
  if (!w || !g || !m || !v || (n % 256u) || blocks_per_cu > 32u ||
      (((uintptr_t)w | (uintptr_t)g | (uintptr_t)m | (uintptr_t)v) & 15u))
    return -1;
  const uint64_t rows = n / 256u;
  if (rows > 0x7FFFFFFFull / 64u) return -1;
  written(w, n * 2u);
  written(m, n * 4u);
  written(v, n * 4u);
  const uint32_t lds =
      ark::resident_lds_bytes((const void*)stream_mix_kernel, 64, (int)blocks_per_cu);
  hipLaunchKernelGGL(stream_mix_kernel, dim3((uint32_t)rows), dim3(64), lds, (hipStream_t)stream,
                     w, g, m, v, spacing, 0.0f, 1.0f, 0.0f);
  return status(hipGetLastError());
}

int ark_synth_fill_u16(uint16_t* out, uint64_t n, uint16_t bits, void* stream) {
  if (n == 0) return 0;
  if (!out) return -1;
  written(out, n * 2u);
  hipLaunchKernelGGL(fill_kernel, dim3(grid_for(n)), dim3(256), 0,
                     (hipStream_t)stream, out, n, bits);
  return status(hipGetLastError());
}

}  // extern "C"
