// ark_device.hpp -- device-side helpers shared by the gfx950 kernels: global
// (address space 1) loads and stores with and without the non-temporal hint,
// short vector types, and the fp16 <-> fp32 conversions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define ARK_GLOBAL __attribute__((address_space(1)))

namespace ark {
namespace dev {

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
// 16 bytes at a 4-byte-aligned address: the compiler emits one dwordx4
// access where the target allows dword alignment, as gfx950 does.
typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));

template <typename T>
__device__ __forceinline__ T ld_nt(const void* p) {
  return __builtin_nontemporal_load((const ARK_GLOBAL T*)p);
}
template <typename T>
__device__ __forceinline__ void st_nt(void* p, T v) {
  __builtin_nontemporal_store(v, (ARK_GLOBAL T*)p);
}
template <typename T>
__device__ __forceinline__ T ld_g(const void* p) {
  return *(const ARK_GLOBAL T*)p;
}
template <typename T>
__device__ __forceinline__ void st_g(void* p, T v) {
  *(ARK_GLOBAL T*)p = v;
}

// fp16 bits -> fp32, exact (v_cvt_f32_f16; denormals kept).
__device__ __forceinline__ float h2f(uint32_t b) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)b);
}

// fp32 -> fp16 bits, round to nearest even (v_cvt_f16_f32).  The empty asm
// makes f opaque, so preceding fp32 arithmetic can never be merged with the
// conversion into a single-rounding mixed-precision fma: a value computed in
// fp32 is rounded to fp32 first, then to fp16.
__device__ __forceinline__ uint32_t f2h(float f) {
  asm("" : "+v"(f));
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// The AArch64 conversions with the default FPCR (RNE, no flush, DN = 0) --
// fcvtl / fcvt s,h and fcvtn / fcvt h,s -- including their NaN rule: a NaN
// keeps its sign and the top payload bits and comes out quiet.  Non-NaN
// inputs take the hardware conversion, which rounds the same way.
__device__ __forceinline__ uint32_t f16_to_f32_bits(uint32_t h) {
  if ((h & 0x7C00u) == 0x7C00u && (h & 0x03FFu) != 0u)
    return ((h & 0x8000u) << 16) | 0x7FC00000u | ((h & 0x03FFu) << 13);
  return __float_as_uint(h2f(h));
}
__device__ __forceinline__ uint32_t f32_to_f16_bits(uint32_t x) {
  if ((x & 0x7F800000u) == 0x7F800000u && (x & 0x007FFFFFu) != 0u)
    return ((x >> 16) & 0x8000u) | 0x7E00u | ((x >> 13) & 0x03FFu);
  return f2h(__uint_as_float(x));
}

}  // namespace dev
}  // namespace ark
