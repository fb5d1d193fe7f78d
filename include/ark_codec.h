/*
 * ark_codec.h -- fp16 <-> fp32 weight codec on MI355X (gfx950).
 *
 * Replaces the reference's NEON conversion kernels
 *   ark_dequant_f16_to_f32  (proyecto_ark/ark01/asm/kern.s:826-869; Rust
 *                            declaration src/ffi.rs:90-92)
 *   ark_quant_f32_to_f16    (asm/kern.s:872-913; src/ffi.rs:87-88)
 * and their loops over the model's tensors: the per-step dequantisation of
 * every weight (src/training.rs:162-186) and sync_weights_to_gpu
 * (src/memory.rs:347-377).
 *
 * Conversion rule, bit for bit that of fcvtl / fcvtn under AArch64's default
 * FPCR (round to nearest even, no flush to zero, DN = 0):
 *   f16 -> f32: exact; a NaN keeps its sign and payload (shifted up 13 bits)
 *               and comes out quiet.
 *   f32 -> f16: round to nearest even; subnormal results kept; overflow to
 *               +-inf; a NaN keeps its sign and the top 10 payload bits and
 *               comes out quiet.
 *
 * All pointers are device pointers (or host memory mapped for the device);
 * every call is stream ordered and returns an ARK_OPT_* status code
 * (include/ark_opt.h), with the message in ark_opt_last_error().
 */
#ifndef ARK_CODEC_H
#define ARK_CODEC_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ARK_CODEC_F16_TO_F32 0u /* dequantise: src uint16 bits, dst float */
#define ARK_CODEC_F32_TO_F16 1u /* quantise:   src float, dst uint16 bits */

/* Drop-in of ark_dequant_f16_to_f32(src, dst, n) (kern.s:826-869) plus a
 * stream.  src and dst must not overlap. */
int ark_hip_dequant_f16_to_f32(const uint16_t *src, float *dst, uint64_t n,
                               void *stream);

/* Drop-in of ark_quant_f32_to_f16(src, dst, n) (kern.s:872-913) plus a
 * stream.  src and dst must not overlap. */
int ark_hip_quant_f32_to_f16(const float *src, uint16_t *dst, uint64_t n,
                             void *stream);

/* A batch of conversions run as one launch: the per-tensor loops of
 * training.rs:166-186 (dequantise every weight) and memory.rs:347-377
 * (sync_weights_to_gpu, quantise every weight).  The plan copies the span
 * table to the device once; each run converts every span.  No span's dst
 * may share a byte with another span's dst or with any span's src (srcs may
 * overlap each other): such a table is refused with ARK_OPT_EINVAL before
 * any device call. */
typedef struct ark_codec_span {
  const void *src; /* direction's source type, n elements */
  void *dst;       /* direction's destination type, n elements */
  uint64_t n;
} ark_codec_span;

typedef struct ark_codec_plan ark_codec_plan;

int ark_codec_plan_create(const ark_codec_span *spans, int32_t n_spans,
                          uint32_t direction, void *stream,
                          ark_codec_plan **out);
/* Queues one conversion of every span on the plan's stream. */
int ark_codec_plan_run(ark_codec_plan *plan);
int ark_codec_plan_destroy(ark_codec_plan *plan);

#ifdef __cplusplus
}
#endif

#endif /* ARK_CODEC_H */
