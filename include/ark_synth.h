/*
 * ark_synth.h -- seeded synthetic inputs on the device, for the parity tests
 * and the benchmark.  No counterpart in the reference: it trains on a real
 * corpus, while the optimizer-step benchmarks use seeded fp16 weights and
 * gradients of the EKO shapes.
 *
 * The generator is counter based and uses only integer arithmetic plus
 * correctly rounded fp32 operations, so a CPU restatement reproduces every
 * output bit exactly:
 *
 *   base  = mix64(seed + GOLDEN * (1 + ((uint64)tensor_id << 32 | step)))
 *   x_i   = mix64(base + GOLDEN * (i + 1))          (SplitMix64 stream)
 *   d_i   = 2 * (u0 + u1 + u2 + u3) - 262140        (u_k = 16-bit fields of x_i,
 *                                                    low field first; int32)
 *   z_i   = (float)d_i * K                          (K = 0x1.bb67aep-17f,
 *                                                    sqrt(3)/131072 in fp32)
 *   out_i = fp16_rne(z_i * sigma_scale)
 *
 * where mix64 is the SplitMix64 finaliser (constants 0xbf58476d1ce4e5b9,
 * 0x94d049bb133111eb; shifts 30, 27, 31) and GOLDEN = 0x9e3779b97f4a7c15.
 * z is an Irwin-Hall(4) approximation of N(0,1): mean 0, variance 1 (up to
 * 2^-32), support |z| <= sqrt(12).
 */
#ifndef ARK_SYNTH_H
#define ARK_SYNTH_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* out[i] = fp16 bits of N(0,1)-like draws times sigma_scale (for gradients,
 * sigma * loss_scale).  Stream ordered. */
int ark_synth_normal_f16(uint16_t *out, uint64_t n, uint64_t seed,
                         uint32_t tensor_id, uint32_t step, float sigma_scale,
                         void *stream);

/* out[i] = the fp32 value z_i * sigma_scale (no fp16 rounding). */
int ark_synth_normal_f32(float *out, uint64_t n, uint64_t seed,
                         uint32_t tensor_id, uint32_t step, float sigma_scale,
                         void *stream);

/* out[i] = bits for all i (e.g. 0x3C00 = 1.0 for RMSNorm gains). */
int ark_synth_fill_u16(uint16_t *out, uint64_t n, uint16_t bits, void *stream);

/* Plain device copy of nbytes (a multiple of 16; both pointers 16-byte
 * aligned) with one 16-byte non-temporal load and store per thread, the
 * access kind of the optimizer kernels.  Reads and writes exactly nbytes:
 * the reference point that calibrates byte counters (FETCH_SIZE /
 * WRITE_SIZE) in profiles. */
int ark_synth_copy(void *dst, const void *src, uint64_t nbytes, void *stream);

/* The optimizer's AdamW pass without its arithmetic: one wave per
 * 256-element row reads g (fp16), w (fp16), m and v (fp32) and writes w, m
 * and v back unchanged, with the same instructions and cache hints, and a
 * chain of `spacing` dependent fp32 fma between the loads and the stores in
 * place of the element math.  22 bytes per element, the pass's stream mix:
 * the measured ceiling for that access pattern.  blocks_per_cu (at most 32)
 * caps the one-wave blocks resident per CU with a dynamic-LDS reservation, as
 * the optimizer holds its AdamW pass; 0 leaves every wave slot open.  n a
 * multiple of 256, every pointer 16-byte aligned; returns -1 otherwise. */
int ark_synth_stream_mix(uint16_t *w, const uint16_t *g, float *m, float *v, uint64_t n,
                         uint32_t spacing, uint32_t blocks_per_cu, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* ARK_SYNTH_H */
