/*
 * ark_oracle.h -- TEST INFRASTRUCTURE ONLY.  CPU restatement of the ARK
 * optimizer-step arithmetic, used as the parity checker by tests/, by
 * __graft_entry__.smoke() and by bench.py's cpu_baseline leg.  Nothing in the
 * product (ark_amd/) links, loads or calls it.
 *
 * Sources restated (paths relative to proyecto_ark/ark01/ of the reference):
 *   asm/opti.s:192-360     per-tensor AdamW, fp16 weights, fp32 g/m/v
 *   src/optimizer.rs:126-228   global clip + step_all order and per-tensor wd
 *   src/training.rs:10-13, 228-245, 289-326   AMP scaler state machine
 *   src/ffi.rs:138-158     vDSP_vsmul = one fp32 multiply per element
 *
 * The struct types are the ABI structs of include/ark_opt.h (types only).
 */
#ifndef ARK_ORACLE_H
#define ARK_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#include "../include/ark_opt.h"

#ifdef __cplusplus
extern "C" {
#endif

/* fp16 <-> fp32, software, IEEE binary16 with subnormals, RNE. */
float ark_ref_f16_to_f32(uint16_t h);
uint16_t ark_ref_f32_to_f16(float f);
void ark_ref_f16_to_f32_array(const uint16_t *in, float *out, uint64_t n);
void ark_ref_f32_to_f16_array(const float *in, uint16_t *out, uint64_t n);

/* Exhaustive cross-checks of the software conversions against the x86 F16C
 * hardware conversion (vcvtph2ps / vcvtps2ph in RNE).  Return the number of
 * mismatching bit patterns (NaN payloads included: F16C follows the same
 * quiet-and-keep-payload rule as fcvtl / fcvtn), or -1 without F16C.
 * f32->f16 covers the inputs [lo, hi) of the 2^32 bit patterns. */
int64_t ark_ref_check_f16_to_f32_f16c(void);
int64_t ark_ref_check_f32_to_f16_f16c(uint64_t lo, uint64_t hi, int nthreads);

/* got[i] against ark_ref_f32_to_f16 of the bit pattern lo + i for the patterns
 * [lo, hi): the number of mismatches; *first_bad = the first mismatching
 * pattern (UINT64_MAX if none).  Used to check a device conversion of every
 * fp32 pattern. */
int64_t ark_ref_compare_f32_to_f16_range(uint64_t lo, uint64_t hi, const uint16_t *got,
                                         int nthreads, uint64_t *first_bad);

/* beta^t by the binary exponentiation of opti.s:223-235 (t used as given). */
float ark_ref_pow_binary(float beta, uint32_t t);

/* Scalar prologue of opti.s:210-271. */
typedef struct ark_ref_scalars {
  float decay;  /* 1 - lr*wd            (opti.s:219-221) */
  float bc1;    /* 1 - beta1^t          (opti.s:223-237) */
  float bc2;    /* 1 - beta2^t          (opti.s:239-253) */
  float lr_eff; /* sqrt(bc2)/bc1 * lr   (opti.s:255-258) */
  float c1;     /* 1 - beta1            (opti.s:263-265) */
  float c2;     /* 1 - beta2            (opti.s:266-268) */
} ark_ref_scalars;
void ark_ref_prologue(float lr, float beta1, float beta2, float wd, uint32_t t,
                      ark_ref_scalars *out);

/* 1: the step's two loops (sum of squares, update) run 8-wide with AVX2/F16C
 * (for timing the CPU baseline; identical bits); 0 (default): the scalar
 * restatement.  Returns the mode in effect (0 without AVX2/F16C/FMA). */
int ark_ref_set_vector(int on);

/* Exact transliteration of ark_asm_adam_step (opti.s:20-177): fp32 weights,
 * the same prologue and element sequence without the fp16 conversions. */
void ark_ref_adam_step_f32(float *w, const float *g, float *m, float *v, uint64_t n,
                           float lr, float beta1, float beta2, float eps, float wd,
                           uint32_t t);

/* Exact transliteration of ark_asm_adam_step_f16 (opti.s:192-360). */
void ark_ref_adam_step_f16(uint16_t *w, const float *g, float *m, float *v,
                           uint64_t n, float lr, float beta1, float beta2,
                           float eps, float wd, uint32_t t);

/* Canonical f64 sum of squares of the unscaled gradients (see
 * ARK_OPT_NORM_SEGMENT) and the non-finite flag over a tensor table. */
double ark_ref_sumsq(const ark_opt_tensor *tab, int32_t nt, uint32_t grad_dtype,
                     float inv_scale, int nthreads, int32_t *nonfinite);

/* Pairwise (index-order binary tree) f64 sum of x[0..n) zero-padded to a
 * power of two. */
double ark_ref_pairwise(const double *x, uint64_t n);

/* Initial state for hparams (t 0, loss_scale_init, counters 0). */
void ark_ref_state_init(const ark_opt_hparams *hp, ark_opt_state *st);

/* One full fused step (training.rs:289-326 + optimizer.rs:171-228), in
 * place on the table's w/m/v, with the state machine on *st.  Same return
 * value and info as ark_opt_step.  nthreads >= 1. */
int ark_ref_opt_step(const ark_opt_tensor *tab, int32_t nt,
                     const ark_opt_hparams *hp, ark_opt_state *st, float lr,
                     int nthreads, ark_opt_step_info *info);

/* The scalar half of ark_ref_opt_step: given the step's canonical sum of
 * squares and non-finite flag (ark_ref_sumsq at inv_scale = 1/loss_scale of
 * the state on entry), the skip / clip / t / loss-scale decisions and the
 * step info, with the state machine on *st; no element is touched.
 * ark_ref_opt_step is ark_ref_sumsq + this + the element update. */
int ark_ref_finalize(const ark_opt_hparams *hp, ark_opt_state *st,
                     double sumsq, int nonfinite, float lr,
                     ark_opt_step_info *info);

/* Same as ark_ref_opt_step but with the global scalars taken from `given`
 * (applied, clipped, clip_coef, inv_scale, lr_eff from another
 * implementation's step info) instead of recomputed: the elementwise update
 * alone.  Used to check elements of a step whose scalars were checked
 * separately. */
int ark_ref_apply_given(const ark_opt_tensor *tab, int32_t nt,
                        const ark_opt_hparams *hp, uint32_t t, float lr,
                        const ark_opt_step_info *given, int nthreads);

/* The AMP state machine alone over a sequence of step outcomes: events[i]
 * nonzero = a non-finite step (skip), zero = an applied step.  Runs the same
 * bookkeeping code as ark_ref_opt_step; scale_out[i] (optional) receives the
 * loss scale after step i.  Returns the last step's status. */
int ark_ref_amp_replay(const ark_opt_hparams *hp, ark_opt_state *st,
                       const uint8_t *events, uint64_t n, float *scale_out);

/* training.rs:228-241: external skip. */
int ark_ref_record_overflow(const ark_opt_hparams *hp, ark_opt_state *st,
                            ark_opt_step_info *info);

/* ark_asm_grad_clip (opti.s:369-432) restated instruction by instruction:
 * four fused fp32 chains over the groups of four (lane l takes elements
 * 4k + l), the faddp pair sums (a0 + a1) + (a2 + a3), the remaining n % 4
 * values fused in order, fsqrt; when norm > thr (an unordered compare does
 * not clip) every value times thr / norm.  Returns the pre-clip norm. */
float ark_ref_grad_clip_literal(float *g, uint64_t n, float thr);

/* The build's definition of the same call (ark_hip_grad_clip): the norm is
 * sqrtf((float)sum) of the canonical f64 sum of squares of the one tensor
 * (ark_ref_sumsq, inf and NaN kept in the sum), then the same compare,
 * division and multiply as the literal form.  n = 0 gives 0. */
float ark_ref_grad_clip(float *g, uint64_t n, float thr, int nthreads);

/* Synthetic generator of include/ark_synth.h. */
uint64_t ark_ref_mix64(uint64_t z);
uint64_t ark_ref_splitmix64_next(uint64_t *state);
uint64_t ark_ref_synth_base(uint64_t seed, uint32_t tensor_id, uint32_t step);
void ark_ref_synth_normal_f32(float *out, uint64_t n, uint64_t seed,
                              uint32_t tensor_id, uint32_t step,
                              float sigma_scale);
void ark_ref_synth_normal_f16(uint16_t *out, uint64_t n, uint64_t seed,
                              uint32_t tensor_id, uint32_t step,
                              float sigma_scale);

/* ------------------------------------------------------------------------ */
/* Gradient hand-off (objc/bridge.m:902-948).                                */
/* ------------------------------------------------------------------------ */

/* dst[i] += src[i], i ascending (bridge.m:910-915, :931-947). */
void ark_ref_grad_accumulate(float *dst, const float *src, uint64_t n);

/* bridge.m:922-928, literally: for i < batch_seq, t = tokens[i] < vocab ?
 * tokens[i] : 0, then embed_grad[t*d + j] += dx0[i*d + j] for j < d. */
void ark_ref_embed_scatter(float *embed_grad, uint32_t vocab, uint32_t d,
                           const uint32_t *tokens, const float *dx0, uint32_t batch_seq);

#ifdef __cplusplus
}
#endif

#endif /* ARK_ORACLE_H */
