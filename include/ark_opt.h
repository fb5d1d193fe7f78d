/*
 * ark_opt.h -- C ABI of the MI355X (gfx950) optimizer step for the ARK/EKO
 * training engine: AMP loss-scale unscale + inf/NaN skip, global L2 gradient
 * norm, global-norm clipping and the fused fp16-weight / fp32-moment AdamW
 * update, all as stream-ordered HIP kernels with no host round trip.
 *
 * Every entry point is plain C: device pointers, sizes, scalars and an opaque
 * stream (a hipStream_t passed as void*, NULL = the default stream).  All
 * functions return an int status (ARK_OPT_OK, ARK_OPT_EARLY_STOP or a negative
 * error code); nothing aborts.  ark_opt_last_error() gives the message of the
 * last failure on the calling thread.
 *
 * Reference interfaces this replaces (paths relative to proyecto_ark/ark01/):
 *   asm/opti.s:189-193           ark_asm_adam_step_f16 (per-tensor NEON kernel)
 *   src/optimizer.rs:44-76       AdamConfig / Optimizer { cfg, step }
 *   src/optimizer.rs:126-168     Optimizer::clip_all_grads (global L2 clip)
 *   src/optimizer.rs:171-228     Optimizer::step_all (272 per-tensor calls)
 *   src/optimizer.rs:237-313     Optimizer::restaurar_momentos (sets step)
 *   src/training.rs:10-13,54-59  AMP loss-scale constants and state
 *   src/training.rs:228-241      logits_grad non-finite skip
 *   src/training.rs:289-326      grad finite check, skip, unscale, step, growth
 */
#ifndef ARK_OPT_H
#define ARK_OPT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ARK_OPT_ABI_VERSION 1

/* ---- status codes ------------------------------------------------------ */
#define ARK_OPT_OK 0
/* More than max_consecutive_nonfinite skipped steps in a row; mirrors the
 * Err("early_stop_nan") of training.rs:235-237 and :298-301.  Sticky: every
 * later step is a no-op that reports it again. */
#define ARK_OPT_EARLY_STOP 1
#define ARK_OPT_EINVAL (-1) /* bad argument (null pointer, size, alignment) */
#define ARK_OPT_EHIP (-2)   /* a HIP runtime call failed */
#define ARK_OPT_ENOMEM (-3) /* device or pinned allocation failed */
#define ARK_OPT_EIO (-4)    /* a file could not be read or written, or is malformed */

/* ---- norm definition --------------------------------------------------- */
/* The global sum of squares is a pairwise (index-order binary tree) f64 sum
 * over the concatenation of every tensor's squared unscaled gradients, each
 * tensor zero-padded to a multiple of ARK_OPT_NORM_SEGMENT elements and the
 * whole zero-padded to a power of two.  Any chip, grid or thread count gives
 * the same bits. */
#define ARK_OPT_NORM_SEGMENT 4096

/* ---- gradient storage -------------------------------------------------- */
#define ARK_OPT_GRAD_F16 0u /* fp16 bits, already multiplied by the loss scale */
#define ARK_OPT_GRAD_F32 1u /* fp32, already multiplied by the loss scale      */

/* ---- per-tensor flags -------------------------------------------------- */
/* Leave this tensor's gradient scaled (no multiply by 1/loss_scale).  The
 * reference's scale_grads (training.rs:133-146) skips gamma_final; set this
 * flag on that tensor to reproduce it bit for bit.  Default: unscale all. */
#define ARK_OPT_TENSOR_NO_UNSCALE 1u

/* One parameter tensor: the fp16 weight with its gradient and fp32 moments
 * (memory.rs:202-255: *_fp16 pointer + grad/m/v Tensor).  All pointers are
 * device memory owned by the caller; the library never frees or reallocates
 * them.  16-byte aligned pointers take the 128-bit vector path; any other
 * alignment is accepted and runs element by element. */
typedef struct ark_opt_tensor {
  uint16_t *w;        /* fp16 weights, updated in place                    */
  const void *g;      /* gradients, ark_opt_hparams.grad_dtype, read only  */
  float *m;           /* first moment, updated in place                    */
  float *v;           /* second moment, updated in place                   */
  uint64_t n;         /* elements (0 allowed: the tensor is ignored)        */
  float weight_decay; /* decoupled wd of this tensor (optimizer.rs:194-226) */
  uint32_t flags;     /* ARK_OPT_TENSOR_*                                   */
} ark_opt_tensor;

/* Hyper-parameters fixed for the life of a handle.  AdamConfig fields
 * (optimizer.rs:44-52) except lr, which is a per-step argument, and
 * weight_decay, which is per tensor; the AMP scaler constants of
 * training.rs:10-13 and config.rs:36. */
typedef struct ark_opt_hparams {
  float beta1;                        /* optimizer.rs:47                      */
  float beta2;                        /* optimizer.rs:48                      */
  float eps;                          /* optimizer.rs:49                      */
  float grad_clip;                    /* optimizer.rs:50; > 0 (config.rs:136-138),
                                         INFINITY never clips */
  float loss_scale_init;              /* training.rs:10 LOSS_SCALE_INIT       */
  float loss_scale_min;               /* training.rs:12 LOSS_SCALE_MIN        */
  float loss_scale_max;               /* config.rs:36 loss_scale_max          */
  uint32_t scale_up_every;            /* training.rs:13 SCALE_UP_EVERY        */
  uint32_t max_consecutive_nonfinite; /* training.rs:235 and :298 (200)       */
  uint32_t grad_dtype;                /* ARK_OPT_GRAD_*                       */
} ark_opt_hparams;

/* Device-resident optimizer + AMP state (Optimizer::step, optimizer.rs:70;
 * Trainer fields training.rs:54-59).  Read/written with get/set_state. */
typedef struct ark_opt_state {
  uint32_t t;                     /* applied AdamW steps ("adam_step")    */
  float loss_scale;               /* current dynamic loss scale            */
  uint32_t clean_steps;           /* applied steps since the last change   */
  uint32_t consecutive_nonfinite; /* skipped steps in a row                */
  uint64_t skipped_steps;         /* total skipped steps                   */
  uint32_t early_stop;            /* 1 once the early-stop limit was hit   */
  uint32_t reserved;
} ark_opt_state;

/* What one step did.  Filled only when a non-NULL pointer is passed, which
 * makes the call wait for the step to finish. */
typedef struct ark_opt_step_info {
  int32_t applied;    /* 1: AdamW ran; 0: skipped (non-finite or early stop) */
  int32_t nonfinite;  /* a gradient held inf or NaN                           */
  int32_t clipped;    /* norm > grad_clip && norm > 0 (optimizer.rs:148)      */
  int32_t status;     /* ARK_OPT_OK or ARK_OPT_EARLY_STOP                     */
  double grad_sumsq;  /* f64 sum of squares of the unscaled gradients (NaN
                         when a gradient is non-finite)                       */
  float grad_norm;    /* sqrtf((float)grad_sumsq): pre-clip norm              */
  float clip_coef;    /* grad_clip / grad_norm when clipped, else 1.0         */
  float inv_scale;    /* 1.0f / loss_scale used to unscale this step          */
  float lr;           /* learning rate passed to this step                    */
  float lr_eff;       /* (sqrtf(bc2) / bc1) * lr (opti.s:255-258)             */
  float reserved;
  ark_opt_state state; /* state after the step                                */
} ark_opt_step_info;

/* Per-kernel device time accumulated while timing is enabled. */
typedef struct ark_opt_timing {
  uint64_t steps;     /* steps timed                                   */
  double ms_norm;     /* total ms in the sum-of-squares / finite kernel */
  double ms_finalize; /* total ms in the scalar finalize kernel         */
  double ms_adamw;    /* total ms in the fused AdamW kernel             */
  double ms_step;     /* total ms from the first to the last kernel     */
} ark_opt_timing;

typedef struct ark_opt_handle ark_opt_handle;

/* Library ABI version (ARK_OPT_ABI_VERSION).  No reference counterpart. */
int ark_opt_abi_version(void);

/* Message of the last failing call on this thread ("" if none). */
const char *ark_opt_last_error(void);

/* sizeof of each public struct, in the order tensor, hparams, state,
 * step_info, timing, then ark_codec_span, ark_ckpt_record, ark_ckpt_info,
 * ark_grad_span (include/ark_codec.h, ark_ckpt.h, ark_grad.h); lets a
 * binding check its layouts.  Returns the count written (at most n). */
int ark_opt_struct_sizes(size_t *out, int n);

/* Defaults: AdamConfig::default (optimizer.rs:54-66: beta1 0.9, beta2 0.999,
 * eps 1e-8, grad_clip 1.0), LOSS_SCALE_INIT 256, LOSS_SCALE_MIN 1,
 * SCALE_UP_EVERY 2000 (training.rs:10-13), loss_scale_max 8192
 * (config.rs:69), early stop after 200 (training.rs:235), fp16 gradients. */
int ark_opt_default_hparams(ark_opt_hparams *out);

/* Optimizer::new (optimizer.rs:74) over a parameter-buffer set.  Copies the
 * table and its segment map to the device, allocates the workspace and the
 * device state (t = 0, loss_scale = loss_scale_init), and binds the handle to
 * `stream` on the current device (a stream of another device is refused with
 * ARK_OPT_EINVAL; so are the plans' creates below).  One handle per stream;
 * not thread safe.
 * The buffers the step writes (every tensor's w, m and v) must be pairwise
 * disjoint and disjoint from every g, as the reference's distinct per-tensor
 * fields are (memory.rs:202-255); a table that lists a tensor twice or
 * overlaps them is refused with ARK_OPT_EINVAL.  Gradients may overlap each
 * other (they are only read). */
int ark_opt_create(const ark_opt_tensor *tensors, int32_t n_tensors,
                   const ark_opt_hparams *hp, void *stream,
                   ark_opt_handle **out);

int ark_opt_destroy(ark_opt_handle *h);

/* One optimizer step over every tensor: the grad finite check, skip or
 * unscale, global norm, clip, AdamW with bias correction, and the loss-scale
 * update of training.rs:289-326 with Optimizer::step_all
 * (optimizer.rs:171-228).  Stream ordered; with info == NULL nothing waits
 * on the host.  `lr` is this step's learning rate (Optimizer::lr_now,
 * optimizer.rs:80-92, evaluated by the caller).  It travels as a kernel
 * argument: a HIP graph that captured a step replays the lr it was captured
 * with (t, the bias corrections and the AMP state still advance on the
 * device), so a schedule that changes lr needs a graph per lr value, a
 * fresh capture, or ark_opt_step_lr_dev.  The step's norm pass reads the
 * gradients, or the units the hand-off's final calls wrote
 * (include/ark_grad.h) when they are fresh; a capture keeps the choice it
 * saw, so capture the step together with the final calls that feed it, or
 * with neither. */
int ark_opt_step(ark_opt_handle *h, float lr, ark_opt_step_info *info);

/* ark_opt_step with this step's learning rate read from the device scalar
 * *lr_dev when the step's finalize kernel runs, instead of a host value.  No
 * counterpart in the reference (its lr is a host value, Optimizer::lr_now,
 * optimizer.rs:80-92); for steps replayed from a HIP graph: a captured call
 * reads the scalar on every replay, so writing this step's lr into it
 * (stream ordered before the replay) makes replays follow a schedule.  A
 * non-finite value makes the step a no-op (state and buffers unchanged)
 * whose info reports ARK_OPT_EINVAL, the status this call then returns when
 * info is not NULL. */
int ark_opt_step_lr_dev(ark_opt_handle *h, const float *lr_dev, ark_opt_step_info *info);

/* The external skip path of training.rs:228-241: the caller found a
 * non-finite value upstream (the logits gradient) and drops this step.
 * Halves the scale, counts the skip, may trigger the early stop.  Gradients
 * and parameters are not touched. */
int ark_opt_record_overflow(ark_opt_handle *h, ark_opt_step_info *info);

/* Read / overwrite the device state (waits for the stream).  set_state is
 * the step-restoring half of restaurar_momentos (optimizer.rs:308); the
 * moments themselves live in the caller's m/v buffers. */
int ark_opt_get_state(ark_opt_handle *h, ark_opt_state *out);
int ark_opt_set_state(ark_opt_handle *h, const ark_opt_state *st);

/* Per-kernel timing with HIP events on the handle's stream.  No reference
 * counterpart (the reference never times its optimizer step). */
int ark_opt_set_timing(ark_opt_handle *h, int enable);
int ark_opt_get_timing(ark_opt_handle *h, ark_opt_timing *out);

/* Drop-in for one call of ark_asm_adam_step (opti.s:20-177, declared at
 * ffi.rs:98-101), the reference's fp32-weight kernel (unused by its trainer):
 * the same arguments in the same order plus the stream, fp32 weights and
 * gradients used as given, t == 0 treated as 1.  One wave per 256-element
 * row, the element sequence of ark_hip_adam_step_f16 without the fp16
 * conversions; w, m, v and g must not share a byte. */
int ark_hip_adam_step(float *w, const float *g, float *m, float *v, uint64_t n, float lr,
                      float beta1, float beta2, float eps, float wd, uint32_t t, void *stream);

/* Drop-in for ark_asm_grad_clip (opti.s:369-432, declared at ffi.rs:111-115,
 * wrapped by grad_clip_global at ffi.rs:206-213), the reference's per-tensor
 * clip (unused by its trainer): the L2 norm of the n fp32 values at grads,
 * and, when norm > threshold, every value multiplied in place by
 * threshold / norm (one fp32 division, one fp32 multiply per value).  The
 * norm is the canonical f64 sum of squares of this header (the tensor taken
 * alone, without unscaling), rounded to fp32 and square-rooted in fp32:
 * within 1e-7 relative of the exact norm where the reference's four
 * sequential fp32 chains drift by ~4e-3 at 24.6M values (N(0, 1e-3) data).  An inf value
 * makes the norm inf (clipping with coefficient 0) and a NaN makes it NaN
 * (no clipping), as in the reference; the compare is its fcmp / b.le, so an
 * unordered one does not clip and n = 0 gives norm 0.
 * norm_out: a host pointer that receives the pre-clip norm (opti.s:423); the
 * call then waits for the stream, as the reference returns it.  NULL: the
 * work is only queued.  Workspace (8 bytes per 8192 values, at most
 * ~4.2 MB) comes from the stream-ordered pool; n <= 2^32. */
int ark_hip_grad_clip(float *grads, uint64_t n, float threshold, float *norm_out, void *stream);

/* Drop-in for one call of ark_asm_adam_step_f16 (opti.s:189-193, declared
 * at optimizer.rs:20-23 and ffi.rs:105-108): same arguments in the same
 * order, fp32 gradients used as given (no unscale, no clip), t == 0 treated
 * as 1, plus the stream.  Runs the same per-row AdamW code as ark_opt_step
 * over the one tensor, with the step scalars passed as kernel arguments
 * (no table upload, nothing allocated); returns once the work is queued.
 * w, m, v and g must not share a byte (ARK_OPT_EINVAL otherwise). */
int ark_hip_adam_step_f16(uint16_t *w, const float *g, float *m, float *v,
                          uint64_t n, float lr, float beta1, float beta2,
                          float eps, float wd, uint32_t t, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* ARK_OPT_H */
