/*
 * ark_grad.h -- the gradient hand-off into the optimizer step, on MI355X
 * (gfx950).
 *
 * Replaces the host tail of ark_mps_backward (proyecto_ark/ark01/objc/
 * bridge.m:902-948): after the backward pass the reference waits for the
 * device (:902-905) and then, on the CPU, adds every parameter-gradient
 * buffer into the Rust-side fp32 gradients (`+=`, :931-947), the LM-head
 * gradient into the tied embedding gradient (:910-911), gamma_final's
 * (:914-915), and scatter-adds each row of dL/d(embedding output) into the
 * embedding row of its token (:922-928).  Here the same sums run on the
 * device, stream ordered, with no host wait; the results are bit-identical
 * to those loops (fp32 adds in the same order), and the fp32 gradients they
 * produce go straight to ark_opt_step with ARK_OPT_GRAD_F32.
 *
 * Every function returns an ARK_OPT_* status code (include/ark_opt.h) with
 * the message in ark_opt_last_error().  Pointers are device pointers.
 */
#ifndef ARK_GRAD_H
#define ARK_GRAD_H

#include <stdint.h>

#include "ark_opt.h"

#ifdef __cplusplus
extern "C" {
#endif

/* dst[i] = dst[i] + src[i] for i < n (bridge.m:910-915, :931-947). */
typedef struct ark_grad_span {
  float *dst;
  const float *src;
  uint64_t n;
} ark_grad_span;

/* One span, one launch.  dst and src must not overlap. */
int ark_grad_accumulate(float *dst, const float *src, uint64_t n, void *stream);

/* Every span of a model in one launch; the plan copies the span table to
 * the device once.  No span's dst may share a byte with another span's dst
 * or with any span's src (srcs may overlap each other): such a table is
 * refused with ARK_OPT_EINVAL before any device call. */
typedef struct ark_grad_plan ark_grad_plan;
int ark_grad_plan_create(const ark_grad_span *spans, int32_t n_spans, void *stream,
                         ark_grad_plan **out);
int ark_grad_plan_run(ark_grad_plan *plan);
int ark_grad_plan_destroy(ark_grad_plan *plan);

/* bridge.m:922-928: for i in [0, batch_seq) in order, with
 * t = tokens[i] < vocab ? tokens[i] : 0,
 *     embed_grad[t*d + j] += dx0[i*d + j]   for j < d.
 * Every element receives its additions in increasing i, as in the loop: the
 * positions are stably sorted by token on the device, the dx0 rows copied in
 * that order, and each token's rows added in order, column by column.
 * embed_grad holds vocab*d floats, dx0 batch_seq*d, tokens batch_seq;
 * batch_seq < 2^24 (one 256-lane block per token), d <= 65535 * 256.
 * Stream ordered; the scratch it needs (a copy of dx0, 16 B per token and
 * the sort's) comes from the stream-ordered pool. */
int ark_grad_embed_scatter(float *embed_grad, uint32_t vocab, uint32_t d,
                           const uint32_t *tokens, const float *dx0, uint32_t batch_seq,
                           void *stream);

/* The step's norm without its read of the gradients.  The gradient an
 * optimizer step on fp32 gradients needs is produced here, so the kernels
 * that write its final values can also form the first level of the norm's
 * tree: one f64 per 256 consecutive elements of each ARK_OPT_NORM_SEGMENT
 * segment, the pairwise sum of the squared unscaled gradients (an aligned
 * subtree of the canonical tree of include/ark_opt.h, so the sum keeps its
 * bits).  The next ark_opt_step on that handle then reads these (8 B per 256
 * elements) instead of every gradient (4 B per element).  In the order of
 * bridge.m:907-948:
 *   ark_grad_plan_run_final(plan, opt);              every grad += output
 *   ark_grad_embed_scatter_final(..., opt);          the token scatter
 *   ark_opt_step(opt, lr, info);
 * Between the final calls and the step, a write to the handle's gradients
 * through any other call of this library (ark_grad_accumulate,
 * ark_grad_plan_run, ark_grad_embed_scatter, ark_grad_embed_scatter_noalloc,
 * the codec's dequantisation and plans, a checkpoint load or unpack, the
 * single-tensor Adam steps, the synthetic-input writers) discards the units;
 * a write the library does not see (the caller's own kernel or copy) must
 * not happen: the step would use the units of the old values.  ark_opt_set_state and ark_opt_record_overflow discard the units
 * (the loss scale changes), as does every ark_opt_step after using them; a
 * step without fresh units reads the gradients as usual. */

/* As ark_grad_plan_run, as the last accumulation before opt's next step:
 * also writes the norm's units of every span into opt.  opt must take fp32
 * gradients (ARK_OPT_GRAD_F32), the plan's spans with n > 0 must be, in
 * order, exactly the gradients of opt's tensors with n > 0, and the plan and
 * opt must share a stream; ARK_OPT_EINVAL otherwise, before anything is
 * queued. */
int ark_grad_plan_run_final(ark_grad_plan *plan, ark_opt_handle *opt);

/* As ark_grad_embed_scatter on opt's stream, after ark_grad_plan_run_final
 * (ARK_OPT_EINVAL otherwise): embed_grad must be the gradient of one of
 * opt's tensors with vocab * d elements, and the units of the embedding rows
 * the scatter changes are rewritten from their final values.  When d is not
 * a multiple of 256 the units cannot follow rows: the scatter is done (with
 * or without a final accumulation before it) and the next step reads the
 * gradients instead. */
int ark_grad_embed_scatter_final(float *embed_grad, uint32_t vocab, uint32_t d,
                                 const uint32_t *tokens, const float *dx0, uint32_t batch_seq,
                                 ark_opt_handle *opt);

/* Size of the device array behind ark_grad_embed_scatter_noalloc: 48 MiB.
 * The array is part of the library's code object, so every GPU the library is
 * used on holds one, from the library's first kernel launch or device set-up
 * there until the process ends, whether or not it calls this scatter. */
#define ARK_GRAD_SCRATCH_BYTES (48ull << 20)

/* ark_grad_embed_scatter with the same arguments and bit-identical results,
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  No
 * counterpart in the reference.  Its workspace is the static device array of
 * ARK_GRAD_SCRATCH_BYTES per GPU instead of the stream-ordered pool, so it
 * calls no hipMalloc, hipFree or other allocating routine.  The workspace is
 *   8 * batch_seq bytes, plus 8 * batch_seq + 1024 * ceil(batch_seq / 4096)
 *   more when batch_seq > 4096, plus 4 * batch_seq * d,
 * each part rounded up to 256 bytes (a 2 x 2048-token batch at d = 768
 * needs 12.6 MB, at d = 2048 33.6 MB); a larger one is rejected with
 * ARK_OPT_EINVAL before anything is queued.
 *
 * Set-up: once per GPU the library looks the array's address up and creates
 * one event; ark_opt_create and ark_grad_plan_create do this for their GPU,
 * and so does this call's first use on a GPU not yet set up.  That first use
 * must not come under graph capture: it then returns ARK_OPT_EINVAL before
 * anything is queued.
 *
 * Every call on a GPU shares that GPU's array, and each call writes every
 * workspace byte it reads, so nothing carries over from the previous call.
 * The library orders the calls on one GPU: a call outside graph capture, on
 * any stream and from any host thread, makes its stream wait
 * (hipStreamWaitEvent) for the work of the previous such call before it
 * touches the array.  A call made under graph capture becomes graph nodes
 * that this ordering does not cover: the caller orders each replay of that
 * graph against other uses of the array on the GPU (for instance by
 * replaying on the stream that makes the eager calls). */
int ark_grad_embed_scatter_noalloc(float *embed_grad, uint32_t vocab, uint32_t d,
                                   const uint32_t *tokens, const float *dx0, uint32_t batch_seq,
                                   void *stream);

#ifdef __cplusplus
}
#endif

#endif /* ARK_GRAD_H */
