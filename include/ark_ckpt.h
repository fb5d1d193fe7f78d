/*
 * ark_ckpt.h -- ARK checkpoints (V4 "ARK4", and loading of V3 / V2) straight
 * from and to device-resident optimizer buffers on MI355X (gfx950).
 *
 * Replaces CheckpointV3::save_fp16 and CheckpointV3::load
 * (proyecto_ark/ark01/src/io.rs:432-500 and :504-671), called from
 * Trainer::guardar_checkpoint (src/training.rs:536-604) and the resume path
 * (training.rs:483-531, optimizer.rs:237-313).  File layout, little endian
 * (io.rs:12-24, :412-414):
 *
 *   V4: u32 magic 0x4B345241 ("ARK4"), u64 global_step, u64 adam_step,
 *       u64 n_tensors, then per tensor: u64 n, u64 type (0 = F16, 1 = F32),
 *       n * (2 or 4) bytes of data.  No padding anywhere.
 *   V3: magic 0x4B335241 ("ARK3"), u64 global_step, u64 adam_step,
 *       u64 n_tensors, per tensor u64 n + n fp32.
 *   V2: magic 0x4B325241 ("ARK2"), u64 global_step, u64 n_tensors, per
 *       tensor u64 n + n fp32 (weights only).
 *
 * The tensor order of save_fp16 (io.rs:473-494): embed w, m, v; per layer the
 * 9 weights (F16), the 9 m, the 9 v (F32); gamma_final w, m, v.  Here the
 * caller lists the records in file order, so any order of that format works.
 *
 * Extension: a file written with an AMP state carries a 40-byte trailer
 * after the last tensor -- u32 magic 0x53504D41 ("AMPS"), u32 version 1, the
 * 32-byte ark_opt_state -- which the reference's loader never reads (it stops
 * after n_tensors), so the file stays a valid V4 checkpoint for it.  The
 * reference drops the loss-scaler state on resume (training.rs:120-124).
 *
 * The device work: a pack kernel writes the whole file image (headers and
 * data, unaligned as the format is) into device memory in one launch, which
 * then streams to the file through pinned host buffers; loading streams the
 * file into a device image and an unpack kernel scatters (and converts) it
 * into the records.  Device memory used per call: the file size.
 *
 * Every function returns an ARK_OPT_* status code (include/ark_opt.h) with
 * the message in ark_opt_last_error().
 */
#ifndef ARK_CKPT_H
#define ARK_CKPT_H

#include <stdint.h>

#include "ark_opt.h"

#ifdef __cplusplus
extern "C" {
#endif

#define ARK_CKPT_F16 0u /* element type: fp16 bits (file type 0) */
#define ARK_CKPT_F32 1u /* element type: fp32 (file type 1) */

#define ARK_CKPT_MAGIC_V2 0x4B325241u
#define ARK_CKPT_MAGIC_V3 0x4B335241u
#define ARK_CKPT_MAGIC_V4 0x4B345241u
#define ARK_CKPT_MAGIC_AMP 0x53504D41u

/* One tensor of a checkpoint: n elements of dtype at data (a device
 * pointer).  Saving writes the record with file type = dtype.  Loading
 * converts from the file's type to dtype by the reference's own chain: an
 * F16 tensor is read as fp32 (half::f16::to_f32, memory.rs:111-113) and a
 * weight goes back to fp16 through ark_quant_f32_to_f16 (memory.rs:347-377),
 * so F16 -> F16 keeps every value and quiets signalling NaNs, F32 -> F16
 * rounds to nearest even, F16 -> F32 is exact, F32 -> F32 copies. */
typedef struct ark_ckpt_record {
  void *data;
  uint64_t n;
  uint32_t dtype;    /* ARK_CKPT_F16 or ARK_CKPT_F32 */
  uint32_t reserved; /* 0 */
} ark_ckpt_record;

typedef struct ark_ckpt_info {
  uint32_t version;     /* 2, 3 or 4 */
  uint32_t has_moments; /* tiene_momentos: 1 for V3 / V4, 0 for V2 */
  uint64_t global_step;
  uint64_t adam_step;   /* 0 for V2 (io.rs:657) */
  uint64_t n_tensors;
  uint64_t file_bytes;
  uint32_t has_amp;     /* the AMP trailer is present */
  uint32_t reserved;
} ark_ckpt_info;

/* CheckpointV3::save_fp16 (io.rs:432-500): writes the file as
 * "<target>.tmp.<pid>.<n>" (created exclusively, unique to the call) and
 * renames it over the target once complete, so a failed save leaves no
 * partial file and an existing file unchanged.  The target is path, or the
 * file a symbolic link at path names, followed link by link as open(2) does,
 * also when the link dangles (the link is kept and the file it names is
 * created, as File::create does; io.rs:450).  A new file gets mode 0666 less
 * the umask (File::create's); a file replaced hands its mode, and where
 * permitted its owner and group, on to the new file, as File::create keeps
 * them by truncating in place.  One difference remains: other hard links to
 * a replaced file keep naming the old contents, where File::create would
 * have rewritten the one file they share.  amp may be NULL (no trailer).
 * The records are read on the given stream; the call returns when the file
 * is written, flushed, closed and renamed. */
int ark_ckpt_save_v4(const char *path, uint64_t global_step, uint64_t adam_step,
                     const ark_ckpt_record *records, int32_t n_records,
                     const ark_opt_state *amp, void *stream);

/* Reads a checkpoint's header and tensor list without its data: info, and
 * for i < min(max, n_tensors) the element count n_out[i] and file type
 * type_out[i] (F32 for V2 / V3).  Either array may be NULL.  Fails like the
 * reference's loader on a bad magic (io.rs:665-668) or a truncated file. */
int ark_ckpt_probe(const char *path, ark_ckpt_info *info, uint64_t *n_out,
                   uint32_t *type_out, int32_t max);

/* CheckpointV3::load (io.rs:504-671) into device records: n_records must
 * equal the file's n_tensors and every record's n the file's n, and no two
 * records may share a byte (all are written by one launch).  amp (may be
 * NULL) receives the trailer's state when info->has_amp. */
int ark_ckpt_load(const char *path, const ark_ckpt_record *records, int32_t n_records,
                  ark_ckpt_info *info, ark_opt_state *amp, void *stream);

/* The device halves, for callers that move the bytes themselves and for
 * measurement.  ark_ckpt_v4_image_bytes: the V4 file size of the records
 * (with the 40-byte trailer if with_amp).  ark_ckpt_v4_pack: writes that
 * whole image into image (device memory, 16-byte aligned, at least that
 * many bytes): one kernel for the headers, one for the data.
 * ark_ckpt_v4_unpack: the inverse, from a V4 image in device memory laid out
 * as these records with the given file types would be; the file header and
 * every record header are checked on the device first.  Both return when
 * the stream has finished the work.  The image (image_bytes of it) may share
 * no byte with any record, and unpack's records none with each other; such
 * tables are refused with ARK_OPT_EINVAL before any device call. */
int ark_ckpt_v4_image_bytes(const ark_ckpt_record *records, int32_t n_records,
                            int with_amp, uint64_t *bytes);
int ark_ckpt_v4_pack(const ark_ckpt_record *records, int32_t n_records,
                     uint64_t global_step, uint64_t adam_step,
                     const ark_opt_state *amp, void *image, uint64_t image_bytes,
                     void *stream);
int ark_ckpt_v4_unpack(const void *image, uint64_t image_bytes,
                       const ark_ckpt_record *records, int32_t n_records,
                       const uint32_t *file_types, void *stream);

/* A pack prepared once for repeated saves of the same records into the same
 * device image: the trainer's checkpoint every N steps (training.rs:483-604,
 * CheckpointV3::save_fp16 at io.rs:432-502) kept in device memory, or staged
 * there for a copy that overlaps the next steps.  Create checks the
 * arguments as ark_ckpt_v4_pack does (with_amp: the image carries the
 * trailer) and uploads the record headers and data descriptors once.  Each
 * run queues the headers and the data on the plan's stream and returns
 * without waiting: the file header's steps and the trailer's state (amp,
 * required exactly when with_amp) are taken at the call, by value.  The
 * image is the same bytes ark_ckpt_v4_pack writes.  A run captured in a HIP
 * graph replays the steps and state it was captured with.  The records and
 * the image must stay allocated while runs are queued; destroy frees the
 * plan's device tables. */
typedef struct ark_ckpt_plan ark_ckpt_plan;

int ark_ckpt_v4_pack_plan_create(const ark_ckpt_record *records, int32_t n_records,
                                 int with_amp, void *image, uint64_t image_bytes,
                                 void *stream, ark_ckpt_plan **out);
int ark_ckpt_v4_pack_plan_run(ark_ckpt_plan *plan, uint64_t global_step,
                              uint64_t adam_step, const ark_opt_state *amp);
int ark_ckpt_plan_destroy(ark_ckpt_plan *plan);

#ifdef __cplusplus
}
#endif

#endif /* ARK_CKPT_H */
