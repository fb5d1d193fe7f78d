//! Raw FFI to libark_opt.so, the MI355X (gfx950) optimizer step of ARK and the
//! paths on either side of it.  One item per declaration of `include/*.h`,
//! same names, same field order (`#[repr(C)]`), same argument order; the
//! C headers document each call.  Every function returns an `ARK_OPT_*`
//! status (`ark_synth_*`: 0 or -1) with the message in `ark_opt_last_error()`.
//! All buffer pointers are device pointers; `stream` is a `hipStream_t`.
//!
//! Replaces the extern block of `src/optimizer.rs:15-24` (and the kernel
//! declarations of `src/ffi.rs:87-116`) in the reference.  The repository's
//! `tests/test_c_abi.py` checks every struct layout, function and constant
//! here against the C headers.
#![allow(non_camel_case_types)]
#![no_std]

use core::ffi::{c_char, c_int, c_void};

// ---- include/ark_opt.h -------------------------------------------------------

pub const ARK_OPT_ABI_VERSION: c_int = 1;
pub const ARK_OPT_OK: c_int = 0;
pub const ARK_OPT_EARLY_STOP: c_int = 1;
pub const ARK_OPT_EINVAL: c_int = -1;
pub const ARK_OPT_EHIP: c_int = -2;
pub const ARK_OPT_ENOMEM: c_int = -3;
pub const ARK_OPT_EIO: c_int = -4;
pub const ARK_OPT_NORM_SEGMENT: u32 = 4096;
pub const ARK_OPT_GRAD_F16: u32 = 0;
pub const ARK_OPT_GRAD_F32: u32 = 1;
pub const ARK_OPT_TENSOR_NO_UNSCALE: u32 = 1;

/// One parameter tensor: the fp16 weight with its gradient and fp32 moments
/// (`src/memory.rs:202-255`).
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct ark_opt_tensor {
    pub w: *mut u16,
    pub g: *const c_void,
    pub m: *mut f32,
    pub v: *mut f32,
    pub n: u64,
    pub weight_decay: f32,
    pub flags: u32,
}

/// `AdamConfig` (`src/optimizer.rs:44-66`) plus the AMP scaler constants
/// (`src/training.rs:10-13`, `src/config.rs:36,69`).
#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct ark_opt_hparams {
    pub beta1: f32,
    pub beta2: f32,
    pub eps: f32,
    pub grad_clip: f32,
    pub loss_scale_init: f32,
    pub loss_scale_min: f32,
    pub loss_scale_max: f32,
    pub scale_up_every: u32,
    pub max_consecutive_nonfinite: u32,
    pub grad_dtype: u32,
}

/// `Optimizer::step` and the trainer's AMP counters (`src/training.rs:54-59`).
#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct ark_opt_state {
    pub t: u32,
    pub loss_scale: f32,
    pub clean_steps: u32,
    pub consecutive_nonfinite: u32,
    pub skipped_steps: u64,
    pub early_stop: u32,
    pub reserved: u32,
}

#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct ark_opt_step_info {
    pub applied: i32,
    pub nonfinite: i32,
    pub clipped: i32,
    pub status: i32,
    pub grad_sumsq: f64,
    pub grad_norm: f32,
    pub clip_coef: f32,
    pub inv_scale: f32,
    pub lr: f32,
    pub lr_eff: f32,
    pub reserved: f32,
    pub state: ark_opt_state,
}

#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct ark_opt_timing {
    pub steps: u64,
    pub ms_norm: f64,
    pub ms_finalize: f64,
    pub ms_adamw: f64,
    pub ms_step: f64,
}

/// Opaque optimizer handle.
#[repr(C)]
pub struct ark_opt_handle {
    _private: [u8; 0],
}

extern "C" {
    pub fn ark_opt_abi_version() -> c_int;
    pub fn ark_opt_last_error() -> *const c_char;
    pub fn ark_opt_struct_sizes(out: *mut usize, n: c_int) -> c_int;
    pub fn ark_opt_default_hparams(out: *mut ark_opt_hparams) -> c_int;
    /// `Optimizer::new` (`src/optimizer.rs:74`) over a tensor table.
    pub fn ark_opt_create(tensors: *const ark_opt_tensor, n_tensors: i32,
                          hp: *const ark_opt_hparams, stream: *mut c_void,
                          out: *mut *mut ark_opt_handle) -> c_int;
    pub fn ark_opt_destroy(h: *mut ark_opt_handle) -> c_int;
    /// `Optimizer::step_all` (`src/optimizer.rs:171-228`) with the AMP block of
    /// `Trainer::train_step` (`src/training.rs:289-326`).
    pub fn ark_opt_step(h: *mut ark_opt_handle, lr: f32, info: *mut ark_opt_step_info) -> c_int;
    /// No reference counterpart: the step with lr read from a device scalar
    /// (HIP graph replays that follow a schedule).
    pub fn ark_opt_step_lr_dev(h: *mut ark_opt_handle, lr_dev: *const f32,
                               info: *mut ark_opt_step_info) -> c_int;
    /// The logits-gradient skip (`src/training.rs:228-241`).
    pub fn ark_opt_record_overflow(h: *mut ark_opt_handle, info: *mut ark_opt_step_info) -> c_int;
    pub fn ark_opt_get_state(h: *mut ark_opt_handle, out: *mut ark_opt_state) -> c_int;
    pub fn ark_opt_set_state(h: *mut ark_opt_handle, st: *const ark_opt_state) -> c_int;
    pub fn ark_opt_set_timing(h: *mut ark_opt_handle, enable: c_int) -> c_int;
    pub fn ark_opt_get_timing(h: *mut ark_opt_handle, out: *mut ark_opt_timing) -> c_int;
    /// `ark_asm_adam_step` (`asm/opti.s:20-177`, `src/ffi.rs:98-101`), fp32
    /// weights, plus a stream.
    pub fn ark_hip_adam_step(w: *mut f32, g: *const f32, m: *mut f32, v: *mut f32, n: u64,
                             lr: f32, beta1: f32, beta2: f32, eps: f32, wd: f32, t: u32,
                             stream: *mut c_void) -> c_int;
    /// `ark_asm_grad_clip` (`asm/opti.s:369-432`, `src/ffi.rs:111-115`): the
    /// pre-clip norm into `*norm_out` (a host pointer; the call then waits for
    /// the stream), grads scaled in place by threshold / norm when it clips.
    pub fn ark_hip_grad_clip(grads: *mut f32, n: u64, threshold: f32, norm_out: *mut f32,
                             stream: *mut c_void) -> c_int;
    /// `ark_asm_adam_step_f16` (`asm/opti.s:189-193`, `src/optimizer.rs:20-23`)
    /// plus a stream.
    pub fn ark_hip_adam_step_f16(w: *mut u16, g: *const f32, m: *mut f32, v: *mut f32, n: u64,
                                 lr: f32, beta1: f32, beta2: f32, eps: f32, wd: f32, t: u32,
                                 stream: *mut c_void) -> c_int;
}

// ---- include/ark_codec.h -----------------------------------------------------

pub const ARK_CODEC_F16_TO_F32: u32 = 0;
pub const ARK_CODEC_F32_TO_F16: u32 = 1;

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct ark_codec_span {
    pub src: *const c_void,
    pub dst: *mut c_void,
    pub n: u64,
}

/// Opaque codec plan.
#[repr(C)]
pub struct ark_codec_plan {
    _private: [u8; 0],
}

extern "C" {
    /// `ark_dequant_f16_to_f32` / `ark_quant_f32_to_f16` (`src/ffi.rs:87-92`,
    /// `asm/kern.s:826-913`) plus a stream.
    pub fn ark_hip_dequant_f16_to_f32(src: *const u16, dst: *mut f32, n: u64,
                                      stream: *mut c_void) -> c_int;
    pub fn ark_hip_quant_f32_to_f16(src: *const f32, dst: *mut u16, n: u64,
                                    stream: *mut c_void) -> c_int;
    /// Every tensor's conversion in one launch (`src/training.rs:162-186`,
    /// `src/memory.rs:347-377`).
    pub fn ark_codec_plan_create(spans: *const ark_codec_span, n_spans: i32, direction: u32,
                                 stream: *mut c_void, out: *mut *mut ark_codec_plan) -> c_int;
    pub fn ark_codec_plan_run(plan: *mut ark_codec_plan) -> c_int;
    pub fn ark_codec_plan_destroy(plan: *mut ark_codec_plan) -> c_int;
}

// ---- include/ark_ckpt.h ------------------------------------------------------

pub const ARK_CKPT_F16: u32 = 0;
pub const ARK_CKPT_F32: u32 = 1;
pub const ARK_CKPT_MAGIC_V2: u32 = 0x4B32_5241;
pub const ARK_CKPT_MAGIC_V3: u32 = 0x4B33_5241;
pub const ARK_CKPT_MAGIC_V4: u32 = 0x4B34_5241;
pub const ARK_CKPT_MAGIC_AMP: u32 = 0x5350_4D41;

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct ark_ckpt_record {
    pub data: *mut c_void,
    pub n: u64,
    pub dtype: u32,
    pub reserved: u32,
}

#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct ark_ckpt_info {
    pub version: u32,
    pub has_moments: u32,
    pub global_step: u64,
    pub adam_step: u64,
    pub n_tensors: u64,
    pub file_bytes: u64,
    pub has_amp: u32,
    pub reserved: u32,
}

extern "C" {
    /// `CheckpointV3::save_fp16` (`src/io.rs:432-500`) from device buffers.
    pub fn ark_ckpt_save_v4(path: *const c_char, global_step: u64, adam_step: u64,
                            records: *const ark_ckpt_record, n_records: i32,
                            amp: *const ark_opt_state, stream: *mut c_void) -> c_int;
    pub fn ark_ckpt_probe(path: *const c_char, info: *mut ark_ckpt_info, n_out: *mut u64,
                          type_out: *mut u32, max: i32) -> c_int;
    /// `CheckpointV3::load` (`src/io.rs:504-671`) into device buffers.
    pub fn ark_ckpt_load(path: *const c_char, records: *const ark_ckpt_record, n_records: i32,
                         info: *mut ark_ckpt_info, amp: *mut ark_opt_state,
                         stream: *mut c_void) -> c_int;
    pub fn ark_ckpt_v4_image_bytes(records: *const ark_ckpt_record, n_records: i32,
                                   with_amp: c_int, bytes: *mut u64) -> c_int;
    pub fn ark_ckpt_v4_pack(records: *const ark_ckpt_record, n_records: i32, global_step: u64,
                            adam_step: u64, amp: *const ark_opt_state, image: *mut c_void,
                            image_bytes: u64, stream: *mut c_void) -> c_int;
    pub fn ark_ckpt_v4_unpack(image: *const c_void, image_bytes: u64,
                              records: *const ark_ckpt_record, n_records: i32,
                              file_types: *const u32, stream: *mut c_void) -> c_int;
    /// A pack prepared once for repeated saves of the same records into the
    /// same device image (the trainer's periodic checkpoint,
    /// `src/training.rs:483-604`); each run is queued without waiting.
    pub fn ark_ckpt_v4_pack_plan_create(records: *const ark_ckpt_record, n_records: i32,
                                        with_amp: c_int, image: *mut c_void, image_bytes: u64,
                                        stream: *mut c_void,
                                        out: *mut *mut ark_ckpt_plan) -> c_int;
    pub fn ark_ckpt_v4_pack_plan_run(plan: *mut ark_ckpt_plan, global_step: u64, adam_step: u64,
                                     amp: *const ark_opt_state) -> c_int;
    pub fn ark_ckpt_plan_destroy(plan: *mut ark_ckpt_plan) -> c_int;
}

/// Opaque checkpoint pack plan.
#[repr(C)]
pub struct ark_ckpt_plan {
    _private: [u8; 0],
}

// ---- include/ark_grad.h ------------------------------------------------------

pub const ARK_GRAD_SCRATCH_BYTES: u64 = 48 << 20;

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct ark_grad_span {
    pub dst: *mut f32,
    pub src: *const f32,
    pub n: u64,
}

/// Opaque gradient plan.
#[repr(C)]
pub struct ark_grad_plan {
    _private: [u8; 0],
}

extern "C" {
    /// The host tail of `ark_mps_backward` (`objc/bridge.m:902-948`), on the device.
    pub fn ark_grad_accumulate(dst: *mut f32, src: *const f32, n: u64,
                               stream: *mut c_void) -> c_int;
    pub fn ark_grad_plan_create(spans: *const ark_grad_span, n_spans: i32, stream: *mut c_void,
                                out: *mut *mut ark_grad_plan) -> c_int;
    pub fn ark_grad_plan_run(plan: *mut ark_grad_plan) -> c_int;
    pub fn ark_grad_plan_destroy(plan: *mut ark_grad_plan) -> c_int;
    /// The token scatter of `objc/bridge.m:922-928`.
    pub fn ark_grad_embed_scatter(embed_grad: *mut f32, vocab: u32, d: u32, tokens: *const u32,
                                  dx0: *const f32, batch_seq: u32, stream: *mut c_void) -> c_int;
    /// No reference counterpart: the last accumulation and the scatter before a
    /// step, which also hand the step its norm's first level.
    pub fn ark_grad_plan_run_final(plan: *mut ark_grad_plan, opt: *mut ark_opt_handle) -> c_int;
    pub fn ark_grad_embed_scatter_final(embed_grad: *mut f32, vocab: u32, d: u32,
                                        tokens: *const u32, dx0: *const f32, batch_seq: u32,
                                        opt: *mut ark_opt_handle) -> c_int;
    /// No reference counterpart: the scatter for callers that cannot allocate.
    pub fn ark_grad_embed_scatter_noalloc(embed_grad: *mut f32, vocab: u32, d: u32,
                                          tokens: *const u32, dx0: *const f32, batch_seq: u32,
                                          stream: *mut c_void) -> c_int;
}

// ---- include/ark_synth.h (no reference counterpart: test and bench inputs) ---

extern "C" {
    pub fn ark_synth_normal_f16(out: *mut u16, n: u64, seed: u64, tensor_id: u32, step: u32,
                                sigma_scale: f32, stream: *mut c_void) -> c_int;
    pub fn ark_synth_normal_f32(out: *mut f32, n: u64, seed: u64, tensor_id: u32, step: u32,
                                sigma_scale: f32, stream: *mut c_void) -> c_int;
    pub fn ark_synth_fill_u16(out: *mut u16, n: u64, bits: u16, stream: *mut c_void) -> c_int;
    pub fn ark_synth_copy(dst: *mut c_void, src: *const c_void, nbytes: u64,
                          stream: *mut c_void) -> c_int;
    pub fn ark_synth_stream_mix(w: *mut u16, g: *const u16, m: *mut f32, v: *mut f32, n: u64,
                                spacing: u32, blocks_per_cu: u32, stream: *mut c_void) -> c_int;
}
