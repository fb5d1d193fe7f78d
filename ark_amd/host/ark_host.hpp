// ark_host.hpp -- C++ mirror of the reference's optimizer interface over the
// C ABI of libark_opt.so (header only; link -lark_opt -lamdhip64).
//
// The reference is Rust; its interface for this path is mirrored here with
// the same names, argument meaning and failure behaviour (paths relative to
// proyecto_ark/ark01/):
//   AdamConfig                 src/optimizer.rs:44-66 (Default)
//   AmpConfig                  the loss-scaler constants, src/training.rs:10-13,
//                              src/config.rs:36, :69, early stop :235, :298
//   Optimizer::Optimizer       Optimizer::new (src/optimizer.rs:74) over the
//                              device parameter table (src/memory.rs:202-255)
//   Optimizer::lr_now          src/optimizer.rs:80-92
//   Optimizer::step_all        Optimizer::step_all (src/optimizer.rs:171-228)
//                              with the AMP block of Trainer::train_step
//                              (src/training.rs:289-326): one fused device step
//   Optimizer::record_overflow src/training.rs:228-241
//   Optimizer::restaurar_momentos  src/optimizer.rs:237-313
//   CheckpointV3::save_fp16 / load src/io.rs:432-671
//   grad_clip_global / grad_clip  src/ffi.rs:206-220 (ark_asm_grad_clip,
//                              asm/opti.s:369-432) over a device buffer
// Errors: anyhow::Result becomes an ark::host::Error exception carrying the
// library status and message; the early stop is Error("early_stop_nan")
// with status ARK_OPT_EARLY_STOP (src/training.rs:236, :300).
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "ark_ckpt.h"
#include "ark_codec.h"
#include "ark_grad.h"
#include "ark_opt.h"

namespace ark {
namespace host {

class Error : public std::runtime_error {
 public:
  Error(int code, const std::string& msg) : std::runtime_error(msg), code_(code) {}
  int code() const { return code_; }

 private:
  int code_;
};

// A negative status becomes an Error with the library's message.
inline int check(int rc) {
  if (rc < 0) throw Error(rc, ark_opt_last_error());
  return rc;
}

inline void hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess)
    throw Error(ARK_OPT_EHIP, std::string(what) + ": " + hipGetErrorString(e));
}

struct AdamConfig {  // optimizer.rs:54-66
  float lr = 3e-4f;
  float beta1 = 0.9f;
  float beta2 = 0.999f;
  float eps = 1e-8f;
  float weight_decay = 0.01f;
  float grad_clip = 1.0f;
  uint32_t warmup_steps = 100;
};

struct AmpConfig {
  float loss_scale_init = 256.0f;         // training.rs:10
  float loss_scale_min = 1.0f;            // training.rs:12
  float loss_scale_max = 8192.0f;         // config.rs:69
  uint32_t scale_up_every = 2000;         // training.rs:13
  uint32_t max_consecutive_nonfinite = 200;  // training.rs:235, :298
};

// One tensor of the parameter set: device buffers of n elements.  decay:
// takes cfg.weight_decay (matrices and the embedding; the RMSNorm gains take
// none, optimizer.rs:194-200, :216-226).  no_unscale: the gradient is used
// as is (the reference's gamma_final, training.rs:133-146).
struct TensorRef {
  uint16_t* w;
  const void* g;
  float* m;
  float* v;
  uint64_t n;
  bool decay;
  bool no_unscale;
};

// optimizer.rs:80-92: linear warmup, then a cosine to lr/10 over 800k steps;
// `step` is the already-incremented Optimizer::step (step_all increments it
// before asking, optimizer.rs:172-173).
inline float lr_now(const AdamConfig& cfg, uint32_t step) {
  if (step < cfg.warmup_steps)
    return cfg.lr * ((float)step + 1.0f) / (float)cfg.warmup_steps;
  const float decay_steps = (float)(step - cfg.warmup_steps);
  const float total_decay = 800000.0f;
  const float progress = fminf(decay_steps / total_decay, 1.0f);
  // f32::cos as the correctly rounded fp32 cosine: libm's double cos rounded
  // once, which is exact rounding over every argument this schedule makes.
  const float cosine =
      0.5f * (1.0f + (float)::cos((double)(3.14159274101257324f * progress)));
  const float lr_min = cfg.lr * 0.1f;
  return lr_min + (cfg.lr - lr_min) * cosine;
}

class Optimizer {
 public:
  AdamConfig cfg;

  Optimizer(const AdamConfig& c, const std::vector<TensorRef>& table, const AmpConfig& amp = {},
            uint32_t grad_dtype = ARK_OPT_GRAD_F16, hipStream_t stream = nullptr)
      : cfg(c), stream_(stream) {
    ark_opt_hparams hp;
    check(ark_opt_default_hparams(&hp));
    hp.beta1 = c.beta1;
    hp.beta2 = c.beta2;
    hp.eps = c.eps;
    hp.grad_clip = c.grad_clip;
    hp.loss_scale_init = amp.loss_scale_init;
    hp.loss_scale_min = amp.loss_scale_min;
    hp.loss_scale_max = amp.loss_scale_max;
    hp.scale_up_every = amp.scale_up_every;
    hp.max_consecutive_nonfinite = amp.max_consecutive_nonfinite;
    hp.grad_dtype = grad_dtype;
    std::vector<ark_opt_tensor> t(table.size());
    for (size_t i = 0; i < table.size(); ++i) {
      t[i].w = table[i].w;
      t[i].g = table[i].g;
      t[i].m = table[i].m;
      t[i].v = table[i].v;
      t[i].n = table[i].n;
      t[i].weight_decay = table[i].decay ? c.weight_decay : 0.0f;
      t[i].flags = table[i].no_unscale ? ARK_OPT_TENSOR_NO_UNSCALE : 0u;
    }
    tensors_ = table;
    check(ark_opt_create(t.data(), (int32_t)t.size(), &hp, stream, &h_));
  }
  ~Optimizer() {
    if (h_) ark_opt_destroy(h_);
  }
  Optimizer(const Optimizer&) = delete;
  Optimizer& operator=(const Optimizer&) = delete;
  Optimizer(Optimizer&& o) noexcept
      : cfg(o.cfg), stream_(o.stream_), tensors_(std::move(o.tensors_)), h_(o.h_) {
    o.h_ = nullptr;
  }

  ark_opt_handle* handle() const { return h_; }

  // Optimizer::step: applied AdamW steps (waits for the device).
  uint32_t step() const { return state().t; }

  ark_opt_state state() const {
    ark_opt_state s;
    check(ark_opt_get_state(h_, &s));
    return s;
  }
  void set_state(const ark_opt_state& s) { check(ark_opt_set_state(h_, &s)); }

  // lr_now for the step this call would take.
  float lr_now() const { return host::lr_now(cfg, step() + 1u); }

  // One fused step at learning rate lr: the finite check, skip or unscale,
  // global norm and clip, AdamW on every tensor, loss-scale growth.  Returns
  // true when the update ran (false: a skipped step, training.rs:293-305);
  // throws Error("early_stop_nan") past max_consecutive_nonfinite skips.
  // With info == nullptr nothing waits on the host and the return value is
  // true (the outcome is on the device; read it with state()).
  bool step_all(float lr, ark_opt_step_info* info = nullptr) {
    const int rc = check(ark_opt_step(h_, lr, info));
    if (rc == ARK_OPT_EARLY_STOP) throw Error(rc, "early_stop_nan");
    return info ? info->applied != 0 : true;
  }
  // step_all with the reference's schedule (cfg.lr through lr_now).
  bool step_all_scheduled(ark_opt_step_info* info = nullptr) { return step_all(lr_now(), info); }

  // training.rs:228-241: a non-finite logits gradient, found before the
  // backward pass, counts as a skipped step.
  void record_overflow() {
    ark_opt_step_info info;
    const int rc = check(ark_opt_record_overflow(h_, &info));
    if (rc == ARK_OPT_EARLY_STOP) throw Error(rc, "early_stop_nan");
  }

  // optimizer.rs:237-313 over the table order embed, gamma_final, then per
  // layer wq..g2 (the order of step_all, optimizer.rs:185-227).  The moments
  // come in the checkpoint order: embed, 9 per layer, then gamma_final when
  // present (271 or 272 entries for EKO-237M).  Same tolerance as the
  // reference: a count mismatch restores nothing, an embed or layer size
  // mismatch stops there (what was copied stays) and leaves step unchanged,
  // a gamma_final size mismatch is skipped.  Returns true when step was set.
  bool restaurar_momentos(const std::vector<std::vector<float>>& momentos_m,
                          const std::vector<std::vector<float>>& momentos_v, uint32_t adam_step) {
    if (tensors_.size() < 2) throw Error(ARK_OPT_EINVAL, "restaurar_momentos needs an EKO set");
    const size_t n_capas = (tensors_.size() - 2) / 9;
    const size_t esperados = 1 + n_capas * 9;
    if ((momentos_m.size() != esperados && momentos_m.size() != esperados + 1) ||
        (momentos_v.size() != esperados && momentos_v.size() != esperados + 1))
      return false;
    // Every exit (a false return, a throw) waits for the copies already
    // queued from the caller's vectors.
    struct Drain {
      hipStream_t s;
      ~Drain() { (void)hipStreamSynchronize(s); }
    } drain{stream_};
    auto put = [&](size_t ti, size_t k) {
      const TensorRef& t = tensors_[ti];
      if (momentos_m[k].size() != t.n) return false;
      if (momentos_v[k].size() != t.n)  // copy_from_slice panics (memory.rs:60)
        throw Error(ARK_OPT_EINVAL, "momento v: size mismatch");
      hip_check(hipMemcpyAsync(t.m, momentos_m[k].data(), t.n * 4, hipMemcpyHostToDevice, stream_),
                "restaurar_momentos m");
      hip_check(hipMemcpyAsync(t.v, momentos_v[k].data(), t.n * 4, hipMemcpyHostToDevice, stream_),
                "restaurar_momentos v");
      return true;
    };
    if (!put(0, 0)) return false;                                   // :260-266 embed
    if (momentos_m.size() == esperados + 1) (void)put(1, esperados);  // :269-275 gamma_final
    for (size_t k = 1; k < esperados; ++k)                          // :278-306 layers
      if (!put(2 + (k - 1), k)) return false;
    hip_check(hipStreamSynchronize(stream_), "restaurar_momentos");
    ark_opt_state s = state();
    s.t = adam_step;                                                // :308
    set_state(s);
    return true;
  }

 private:
  hipStream_t stream_ = nullptr;
  std::vector<TensorRef> tensors_;
  ark_opt_handle* h_ = nullptr;
};

// src/ffi.rs:206-213: the pre-clip L2 norm of grads[0, n) (device memory),
// which are scaled in place by threshold / norm when it exceeds threshold;
// 0 for an empty slice.  Waits for the stream, as the reference returns the
// norm.
inline float grad_clip_global(float* grads, uint64_t n, float threshold,
                              hipStream_t stream = nullptr) {
  if (n == 0) return 0.0f;
  float norm = 0.0f;
  check(ark_hip_grad_clip(grads, n, threshold, &norm, stream));
  return norm;
}

// src/ffi.rs:216-220: the reference's alias.
inline float grad_clip(float* grads, uint64_t n, float threshold, hipStream_t stream = nullptr) {
  return grad_clip_global(grads, n, threshold, stream);
}

// src/io.rs:417-671 over device buffers.
struct CheckpointV3 {
  // save_fp16 (io.rs:432-500): embed w/m/v, per layer 9 w, 9 m, 9 v,
  // gamma_final w/m/v; w fp16, m/v fp32, each pointer n elements.  amp
  // (optional) adds the loss-scaler trailer the reference's loader skips.
  struct Layer {
    uint16_t* w[9];
    float* m[9];
    float* v[9];
  };
  static void save_fp16(const std::string& path, uint64_t global_step, uint64_t adam_step,
                        uint16_t* embed_w, float* embed_m, float* embed_v, uint64_t embed_n,
                        uint16_t* gamma_w, float* gamma_m, float* gamma_v, uint64_t gamma_n,
                        const std::vector<Layer>& layers, const uint64_t layer_n[9],
                        const ark_opt_state* amp = nullptr, hipStream_t stream = nullptr) {
    std::vector<ark_ckpt_record> r;
    auto add = [&](void* p, uint64_t n, uint32_t t) { r.push_back({p, n, t, 0u}); };
    add(embed_w, embed_n, ARK_CKPT_F16);
    add(embed_m, embed_n, ARK_CKPT_F32);
    add(embed_v, embed_n, ARK_CKPT_F32);
    for (const Layer& l : layers) {
      for (int i = 0; i < 9; ++i) add(l.w[i], layer_n[i], ARK_CKPT_F16);
      for (int i = 0; i < 9; ++i) add(l.m[i], layer_n[i], ARK_CKPT_F32);
      for (int i = 0; i < 9; ++i) add(l.v[i], layer_n[i], ARK_CKPT_F32);
    }
    add(gamma_w, gamma_n, ARK_CKPT_F16);
    add(gamma_m, gamma_n, ARK_CKPT_F32);
    add(gamma_v, gamma_n, ARK_CKPT_F32);
    check(ark_ckpt_save_v4(path.c_str(), global_step, adam_step, r.data(), (int32_t)r.size(), amp,
                           stream));
  }

  // load (io.rs:504-671) into device records given in file order (see
  // ark_ckpt_probe for the layout); returns the header, fills *amp when the
  // file carries the trailer.
  static ark_ckpt_info load(const std::string& path, const std::vector<ark_ckpt_record>& records,
                            ark_opt_state* amp = nullptr, hipStream_t stream = nullptr) {
    ark_ckpt_info info;
    check(ark_ckpt_load(path.c_str(), records.data(), (int32_t)records.size(), &info, amp,
                        stream));
    return info;
  }
};

}  // namespace host
}  // namespace ark
