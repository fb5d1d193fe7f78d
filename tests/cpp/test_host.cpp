// Parity of the C++ mirror of the reference's interface (ark_amd/host/
// ark_host.hpp) against the CPU oracle, written the way the reference's own
// Rust would be exercised: Optimizer::new over an EKO parameter set held in
// one device buffer per tensor (as memory.rs:202-255 allocates them), twelve
// step_all calls with the lr_now warmup schedule (optimizer.rs:80-92), an
// inf gradient that must skip (training.rs:289-305), the logits-gradient
// overflow (training.rs:228-241), restaurar_momentos (optimizer.rs:237-313),
// CheckpointV3::save_fp16 / load (io.rs:432-671), the early stop
// (training.rs:298-301) and grad_clip_global (ffi.rs:206-213).  Every step's scalars and every w/m/v bit are
// compared with the oracle.  Prints "ark_host_test: OK ..." on success.
#include <stdio.h>
#include <string.h>
#include <unistd.h>

#include <string>
#include <vector>

#include "ark_host.hpp"
#include "ark_synth.h"
#include "ark_oracle.h"

using ark::host::AdamConfig;
using ark::host::AmpConfig;
using ark::host::CheckpointV3;
using ark::host::Error;
using ark::host::Optimizer;
using ark::host::TensorRef;

namespace {

int g_fail = 0;
long g_checks = 0;

#define EXPECT(cond, ...)                          \
  do {                                             \
    ++g_checks;                                    \
    if (!(cond)) {                                 \
      ++g_fail;                                    \
      printf("FAIL %s:%d: ", __FILE__, __LINE__);  \
      printf(__VA_ARGS__);                         \
      printf("\n");                                \
      fflush(stdout);                              \
    }                                              \
  } while (0)

void hip(hipError_t e, const char* what) {
  if (e != hipSuccess) {
    printf("HIP error in %s: %s\n", what, hipGetErrorString(e));
    fflush(stdout);
    exit(2);
  }
}

struct Spec {
  std::string name;
  uint64_t n;
  bool decay, gain;
};

// The step_all order (optimizer.rs:185-227): embed, gamma_final, per layer
// wq wk wv wo w1 w2 w3 g1 g2.
std::vector<Spec> eko(int layers, uint64_t d, uint64_t h, uint64_t vocab) {
  std::vector<Spec> s = {{"embed", vocab * d, true, false}, {"gamma_final", d, false, true}};
  const char* nm[9] = {"wq", "wk", "wv", "wo", "w1", "w2", "w3", "g1", "g2"};
  const uint64_t n[9] = {d * d, d * d, d * d, d * d, d * h, h * d, d * h, d, d};
  for (int l = 0; l < layers; ++l)
    for (int i = 0; i < 9; ++i) s.push_back({"l" + std::to_string(l) + "." + nm[i], n[i], i < 7, i >= 7});
  return s;
}

struct Set {  // device buffers, one allocation per array per tensor
  std::vector<uint16_t*> w, g;
  std::vector<float*> m, v;
};
struct Host {  // the oracle's copies
  std::vector<std::vector<uint16_t>> w, g;
  std::vector<std::vector<float>> m, v;
};

const uint64_t kSeed = 77;
const float kScale = 1024.0f;

void gen_grads(const std::vector<Spec>& sp, Set& d, Host& h, uint32_t step) {
  for (size_t i = 0; i < sp.size(); ++i) {
    const float ss = 1e-3f * kScale;
    ark::host::check(ark_synth_normal_f16(d.g[i], sp[i].n, kSeed, (uint32_t)i, step, ss, nullptr));
    ark_ref_synth_normal_f16(h.g[i].data(), sp[i].n, kSeed, (uint32_t)i, step, ss);
  }
}

void make(const std::vector<Spec>& sp, Set& d, Host& h) {
  for (size_t i = 0; i < sp.size(); ++i) {
    const uint64_t n = sp[i].n;
    uint16_t *w, *g;
    float *m, *v;
    hip(hipMalloc(&w, n * 2), "w");
    hip(hipMalloc(&g, n * 2), "g");
    hip(hipMalloc(&m, n * 4), "m");
    hip(hipMalloc(&v, n * 4), "v");
    hip(hipMemset(m, 0, n * 4), "m0");
    hip(hipMemset(v, 0, n * 4), "v0");
    d.w.push_back(w), d.g.push_back(g), d.m.push_back(m), d.v.push_back(v);
    h.w.emplace_back(n), h.g.emplace_back(n), h.m.emplace_back(n, 0.0f), h.v.emplace_back(n, 0.0f);
    if (sp[i].gain) {
      ark::host::check(ark_synth_fill_u16(w, n, 0x3C00, nullptr));
      for (auto& x : h.w[i]) x = 0x3C00;
    } else {
      ark::host::check(ark_synth_normal_f16(w, n, kSeed, (uint32_t)i, 0xFFFFFFFFu, 0.02f, nullptr));
      ark_ref_synth_normal_f16(h.w[i].data(), n, kSeed, (uint32_t)i, 0xFFFFFFFFu, 0.02f);
    }
  }
  gen_grads(sp, d, h, 0);
  hip(hipDeviceSynchronize(), "make");
}

// Bits of the device arrays against the oracle's (NaNs as a class).
uint64_t diff(const std::vector<Spec>& sp, const Set& d, const Host& h) {
  uint64_t bad = 0;
  for (size_t i = 0; i < sp.size(); ++i) {
    const uint64_t n = sp[i].n;
    std::vector<uint16_t> w(n);
    std::vector<uint32_t> m(n), v(n);
    hip(hipMemcpy(w.data(), d.w[i], n * 2, hipMemcpyDeviceToHost), "w back");
    hip(hipMemcpy(m.data(), d.m[i], n * 4, hipMemcpyDeviceToHost), "m back");
    hip(hipMemcpy(v.data(), d.v[i], n * 4, hipMemcpyDeviceToHost), "v back");
    for (uint64_t k = 0; k < n; ++k) {
      uint32_t hm, hv;
      memcpy(&hm, &h.m[i][k], 4);
      memcpy(&hv, &h.v[i][k], 4);
      bad += w[k] != h.w[i][k];
      bad += m[k] != hm;
      bad += v[k] != hv;
    }
  }
  return bad;
}

std::vector<ark_opt_tensor> oracle_table(const std::vector<Spec>& sp, Host& h, float wd) {
  std::vector<ark_opt_tensor> t(sp.size());
  for (size_t i = 0; i < sp.size(); ++i) {
    t[i].w = h.w[i].data();
    t[i].g = h.g[i].data();
    t[i].m = h.m[i].data();
    t[i].v = h.v[i].data();
    t[i].n = sp[i].n;
    t[i].weight_decay = sp[i].decay ? wd : 0.0f;
    t[i].flags = 0;
  }
  return t;
}

bool same_f(float a, float b) { return a == b || (a != a && b != b); }
bool same_d(double a, double b) { return a == b || (a != a && b != b); }

void compare_info(const ark_opt_step_info& a, const ark_opt_step_info& b, int step) {
  EXPECT(a.applied == b.applied && a.nonfinite == b.nonfinite && a.clipped == b.clipped &&
             a.status == b.status,
         "step %d: flags %d/%d %d/%d %d/%d %d/%d", step, a.applied, b.applied, a.nonfinite,
         b.nonfinite, a.clipped, b.clipped, a.status, b.status);
  EXPECT(same_d(a.grad_sumsq, b.grad_sumsq) && same_f(a.grad_norm, b.grad_norm) &&
             same_f(a.clip_coef, b.clip_coef) && same_f(a.lr_eff, b.lr_eff) &&
             same_f(a.inv_scale, b.inv_scale),
         "step %d: sumsq %.17g/%.17g norm %.9g/%.9g", step, a.grad_sumsq, b.grad_sumsq,
         a.grad_norm, b.grad_norm);
  EXPECT(a.state.t == b.state.t && a.state.loss_scale == b.state.loss_scale &&
             a.state.clean_steps == b.state.clean_steps &&
             a.state.skipped_steps == b.state.skipped_steps &&
             a.state.consecutive_nonfinite == b.state.consecutive_nonfinite,
         "step %d: state t %u/%u scale %g/%g", step, a.state.t, b.state.t, a.state.loss_scale,
         b.state.loss_scale);
}

}  // namespace

int main() {
  const std::vector<Spec> sp = eko(2, 64, 96, 500);
  Set d;
  Host h;
  make(sp, d, h);
  AdamConfig cfg;  // AdamConfig::default, with the benchmark configurations' overrides
  cfg.beta2 = 0.95f;
  cfg.weight_decay = 0.1f;
  cfg.warmup_steps = 5;
  AmpConfig amp;
  amp.loss_scale_init = kScale;
  amp.loss_scale_max = 16777216.0f;
  amp.scale_up_every = 4;  // small, so the growth branch runs within the test
  std::vector<TensorRef> table;
  for (size_t i = 0; i < sp.size(); ++i)
    table.push_back({d.w[i], d.g[i], d.m[i], d.v[i], sp[i].n, sp[i].decay, false});

  {
    Optimizer opt(cfg, table, amp);
    std::vector<ark_opt_tensor> otab = oracle_table(sp, h, cfg.weight_decay);
    ark_opt_hparams hp;
    ark_opt_default_hparams(&hp);
    hp.beta1 = cfg.beta1, hp.beta2 = cfg.beta2, hp.eps = cfg.eps, hp.grad_clip = cfg.grad_clip;
    hp.loss_scale_init = amp.loss_scale_init, hp.loss_scale_max = amp.loss_scale_max;
    hp.scale_up_every = amp.scale_up_every;
    ark_opt_state ost;
    ark_ref_state_init(&hp, &ost);

    for (int step = 0; step < 12; ++step) {
      if (step) gen_grads(sp, d, h, (uint32_t)step);
      if (step == 6) {  // one +inf gradient in a layer matrix: both skip
        const uint16_t inf = 0x7C00;
        hip(hipMemcpy(d.g[5] + 3, &inf, 2, hipMemcpyHostToDevice), "inject");
        h.g[5][3] = inf;
      }
      const float lr = opt.lr_now();  // optimizer.rs:172-173: lr of step + 1
      EXPECT(lr == ark::host::lr_now(cfg, ost.t + 1), "lr_now at step %d", step);
      ark_opt_step_info gi, ri;
      const bool applied = opt.step_all(lr, &gi);
      ark_ref_opt_step(otab.data(), (int32_t)otab.size(), &hp, &ost, lr, 4, &ri);
      compare_info(gi, ri, step);
      EXPECT(applied == (step != 6), "step %d applied=%d", step, (int)applied);
      const uint64_t bad = diff(sp, d, h);
      EXPECT(bad == 0, "step %d: %llu w/m/v elements differ", step, (unsigned long long)bad);
    }
    EXPECT(opt.step() == 11, "Optimizer::step = %u after 11 applied steps", opt.step());

    // the logits-gradient skip
    opt.record_overflow();
    ark_opt_step_info ri;
    ark_ref_record_overflow(&hp, &ost, &ri);
    const ark_opt_state s = opt.state();
    EXPECT(s.skipped_steps == ost.skipped_steps && s.loss_scale == ost.loss_scale &&
               s.t == ost.t,
           "record_overflow: skipped %llu/%llu scale %g/%g",
           (unsigned long long)s.skipped_steps, (unsigned long long)ost.skipped_steps,
           s.loss_scale, ost.loss_scale);

    // restaurar_momentos: checkpoint order (embed, layers, gamma_final)
    std::vector<std::vector<float>> mm, vv;
    mm.push_back(std::vector<float>(sp[0].n, 0.25f));
    vv.push_back(std::vector<float>(sp[0].n, 0.5f));
    for (size_t i = 2; i < sp.size(); ++i) {
      mm.push_back(std::vector<float>(sp[i].n, (float)i));
      vv.push_back(std::vector<float>(sp[i].n, 1.0f / (float)i));
    }
    mm.push_back(std::vector<float>(sp[1].n, -3.0f));
    vv.push_back(std::vector<float>(sp[1].n, 3.0f));
    EXPECT(opt.restaurar_momentos(mm, vv, 4321), "restaurar_momentos returned false");
    EXPECT(opt.step() == 4321, "step after restaurar_momentos = %u", opt.step());
    std::vector<float> back(sp[1].n);
    hip(hipMemcpy(back.data(), d.m[1], sp[1].n * 4, hipMemcpyDeviceToHost), "m gamma");
    EXPECT(back[0] == -3.0f && back.back() == -3.0f, "gamma_final m restored to %g", back[0]);
    hip(hipMemcpy(back.data(), d.v[1], sp[1].n * 4, hipMemcpyDeviceToHost), "v gamma");
    EXPECT(back[0] == 3.0f, "gamma_final v restored to %g", back[0]);
    std::vector<float> mbad = {1.0f};  // wrong count: nothing restored
    EXPECT(!opt.restaurar_momentos({mbad}, {mbad}, 9), "restaurar_momentos accepted 1 tensor");
    EXPECT(opt.step() == 4321, "step changed by a rejected restore");

    // CheckpointV3 round trip through a file, into fresh buffers
    const std::string path = "/tmp/ark_host_test_" + std::to_string(getpid()) + ".bin";
    std::vector<CheckpointV3::Layer> layers(2);
    uint64_t ln[9];
    for (int l = 0; l < 2; ++l)
      for (int i = 0; i < 9; ++i) {
        const size_t t = 2 + 9 * l + i;
        layers[l].w[i] = d.w[t], layers[l].m[i] = d.m[t], layers[l].v[i] = d.v[t];
        ln[i] = sp[t].n;
      }
    const ark_opt_state amp_state = opt.state();
    CheckpointV3::save_fp16(path, 1000, amp_state.t, d.w[0], d.m[0], d.v[0], sp[0].n, d.w[1],
                            d.m[1], d.v[1], sp[1].n, layers, ln, &amp_state);
    ark_ckpt_info info;
    ark::host::check(ark_ckpt_probe(path.c_str(), &info, nullptr, nullptr, 0));
    EXPECT(info.version == 4 && info.n_tensors == 3 + 27 * 2 + 3 && info.has_amp == 1 &&
               info.adam_step == 4321,
           "probe: version %u tensors %llu amp %u", info.version,
           (unsigned long long)info.n_tensors, info.has_amp);
    Set e;
    Host eh;
    make(sp, e, eh);
    std::vector<ark_ckpt_record> recs;
    auto rec = [&](size_t t) {
      recs.push_back({e.w[t], sp[t].n, ARK_CKPT_F16, 0});
    };
    auto recmv = [&](size_t t, bool v) {
      recs.push_back({v ? (void*)e.v[t] : (void*)e.m[t], sp[t].n, ARK_CKPT_F32, 0});
    };
    rec(0), recmv(0, false), recmv(0, true);
    for (int l = 0; l < 2; ++l) {
      for (int i = 0; i < 9; ++i) rec(2 + 9 * l + i);
      for (int i = 0; i < 9; ++i) recmv(2 + 9 * l + i, false);
      for (int i = 0; i < 9; ++i) recmv(2 + 9 * l + i, true);
    }
    rec(1), recmv(1, false), recmv(1, true);
    ark_opt_state loaded;
    const ark_ckpt_info li = CheckpointV3::load(path, recs, &loaded);
    unlink(path.c_str());
    EXPECT(li.has_amp && loaded.t == amp_state.t && loaded.loss_scale == amp_state.loss_scale,
           "loaded state t %u scale %g", loaded.t, loaded.loss_scale);
    uint64_t bad = 0;
    for (size_t t = 0; t < sp.size(); ++t) {
      const uint64_t n = sp[t].n;
      std::vector<uint8_t> a(n * 4), b(n * 4);
      hip(hipMemcpy(a.data(), d.w[t], n * 2, hipMemcpyDeviceToHost), "w0");
      hip(hipMemcpy(b.data(), e.w[t], n * 2, hipMemcpyDeviceToHost), "w1");
      bad += memcmp(a.data(), b.data(), n * 2) != 0;
      hip(hipMemcpy(a.data(), d.m[t], n * 4, hipMemcpyDeviceToHost), "m0");
      hip(hipMemcpy(b.data(), e.m[t], n * 4, hipMemcpyDeviceToHost), "m1");
      bad += memcmp(a.data(), b.data(), n * 4) != 0;
      hip(hipMemcpy(a.data(), d.v[t], n * 4, hipMemcpyDeviceToHost), "v0");
      hip(hipMemcpy(b.data(), e.v[t], n * 4, hipMemcpyDeviceToHost), "v1");
      bad += memcmp(a.data(), b.data(), n * 4) != 0;
    }
    EXPECT(bad == 0, "checkpoint round trip: %llu arrays differ", (unsigned long long)bad);
  }

  {  // early stop: the third consecutive skip past a limit of 2 (training.rs:298-301)
    AmpConfig a2 = amp;
    a2.max_consecutive_nonfinite = 2;
    Optimizer opt(cfg, table, a2);
    const uint16_t nan = 0x7E00;
    hip(hipMemcpy(d.g[0], &nan, 2, hipMemcpyHostToDevice), "nan");
    ark_opt_step_info gi;
    EXPECT(!opt.step_all(1e-3f, &gi), "first non-finite step applied");
    EXPECT(!opt.step_all(1e-3f, &gi), "second non-finite step applied");
    bool threw = false;
    try {
      opt.step_all(1e-3f, &gi);
    } catch (const Error& err) {
      threw = err.code() == ARK_OPT_EARLY_STOP && std::string(err.what()) == "early_stop_nan";
    }
    EXPECT(threw, "no early_stop_nan after 3 consecutive skips");
    bool rejected = false;
    try {
      std::vector<TensorRef> bad = table;
      bad[0].w = (uint16_t*)((char*)bad[0].w + 1);  // misaligned: refused before any launch
      Optimizer o2(cfg, bad, amp);
    } catch (const Error& err) {
      rejected = err.code() == ARK_OPT_EINVAL;
    }
    EXPECT(rejected, "misaligned table accepted");
  }

  {  // grad_clip_global (ffi.rs:206-213) on a device slice against the oracle's form of
     // ark_asm_grad_clip, clipped and not, and the empty slice
    const uint64_t n = 100003;  // a ragged last block and an n % 4 tail
    std::vector<float> h(n);
    ark_ref_synth_normal_f32(h.data(), n, 77, 1, 0, 1e-2f);
    float* dg = nullptr;
    hip(hipMalloc(&dg, n * 4), "clip buffer");
    for (float thr : {0.5f, 1e6f}) {
      std::vector<float> want = h;
      const float wn = ark_ref_grad_clip(want.data(), n, thr, 1);
      hip(hipMemcpy(dg, h.data(), n * 4, hipMemcpyHostToDevice), "clip upload");
      const float gn = ark::host::grad_clip_global(dg, n, thr);
      std::vector<float> got(n);
      hip(hipMemcpy(got.data(), dg, n * 4, hipMemcpyDeviceToHost), "clip read");
      EXPECT(memcmp(&gn, &wn, 4) == 0, "clip norm %.9g vs oracle %.9g", gn, wn);
      EXPECT(memcmp(got.data(), want.data(), n * 4) == 0, "clipped values differ (thr %g)", thr);
    }
    EXPECT(ark::host::grad_clip(dg, 0, 1.0f) == 0.0f, "empty slice norm not 0");
    hip(hipFree(dg), "clip free");
  }

  printf("ark_host_test: %s (%ld checks, %d failed)\n", g_fail ? "FAIL" : "OK", g_checks, g_fail);
  return g_fail ? 1 : 0;
}
