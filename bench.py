#!/usr/bin/env python3
"""Benchmark of the fused optimizer step on one MI355X.

Default workload: configuration c2, the full EKO-237M parameter set (272
tensors, 236,959,488 params): fp16 weights ~N(0,0.02) (gains 1.0), fp16
gradients N(0, sigma_t) * 65536 with per-tensor sigma_t = 10^U(-5,-2), fp32
m/v, one fused unscale + finite check + norm + clip + AdamW + loss-scale step
repeated --steps times.  Inputs are generated on the device before timing.

Prints one JSON line: value = achieved algorithmic HBM throughput of the
whole step (24 B/param / step time) in GB/s; ms_per_step; a roofline object
for the dominant kernel (the fused AdamW pass, 22 B/param, timed with HIP
events on the stream it runs on); a cpu_baseline object (the C oracle on the
host cores -- its 8-wide AVX2/F16C loops, bit-identical to the scalar
restatement -- on a bounded sample of the same workload).
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "EKO-237M fused AdamW step ms + achieved HBM GB/s vs peak (1 GPU)"
PEAK_HBM_GBS = 8000.0


def step_bytes(grad):
    """Algorithmic bytes per parameter of the step and of its AdamW pass: the
    norm pass reads g, the fused update reads g, w, m, v and writes w, m, v
    (g 2 B fp16 / 4 B fp32, w 2+2, m 4+4, v 4+4): 24 and 22 B for fp16
    gradients, 28 and 24 B for fp32."""
    gs = 2 if grad == "f16" else 4
    if grad == "f32-fused":  # the norm's first level comes from the producer
        return gs + 20, gs + 20
    return 2 * gs + 20, gs + 20


WORKLOADS = {
    "c2": dict(desc="EKO-237M: 30 layers, d 768, ffn 2048, tied embed 32000x768 (272 tensors)",
               loss_scale=65536.0, sigma="loguniform"),
    "c3": dict(desc="EKO-237M AMP stress set (272 tensors): applied steps, then skipped steps "
                    "(an inf in one gradient; training.rs:293-305)",
               loss_scale=65536.0, sigma="loguniform"),
    "c4": dict(desc="1.3B scale-up: 24 layers, d 2048, ffn 5504, tied embed 32000x2048 (218 tensors)",
               loss_scale=65536.0, sigma=1e-3),
    "c2s8": dict(desc="one GPU's share of c2 over 8 GPUs: rank 0's contiguous eighth of the "
                      "segment list (tied embed, gamma_final, l0.wq..w1 and a slice of l0.w2); "
                      "the step as that rank runs it, without the cross-GPU norm exchange",
                 loss_scale=65536.0, sigma="loguniform"),
    "c4s8": dict(desc="one GPU's share of c4 over 8 GPUs: rank 0's contiguous eighth of the "
                      "segment list; the step as that rank runs it, without the cross-GPU "
                      "norm exchange",
                 loss_scale=65536.0, sigma=1e-3),
    "c1": dict(desc="one EKO layer (9 tensors)", loss_scale=1024.0, sigma=1e-3),
    "c0": dict(desc="single 768x768 tensor", loss_scale=1024.0, sigma=1e-3),
}
HP = dict(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1, grad_clip=1.0)
SEED = 20260501


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def sigmas_for(name, specs):
    from ark_amd import synth
    w = WORKLOADS[name]
    if w["sigma"] == "loguniform":
        return synth.log_uniform_sigmas(len(specs), SEED)
    return [w["sigma"]] * len(specs)


def run_gpu(name, steps, warmup, grad="f16", skip=False):
    """skip: also time skipped steps on the same handle afterwards (always
    for c3; c2's tensor set is c3's)."""
    import torch
    torch.cuda.set_device(0)
    # everything on one non-default stream, so the step can also be captured
    # in a HIP graph
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        return _run_gpu(name, steps, warmup, stream, grad, skip)


def _run_gpu(name, steps, warmup, stream, grad="f16", skip=False):
    import torch
    from ark_amd import _abi, synth
    from ark_amd.eko import config_tensors
    from ark_amd.optimizer import AdamConfig, AmpConfig, Optimizer

    specs = config_tensors(name)
    w = WORKLOADS[name]
    sig = sigmas_for(name, specs)
    cfg = AdamConfig(**HP)
    skip = skip or name == "c3"
    # skipped steps are timed back to back: no early stop after 200 of them
    amp = AmpConfig(loss_scale_init=w["loss_scale"], loss_scale_max=2.0 ** 24,
                    max_consecutive_nonfinite=(2 ** 31 if skip else 200))
    log(f"[bench] building {name}: {sum(s.n for s in specs)} params, {len(specs)} tensors")
    gdt = _abi.GRAD_F16 if grad == "f16" else _abi.GRAD_F32
    ps = synth.problem(specs, SEED, cfg.weight_decay, sig, w["loss_scale"], grad_dtype=gdt)
    opt = Optimizer(cfg, ps, amp)
    torch.cuda.synchronize()
    if grad == "f32-fused":
        return _run_fused(specs, ps, opt, cfg, steps, warmup, stream)
    _, info = opt.step_all(cfg.lr, info=True)
    log(f"[bench] first step: applied={info.applied} norm={info.grad_norm:.6g} "
        f"clipped={info.clipped} scale={info.state.loss_scale}")
    for _ in range(warmup):
        opt.step_all(cfg.lr)
    torch.cuda.synchronize()

    # timed region: K steps, no per-kernel events
    t0 = time.perf_counter()
    for _ in range(steps):
        opt.step_all(cfg.lr)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = wall * 1e3 / steps

    # per-kernel HIP-event timing over the same number of steps
    opt.set_timing(True)
    for _ in range(steps):
        opt.step_all(cfg.lr)
    torch.cuda.synchronize()
    tm = opt.get_timing()
    opt.set_timing(False)

    # the same step captured once in a HIP graph and replayed K times
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        opt.step_all(cfg.lr)
    for _ in range(min(warmup, 5)):
        graph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        graph.replay()
    torch.cuda.synchronize()
    graph_ms = (time.perf_counter() - t0) * 1e3 / steps
    del graph

    _, last = opt.step_all(cfg.lr, info=True)
    skip = _time_skipped(ps, opt, cfg, steps) if skip else None
    n = ps.n_params
    res = dict(skip=skip,
        n_params=n, n_tensors=len(specs), ms_step=ms_step,
        ms_adamw=tm.ms_adamw / tm.steps, ms_norm=tm.ms_norm / tm.steps,
        ms_finalize=tm.ms_finalize / tm.steps, ms_step_events=tm.ms_step / tm.steps,
        clipped=int(last.clipped), applied=int(last.applied), t=int(last.state.t),
        grad_norm=float(last.grad_norm), graph_ms=graph_ms,
    )
    opt.close()
    del ps
    torch.cuda.empty_cache()
    return res


def _time_skipped(ps, opt, cfg, steps):
    """steps skipped steps (training.rs:293-305): +inf planted in one fp16
    gradient, so the norm pass flags it, the finalize halves the loss scale
    and counts the skip, and the AdamW pass exits at once.  Wall clock over
    the steps, and the kernels with the handle's events; the gradient is
    restored afterwards."""
    import torch
    g16 = ps.g(0).view(torch.int16)
    old = int(g16[0].item())
    g16[0] = 0x7C00  # +inf
    _, first = opt.step_all(cfg.lr, info=True)
    assert first.applied == 0
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        opt.step_all(cfg.lr)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / steps
    opt.set_timing(True)
    for _ in range(steps):
        opt.step_all(cfg.lr)
    torch.cuda.synchronize()
    tm = opt.get_timing()
    opt.set_timing(False)
    _, last = opt.step_all(cfg.lr, info=True)
    g16[0] = old
    assert last.applied == 0 and last.state.skipped_steps >= 2 * steps + 2
    log(f"[bench] skipped step: {wall_ms:.4f} ms (norm {tm.ms_norm / tm.steps:.4f}, finalize "
        f"{tm.ms_finalize / tm.steps:.4f})")
    # the AdamW launch's own event interval is left out: events around a
    # launch whose blocks all exit at once read longer than the whole
    # skipped step's wall clock; rocprofv3's kernel trace times that dispatch
    return dict(ms_per_skipped_step=round(wall_ms, 4),
                kernels_ms={"sumsq": round(tm.ms_norm / tm.steps, 4),
                            "finalize": round(tm.ms_finalize / tm.steps, 4)},
                skipped_total=int(last.state.skipped_steps))


def _run_fused(specs, ps, opt, cfg, steps, warmup, stream):
    """The step on fp32 gradients that a gradient plan's final accumulation
    has just produced (GradPlan.run(final_for=opt), include/ark_grad.h): the
    accumulation also writes the norm's units, so the step reads no gradient
    for its norm.  Each step is preceded by that accumulation (gradients +=
    fixed backward outputs); the step itself is timed with the handle's HIP
    events, the accumulation and the accumulate + step pair separately, and
    the same pair with the plain accumulation and the reading step for
    comparison."""
    import torch
    from ark_amd import grad as G
    n = len(specs)
    outs = [ps.g(i).clone() for i in range(n)]
    for i in range(n):
        ps.g(i).zero_()
    plan = G.GradPlan([(ps.g(i), outs[i]) for i in range(n)], stream=stream)

    def pair(fused, k):
        for _ in range(k):
            plan.run(final_for=opt if fused else None)
            opt.step_all(cfg.lr)

    def wall(fused):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        pair(fused, steps)
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3 / steps

    def events(fused):
        opt.set_timing(True)
        pair(fused, steps)
        torch.cuda.synchronize()
        tm = opt.get_timing()
        opt.set_timing(False)
        return tm

    pair(True, warmup)
    pair_fused, pair_plain = wall(True), wall(False)
    tf, tp = events(True), events(False)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(steps):
        plan.run(final_for=opt)
    e1.record(stream)
    torch.cuda.synchronize()
    producer_ms = e0.elapsed_time(e1) / steps
    e0.record(stream)
    for _ in range(steps):
        plan.run()
    e1.record(stream)
    torch.cuda.synchronize()
    plain_producer_ms = e0.elapsed_time(e1) / steps
    plan.run(final_for=opt)
    _, last = opt.step_all(cfg.lr, info=True)
    # The step's time: the accumulate + step pair (wall clock over K pairs,
    # synchronised on both sides) minus the accumulation alone (HIP events).
    # The handle's own events around the step misplace the norm pass when a
    # kernel of the accumulation precedes it on the stream (they report
    # 0.08 ms for a norm pass the kernel trace times at 0.151 ms); the pair
    # difference agrees with the kernel trace for both flows.
    step_fused = pair_fused - producer_ms
    step_plain = pair_plain - plain_producer_ms
    log(f"[bench] fused: step {step_fused:.4f} ms, reading step {step_plain:.4f} ms; pairs "
        f"{pair_fused:.4f} / {pair_plain:.4f} ms; accumulations {producer_ms:.4f} / "
        f"{plain_producer_ms:.4f} ms")
    res = dict(
        n_params=ps.n_params, n_tensors=n, ms_step=step_fused,
        ms_adamw=tf.ms_adamw / tf.steps, ms_norm=tf.ms_norm / tf.steps,
        ms_finalize=tf.ms_finalize / tf.steps, ms_step_events=tf.ms_step / tf.steps,
        clipped=int(last.clipped), applied=int(last.applied), t=int(last.state.t),
        grad_norm=float(last.grad_norm), graph_ms=None,
        fused=dict(producer_ms=round(producer_ms, 4), pair_ms=round(pair_fused, 4),
                   step_events_ms=round(tf.ms_step / tf.steps, 4),
                   plain_producer_ms=round(plain_producer_ms, 4),
                   plain_step_ms=round(step_plain, 4),
                   plain_pair_ms=round(pair_plain, 4)),
    )
    plan.close()
    opt.close()
    del ps
    torch.cuda.empty_cache()
    return res


def run_ceiling(a):
    """The measured ceiling of the AdamW pass's access pattern, on the same
    memory as the pass: the stream-mix probe (ark_synth_stream_mix: AdamW's
    one-wave-per-row shape, seven streams and cache hints, 22 B/param, its
    arithmetic replaced by a chain of `spacing` dependent fma) run over the
    workload's own parameter arenas.  First a sweep of spacing and of the
    resident blocks per CU (every wave slot, 20, 16 -- the AdamW pass's --
    and 14; median of --steps launches each, HIP events); then --steps
    rounds that each time one probe launch at the best point and one
    optimizer step with the handle's per-kernel events, so the probe and the
    AdamW pass are compared interleaved on the same box and the same pages."""
    import torch
    from ark_amd import synth
    from ark_amd.eko import config_tensors
    from ark_amd.optimizer import AdamConfig, AmpConfig, Optimizer
    torch.cuda.set_device(0)
    name = a.workload
    specs = config_tensors(name)
    w = WORKLOADS[name]
    cfg = AdamConfig(**HP)
    ps = synth.problem(specs, SEED, cfg.weight_decay, sigmas_for(name, specs), w["loss_scale"])
    opt = Optimizer(cfg, ps, AmpConfig(loss_scale_init=w["loss_scale"], loss_scale_max=2.0 ** 24))
    n = ps.total - ps.total % 256
    arenas = (ps.w_arena[:n].view(torch.int16), ps.g_arena[:n].view(torch.int16),
              ps.m_arena[:n], ps.v_arena[:n])
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def probe(spacing, per_cu):
        e0.record()
        synth.stream_mix(*arenas, spacing, per_cu)
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1)

    sweep = []
    for per_cu in (0, 20, 16, 14):
        for spacing in (0, 16, 32, 64, 128, 256):
            probe(spacing, per_cu)
            ms = sorted(probe(spacing, per_cu) for _ in range(a.steps))[a.steps // 2]
            sweep.append(dict(spacing=spacing, blocks_per_cu=per_cu, ms=round(ms, 4),
                              gbs=round(22 * n / (ms * 1e-3) / 1e9, 1)))
            log(f"[bench] stream mix {per_cu:2d} blocks per CU, spacing {spacing:4d}: "
                f"{ms:.4f} ms = {sweep[-1]['gbs']} GB/s")
    best_pt = min(sweep, key=lambda r: r["ms"])
    best, best_cu = best_pt["spacing"], best_pt["blocks_per_cu"]
    for _ in range(3):
        opt.step_all(cfg.lr)
    probe_ms, adam_ms = [], []
    for _ in range(a.steps):
        probe_ms.append(probe(best, best_cu))
        opt.set_timing(True)
        opt.step_all(cfg.lr)
        torch.cuda.synchronize()
        tm = opt.get_timing()
        opt.set_timing(False)
        adam_ms.append(tm.ms_adamw / tm.steps)
    pm = sorted(probe_ms)[a.steps // 2]
    am = sorted(adam_ms)[a.steps // 2]
    n_params = ps.n_params
    log(f"[bench] interleaved: probe {pm:.4f} ms ({n} elements), AdamW {am:.4f} ms "
        f"({n_params} params): AdamW / probe per element {am / pm * n / n_params:.4f}")
    out = {
        "metric": "AdamW stream-mix ceiling (22 B/param, 1 GPU) GB/s",
        "value": round(22 * n / (pm * 1e-3) / 1e9, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": a.steps, "warmup": 1, "ms_per_step": round(pm, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "u16/f32 copy", "data": "synthetic",
        "config": {"workload": f"{name}: the optimizer's parameter arenas ({n} elements; "
                               f"{n_params} params)",
                   "sweep": sweep, "best_spacing": best, "best_blocks_per_cu": best_cu,
                   "interleaved": {"probe_ms": round(pm, 4), "adamw_ms": round(am, 4),
                                   "adamw_gbs": round(22 * n_params / (am * 1e-3) / 1e9, 1),
                                   "adamw_over_probe_per_element":
                                       round(am / pm * n / n_params, 4)}},
    }
    opt.close()
    print(json.dumps(out), flush=True)


def calib_copy(nbytes=1 << 30, reps=3):
    """A plain copy kernel of known size (ark_synth_copy: one 16-byte
    non-temporal load and store per thread): under rocprofv3 --pmc its
    FETCH_SIZE / WRITE_SIZE per dispatch calibrate the counters."""
    import torch
    from ark_amd import synth
    src = torch.ones(nbytes // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(reps):
        synth.copy(dst, src)
    torch.cuda.synchronize()
    log(f"[bench] calibration copy: {reps} x {nbytes} bytes")


def run_cpu_baseline(name, budget_s, threads, grad="f16"):
    """The C oracle (same arithmetic, bit-identical results) timed on the
    host cores: full steps of the same workload until budget_s is spent."""
    import numpy as np
    import oracle
    from oracle import harness as H
    from ark_amd import _abi
    from ark_amd.eko import config_tensors
    from ark_amd.optimizer import AdamConfig, AmpConfig, hparams

    specs = config_tensors(name)
    w = WORKLOADS[name]
    sig = sigmas_for(name, specs)
    cfg = AdamConfig(**HP)
    amp = AmpConfig(loss_scale_init=w["loss_scale"], loss_scale_max=2.0 ** 24)
    gdt = _abi.GRAD_F16 if grad == "f16" else _abi.GRAD_F32
    ts = H.host_problem(specs, SEED, cfg.weight_decay, sig, w["loss_scale"], grad_dtype=gdt)
    ref = oracle.Optimizer(ts, hparams(cfg, amp, gdt), nthreads=threads)
    n = sum(s.n for s in specs)
    vec = oracle.set_vector(True)  # the 8-wide AVX2/F16C loops (same bits as the scalar form)
    ref.step(cfg.lr)  # warm (page in)
    done, t0 = 0, time.perf_counter()
    while True:
        ref.step(cfg.lr)
        done += 1
        el = time.perf_counter() - t0
        if el >= budget_s or done >= 1000:
            break
    oracle.set_vector(False)
    s_step = el / done
    cpu = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return dict(value=round(step_bytes(grad)[0] * n / s_step / 1e9, 3), unit="GB/s", cores=threads,
                kind="port", ms_per_step=round(s_step * 1e3, 3),
                sample=f"{done} full {name} steps ({n} params) in {el:.1f} s on {threads} "
                       f"threads of {os.cpu_count()} ({cpu}), "
                       f"{'8-wide AVX2/F16C' if vec else 'scalar'} loops")


def profile_summary(name, kernel="adamw_kernel"):
    """The committed rocprofv3 figures of `kernel` on this workload
    (profiles/<kernel>_<name>_traffic.txt): HBM-side bytes per launch from
    the byte counters, calibrated against a plain copy, and the kernel
    trace's average launch duration; {} when none is committed."""
    p = os.path.join(ROOT, "profiles", f"{kernel}_{name}_traffic.txt")
    if not os.path.exists(p):
        return {}
    kv = {}
    for line in open(p):
        if ":" in line and not line.startswith("#"):
            k, v = line.split(":", 1)
            kv[k.strip()] = v.strip()
    return kv


def traffic_from_profiles(name, kernel="adamw_kernel"):
    """(bytes per launch, source) from profile_summary; (None, None) when no
    profile of it is committed."""
    kv = profile_summary(name, kernel)
    if not kv:
        return None, None
    return int(kv["bytes_per_launch"]), kv.get("source")


def secondary_c4(steps, warmup):
    """The 1.3B scale-up (c4) step timed the same way as the headline, on a
    problem built after the headline's was freed; no CPU leg."""
    r = run_gpu("c4", steps, warmup, "f16")
    n = r["n_params"]
    b_step, b_adamw = step_bytes("f16")
    gbs = b_step * n / (r["ms_step"] * 1e-3) / 1e9
    adam_gbs = b_adamw * n / (r["ms_adamw"] * 1e-3) / 1e9
    out = dict(workload=f"c4: {WORKLOADS['c4']['desc']}", params=n, tensors=r["n_tensors"],
               ms_per_step=round(r["ms_step"], 4), gbs=round(gbs, 2),
               frac_of_peak_hbm=round(gbs / PEAK_HBM_GBS, 4),
               bytes_per_step=b_step * n, clipped=r["clipped"],
               hip_graph_ms_per_step=round(r["graph_ms"], 4),
               kernels_ms={"sumsq": round(r["ms_norm"], 4), "finalize": round(r["ms_finalize"], 4),
                           "adamw": round(r["ms_adamw"], 4)},
               adamw=dict(achieved=round(adam_gbs, 2), unit="GB/s",
                          frac=round(adam_gbs / PEAK_HBM_GBS, 4),
                          algorithmic_bytes_per_launch=b_adamw * n))
    kv = profile_summary("c4")
    if kv:
        ns = float(kv["avg_launch_ns"])
        out["adamw"].update(
            traffic=int(kv["bytes_per_launch"]), profile_avg_us=round(ns / 1e3, 1),
            profile_frac=round(b_adamw * n / (ns * 1e-9) / 1e9 / PEAK_HBM_GBS, 4),
            profile_source=kv.get("source"))
    return out


def run_codec(a):
    """The weight codec over EKO-237M (include/ark_codec.h): one launch
    dequantising all 272 fp16 weight tensors to fp32 (the per-step loop of
    training.rs:162-186), and one quantising them back (sync_weights_to_gpu,
    memory.rs:347-377).  6 B per element each way."""
    import torch
    from ark_amd import codec
    from ark_amd.eko import config_tensors
    torch.cuda.set_device(0)
    specs = config_tensors("c2")
    n = sum(s.n for s in specs)
    g = torch.Generator(device="cuda").manual_seed(SEED)
    w16 = [(torch.randn(s.n, device="cuda", generator=g) * 0.02).half() for s in specs]
    f32 = [torch.empty(s.n, dtype=torch.float32, device="cuda") for s in specs]
    back = [torch.empty(s.n, dtype=torch.float16, device="cuda") for s in specs]
    dq = codec.CodecPlan(list(zip(w16, f32)), "f16_to_f32")
    qt = codec.CodecPlan(list(zip(f32, back)), "f32_to_f16")
    res = {}
    for name, plan in (("dequant", dq), ("quant", qt)):
        for _ in range(a.warmup):
            plan.run()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record()
        for _ in range(a.steps):
            plan.run()
        e1.record()
        torch.cuda.synchronize()
        wall = (time.perf_counter() - t0) * 1e3 / a.steps
        res[name] = dict(ms=e0.elapsed_time(e1) / a.steps, wall_ms=wall)
    ok = all(torch.equal(x.view(torch.int16), y.view(torch.int16)) for x, y in zip(w16, back))
    dq.close(), qt.close()
    cpu = None
    if not a.no_cpu:
        import numpy as np
        import oracle
        from concurrent.futures import ThreadPoolExecutor
        th = a.cpu_threads or min(16, os.cpu_count() or 1)
        src = w16[0].view(torch.int16).cpu().numpy().view(np.uint16)  # the 24.6M-element embed
        parts = np.array_split(src, th)
        reps, t0 = 0, time.perf_counter()
        with ThreadPoolExecutor(th) as ex:
            while time.perf_counter() - t0 < min(a.cpu_seconds, 10.0):
                list(ex.map(oracle.f16_to_f32, parts))
                reps += 1
        el = time.perf_counter() - t0
        cpu = dict(value=round(6 * src.size * reps / el / 1e9, 3), unit="GB/s", cores=th,
                   kind="port", sample=f"{reps} dequantisations of the {src.size}-element "
                   f"embedding in {el:.1f} s on {th} threads")
    d = res["dequant"]
    gbs = 6 * n / (d["ms"] * 1e-3) / 1e9
    q_gbs = 6 * n / (res["quant"]["ms"] * 1e-3) / 1e9
    out = {
        "metric": "EKO-237M weight dequant fp16->fp32, all tensors, GB/s (1 GPU)",
        "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": round(d["ms"], 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "codec: 272 EKO-237M weight tensors, one launch per direction",
                   "elements": n, "bytes_per_launch": 6 * n, "round_trip_exact": bool(ok),
                   "quant_ms": round(res["quant"]["ms"], 4), "quant_GBs": round(q_gbs, 2)},
        "roofline": {"kernel": "codec_batch<f16_to_f32>", "bound": "hbm", "achieved": round(gbs, 2),
                     "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4),
                     "traffic": traffic_from_profiles("eko237m", "codec_batch")[0],
                     "traffic_source": traffic_from_profiles("eko237m", "codec_batch")[1],
                     "algorithmic_bytes_per_launch": 6 * n},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


def run_ckpt(a):
    """Checkpoint V4 of EKO-237M (include/ark_ckpt.h): the 816-record file
    image (2.37 GB: fp16 w, fp32 m/v) packed from the device buffers and
    unpacked back, in device memory (2 B of traffic per image byte each
    way), then the whole file written and read through the host."""
    import tempfile
    import torch
    from ark_amd import ckpt
    from ark_amd.eko import EKO_237M
    from ark_amd.optimizer import ParamSet
    torch.cuda.set_device(0)
    ps = ParamSet(EKO_237M.tensors(), weight_decay=0.1)
    tens = ckpt.param_tensors(ps)
    g = torch.Generator(device="cuda").manual_seed(SEED)
    for t in tens:
        t.copy_(torch.randn(t.shape, device="cuda", generator=g) * 0.02)
    recs = ckpt.Records(tens)
    nb = ckpt.image_bytes(recs)
    img = torch.empty(nb, dtype=torch.uint8, device="cuda")
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    res = {}
    steps = max(1, min(a.steps, 50))
    for name, fn in (("pack", lambda: ckpt.pack(recs, img, 1000, 999)),
                     ("unpack", lambda: ckpt.unpack(img, recs))):
        for _ in range(min(a.warmup, 5)):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        e0.record()
        for _ in range(steps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        res[name] = dict(ms=e0.elapsed_time(e1) / steps,
                         wall_ms=(time.perf_counter() - t0) * 1e3 / steps)
    # the same pack from a prepared plan: runs queued back to back, so the
    # events time the device work (header kernel + data kernel) without the
    # per-call table upload and host wait
    plan = ckpt.PackPlan(recs, img)
    for _ in range(min(a.warmup, 5)):
        plan.run(1000, 999)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(steps):
        plan.run(1000, 999)
    e1.record()
    torch.cuda.synchronize()
    res["plan"] = dict(ms=e0.elapsed_time(e1) / steps)
    plan.close()
    d = "/dev/shm" if os.path.isdir("/dev/shm") else tempfile.gettempdir()
    path = os.path.join(d, f"ark_bench_ckpt_{os.getpid()}.bin")
    try:
        t0 = time.perf_counter()
        ckpt.save(path, recs, 1000, 999)
        save_s = time.perf_counter() - t0
        t0 = time.perf_counter()
        ckpt.load(path, recs)
        load_s = time.perf_counter() - t0
    finally:
        if os.path.exists(path):
            os.remove(path)
    cpu = None
    if not a.no_cpu:
        import numpy as np
        from oracle import ckpt as K
        host = [t.cpu().numpy() for t in tens[:30]]  # embed w/m/v + layer 0's 27 records
        reps, t0 = 0, time.perf_counter()
        nbytes = 0
        while time.perf_counter() - t0 < min(a.cpu_seconds, 10.0):
            nbytes += len(K.write_v4(1000, 999, host))
            reps += 1
        el = time.perf_counter() - t0
        cpu = dict(value=round(2 * nbytes / el / 1e9, 3), unit="GB/s", cores=1, kind="port",
                   sample=f"{reps} V4 images of embed + layer 0 ({nbytes // reps} B each) built "
                          f"by the oracle writer in {el:.1f} s")
    pk = 2 * nb / (res["plan"]["ms"] * 1e-3) / 1e9
    pk_call = 2 * nb / (res["pack"]["ms"] * 1e-3) / 1e9
    up = 2 * nb / (res["unpack"]["ms"] * 1e-3) / 1e9
    out = {
        "metric": "EKO-237M checkpoint V4 pack from device buffers, GB/s of HBM traffic (1 GPU)",
        "value": round(pk, 2), "unit": "GB/s", "n_gpus": 1, "steps": steps,
        "warmup": min(a.warmup, 5), "ms_per_step": round(res["plan"]["ms"], 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "u8",
        "data": "synthetic",
        "config": {"workload": "ckpt: EKO-237M V4 image, 816 records", "image_bytes": nb,
                   "timing": "value and ms_per_step: pack-plan runs queued back to back "
                             "(ark_ckpt_v4_pack_plan_run, header + data kernels, HIP events); "
                             "pack_call_* and unpack_*: one ark_ckpt_v4_pack / "
                             "ark_ckpt_v4_unpack call each (table upload, kernels, host wait)",
                   "pack_call_ms": round(res["pack"]["ms"], 4),
                   "pack_call_GBs": round(pk_call, 2),
                   "unpack_ms": round(res["unpack"]["ms"], 4), "unpack_GBs": round(up, 2),
                   "pack_call_wall_ms": round(res["pack"]["wall_ms"], 3),
                   "save_file_s": round(save_s, 3), "save_file_GBs": round(nb / save_s / 1e9, 2),
                   "load_file_s": round(load_s, 3), "load_file_GBs": round(nb / load_s / 1e9, 2),
                   "file_dir": d},
        "roofline": {"kernel": "pack_kernel", "bound": "hbm", "achieved": round(pk, 2),
                     "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(pk / PEAK_HBM_GBS, 4),
                     "traffic": traffic_from_profiles("eko237m", "pack_kernel")[0],
                     "traffic_source": traffic_from_profiles("eko237m", "pack_kernel")[1],
                     "algorithmic_bytes_per_launch": 2 * nb},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


def run_grad(a):
    """The gradient hand-off of EKO-237M (include/ark_grad.h): one launch
    adding all 272 backward outputs into the fp32 gradients (12 B/param:
    two reads, one write), and the token scatter of a 2 x 2048-token batch
    (config.rs:62-67) into the 32000 x 768 embedding gradient."""
    import numpy as np
    import torch
    from ark_amd import grad
    from ark_amd.eko import EKO_237M
    torch.cuda.set_device(0)
    specs = EKO_237M.tensors()
    n = sum(s.n for s in specs)
    g = torch.Generator(device="cuda").manual_seed(SEED)
    dst = [torch.randn(s.n, device="cuda", generator=g) for s in specs]
    src = [torch.randn(s.n, device="cuda", generator=g) for s in specs]
    plan = grad.GradPlan(list(zip(dst, src)))
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for _ in range(a.warmup):
        plan.run()
    torch.cuda.synchronize()
    e0.record()
    for _ in range(a.steps):
        plan.run()
    e1.record()
    torch.cuda.synchronize()
    acc_ms = e0.elapsed_time(e1) / a.steps
    plan.close()
    vocab, d, bs = 32000, 768, 4096
    rng = np.random.default_rng(SEED)
    tokens = torch.from_numpy(((rng.zipf(1.2, bs) - 1) % vocab).astype(np.int32)).cuda()
    dx0 = torch.randn(bs, d, device="cuda", generator=g)
    eg = dst[0].view(vocab, d)

    def time_scatter(tok, rows, noalloc=False):
        for _ in range(a.warmup):
            grad.embed_scatter(eg, tok, rows, noalloc=noalloc)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(a.steps):
            grad.embed_scatter(eg, tok, rows, noalloc=noalloc)
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / a.steps

    sc_ms = time_scatter(tokens, dx0)
    sc_na_ms = time_scatter(tokens, dx0, noalloc=True)
    big = 4 * bs  # four tiles: the multi-block sort
    tokens4 = torch.from_numpy(((rng.zipf(1.2, big) - 1) % vocab).astype(np.int32)).cuda()
    dx4 = torch.randn(big, d, device="cuda", generator=g)
    sc4_ms = time_scatter(tokens4, dx4)
    uniq = int(torch.unique(tokens).numel())
    cpu = None
    if not a.no_cpu:
        import oracle
        from concurrent.futures import ThreadPoolExecutor
        th = a.cpu_threads or min(16, os.cpu_count() or 1)
        hd = dst[0].cpu().numpy()
        hs = src[0].cpu().numpy()
        parts = list(zip(np.array_split(hd, th), np.array_split(hs, th)))
        reps, t0 = 0, time.perf_counter()
        with ThreadPoolExecutor(th) as ex:
            while time.perf_counter() - t0 < min(a.cpu_seconds, 10.0):
                list(ex.map(lambda p: oracle.grad_accumulate(*p), parts))
                reps += 1
        el = time.perf_counter() - t0
        cpu = dict(value=round(12 * hd.size * reps / el / 1e9, 3), unit="GB/s", cores=th,
                   kind="port", sample=f"{reps} accumulations of the {hd.size}-element "
                   f"embedding gradient in {el:.1f} s on {th} threads")
    gbs = 12 * n / (acc_ms * 1e-3) / 1e9
    out = {
        "metric": "EKO-237M gradient accumulation (all tensors, fp32 +=) GB/s (1 GPU)",
        "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": round(acc_ms, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "grad: 272 EKO-237M fp32 gradient buffers += backward outputs; "
                               "token scatter of 4096 tokens (Zipf 1.2) into 32000 x 768",
                   "elements": n, "bytes_per_launch": 12 * n,
                   "scatter_ms": round(sc_ms, 4), "scatter_unique_tokens": uniq,
                   "scatter_noalloc_ms": round(sc_na_ms, 4),
                   "scatter_16384_tokens_ms": round(sc4_ms, 4)},
        "roofline": {"kernel": "grad_batch", "bound": "hbm", "achieved": round(gbs, 2),
                     "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4),
                     "traffic": traffic_from_profiles("eko237m", "grad_batch")[0],
                     "traffic_source": traffic_from_profiles("eko237m", "grad_batch")[1],
                     "algorithmic_bytes_per_launch": 12 * n},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


def run_dropin(a):
    """The reference's own call pattern on the device: Optimizer::step_all
    calls ark_asm_adam_step_f16 once per tensor (optimizer.rs:185-227), so
    here ark_hip_adam_step_f16 is launched 272 times per step over EKO-237M
    with fp32 gradients (24 B/param: g 4, w 2+2, m 4+4, v 4+4), no unscale
    or clip.  One step's launches are captured in a HIP graph and replayed,
    so the figure is the kernels', not Python's launch loop.  With --weights
    f32 the same pattern runs ark_hip_adam_step (ark_asm_adam_step,
    opti.s:20-177) over fp32 copies of the weights: 28 B/param (g 4, w 4+4,
    m 4+4, v 4+4)."""
    import ctypes as C
    import numpy as np
    import torch
    from ark_amd import _abi, synth
    from ark_amd._lib import check, lib
    from ark_amd.eko import EKO_237M
    torch.cuda.set_device(0)
    stream = torch.cuda.Stream()
    specs = EKO_237M.tensors()
    with torch.cuda.stream(stream):
        ps = synth.problem(specs, SEED, HP["weight_decay"], [1e-3] * len(specs), 1.0,
                           grad_dtype=_abi.GRAD_F32)
        w32 = [ps.w(i).float() for i in range(len(specs))] if a.weights == "f32" else None
    n = ps.n_params
    L = lib()
    sp = C.c_void_p(stream.cuda_stream)
    fn, bpp, kname, entry = ((L.ark_hip_adam_step, 28, "adamw_single_w32_kernel",
                              "ark_hip_adam_step") if w32 else
                             (L.ark_hip_adam_step_f16, 24, "adamw_single_kernel",
                              "ark_hip_adam_step_f16"))
    calls = [((w32[i] if w32 else ps.w(i)).data_ptr(), ps.g(i).data_ptr(), ps.m(i).data_ptr(),
              ps.v(i).data_ptr(), s.n, HP["weight_decay"] if s.decay else 0.0)
             for i, s in enumerate(specs)]

    def step(t):
        for w, g, m, v, nn, wd in calls:
            rc = fn(w, g, m, v, nn, HP["lr"], HP["beta1"], HP["beta2"], HP["eps"], wd, t, sp)
            if rc:
                check(rc)

    with torch.cuda.stream(stream):
        for t in range(1, 3):
            step(t)
    stream.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        step(3)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        for _ in range(a.warmup):
            graph.replay()
        e0.record(stream)
        for _ in range(a.steps):
            graph.replay()
        e1.record(stream)
    stream.synchronize()
    ms = e0.elapsed_time(e1) / a.steps
    del graph
    cpu = None
    if not a.no_cpu:
        import oracle
        from concurrent.futures import ThreadPoolExecutor
        th = a.cpu_threads or min(16, os.cpu_count() or 1)
        e = [s.name for s in specs].index("embed")
        hg = ps.g(e).cpu().numpy().copy()
        if w32:
            hw = w32[e].cpu().numpy().copy()
            ref = oracle.adam_step_f32
        else:
            hw = ps.w(e).view(torch.int16).cpu().numpy().view(np.uint16).copy()
            ref = oracle.adam_step_f16
        hm, hv = np.zeros_like(hg), np.zeros_like(hg)
        parts = list(zip(*(np.array_split(x, th) for x in (hw, hg, hm, hv))))
        reps, t0 = 0, time.perf_counter()
        with ThreadPoolExecutor(th) as ex:
            while time.perf_counter() - t0 < min(a.cpu_seconds, 10.0):
                list(ex.map(lambda p: ref(*p, HP["lr"], HP["beta1"], HP["beta2"], HP["eps"],
                                          HP["weight_decay"], 3), parts))
                reps += 1
        el = time.perf_counter() - t0
        cpu = dict(value=round(bpp * hw.size * reps / el / 1e9, 3), unit="GB/s", cores=th,
                   kind="port", sample=f"{reps} {entry.replace('hip', 'asm')} restatements over "
                   f"the {hw.size}-element embedding in {el:.1f} s on {th} threads")
    gbs = bpp * n / (ms * 1e-3) / 1e9
    wdesc = "fp32 weights" if w32 else "fp16 weights"
    out = {
        "metric": f"EKO-237M reference call pattern: 272 {entry} launches per step, "
                  "GB/s (1 GPU)",
        "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": f"dropin: 272 single-tensor launches over EKO-237M, {wdesc}, "
                               "fp32 gradients, replayed as one HIP graph",
                   "params": n, "bytes_per_step": bpp * n},
        "roofline": {"kernel": kname, "bound": "hbm", "achieved": round(gbs, 2),
                     "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4),
                     "traffic": None, "algorithmic_bytes_per_launch": bpp * n},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


def run_clip(a):
    """The drop-in for ark_asm_grad_clip (opti.s:369-432) on the largest
    gradient its reference wrapper would take, the 24,576,000-value tied
    embedding of EKO-237M (fp32): calls queued back to back on one stream
    (no host wait), every one clipping (threshold -1: 0 < norm, so each call
    scales by -1 / norm and the norm stays 1; 4 B read for the norm, 4 B
    read and written for the scale = 12 B/value) and, separately, none
    clipping (4 B/value).  HIP events on the call's stream."""
    import ctypes as C
    import torch
    from ark_amd._lib import check, lib
    torch.cuda.set_device(0)
    stream = torch.cuda.Stream()
    n = 32000 * 768
    with torch.cuda.stream(stream):
        g = torch.randn(n, device="cuda") * 1e-3
    L = lib()
    sp = C.c_void_p(stream.cuda_stream)

    def timed(thr):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(stream):
            for _ in range(a.warmup):
                check(L.ark_hip_grad_clip(g.data_ptr(), n, thr, None, sp))
            e0.record(stream)
            for _ in range(a.steps):
                check(L.ark_hip_grad_clip(g.data_ptr(), n, thr, None, sp))
            e1.record(stream)
        stream.synchronize()
        return e0.elapsed_time(e1) / a.steps

    ms_clip = timed(-1.0)
    ms_keep = timed(1e30)
    norm = C.c_float()
    t0 = time.perf_counter()
    for _ in range(20):
        check(L.ark_hip_grad_clip(g.data_ptr(), n, 1e30, C.byref(norm), sp))
    ms_wait = (time.perf_counter() - t0) * 1e3 / 20
    cpu = None
    if not a.no_cpu:
        import oracle
        h = g.cpu().numpy().copy()
        reps, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < min(a.cpu_seconds, 10.0):
            oracle.grad_clip_literal(h, -1.0)
            reps += 1
        el = time.perf_counter() - t0
        cpu = dict(value=round(12 * n * reps / el / 1e9, 3), unit="GB/s", cores=1, kind="port",
                   ms_per_call=round(el * 1e3 / reps, 3),
                   sample=f"{reps} clipping calls of the instruction-by-instruction restatement "
                          f"of ark_asm_grad_clip (four serial fp32 chains, one thread, as the "
                          f"reference runs) over the {n}-value embedding gradient in {el:.1f} s")
    gbs = 12 * n / (ms_clip * 1e-3) / 1e9
    traffic, tsrc = traffic_from_profiles("eko237m_embed", "clip_kernels")
    out = {
        "metric": "ark_asm_grad_clip drop-in on the EKO-237M embedding gradient, GB/s (1 GPU)",
        "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": round(ms_clip, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": f"clip: one ark_hip_grad_clip call per step over {n} fp32 values "
                               "(the tied embedding's gradient), every call clipping",
                   "params": n, "bytes_per_step": 12 * n,
                   "ms_per_call_not_clipping": round(ms_keep, 4),
                   "gbs_not_clipping": round(4 * n / (ms_keep * 1e-3) / 1e9, 2),
                   "ms_per_call_reporting_the_norm": round(ms_wait, 4)},
        "roofline": {"kernel": "clip_norm_kernel + clip_scale_kernel", "bound": "hbm",
                     "achieved": round(gbs, 2), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": traffic,
                     "traffic_source": tsrc, "algorithmic_bytes_per_launch": 12 * n},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="c2", choices=sorted(WORKLOADS))
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--cpu-threads", type=int, default=0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--path", default="step",
                    choices=["step", "codec", "ckpt", "grad", "dropin", "ceiling", "clip"],
                    help="step: the optimizer step (headline); codec: the weight codec; "
                         "ckpt: the V4 checkpoint image; grad: the gradient hand-off; "
                         "dropin: the reference's 272 single-tensor calls per step; "
                         "ceiling: the AdamW pass's access pattern without its arithmetic; "
                         "clip: the per-tensor clip drop-in on the embedding gradient")
    ap.add_argument("--grad", default="f16", choices=["f16", "f32", "f32-fused"],
                    help="step: gradient type handed to the step (f16 loss-scaled, as the benchmark "
                         "configurations; f32, as the gradient hand-off produces; f32-fused, "
                         "produced by the hand-off's final accumulation, which also forms the "
                         "norm's first level so the step does not re-read the gradients)")
    ap.add_argument("--weights", default="f16", choices=["f16", "f32"],
                    help="dropin: fp16 weights (ark_hip_adam_step_f16, the trainer's call) or "
                         "fp32 weights (ark_hip_adam_step)")
    ap.add_argument("--calib-copy", action="store_true",
                    help="also run a 1 GiB device-to-device copy (counter calibration)")
    ap.add_argument("--no-secondary", action="store_true",
                    help="c2 headline only: without the skipped-step (c3) and 1.3B (c4) figures "
                         "the default line also carries")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: the optimizer step of this build runs on a "
              "single MI355X (no collectives); run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    if a.path != "step":
        {"codec": run_codec, "ckpt": run_ckpt, "grad": run_grad, "dropin": run_dropin,
         "ceiling": run_ceiling, "clip": run_clip}[a.path](a)
        if a.calib_copy:
            calib_copy()
        return

    # the default line (c2, fp16 gradients) also carries the secondary
    # configurations: a skipped step (c3's set is c2's, so the c2 handle
    # times it) and the 1.3B scale-up (c4)
    secondary = a.workload == "c2" and a.grad == "f16" and not a.no_secondary
    r = run_gpu(a.workload, a.steps, a.warmup, a.grad, skip=secondary)
    c4 = secondary_c4(a.steps, a.warmup) if secondary else None
    if a.calib_copy:
        calib_copy()
    n = r["n_params"]
    b_step, b_adamw = step_bytes(a.grad)
    gbs = b_step * n / (r["ms_step"] * 1e-3) / 1e9
    adam_gbs = b_adamw * n / (r["ms_adamw"] * 1e-3) / 1e9
    traffic, tsrc = traffic_from_profiles(a.workload) if a.grad == "f16" else (None, None)
    cpu = None
    if not a.no_cpu:
        th = a.cpu_threads or min(16, os.cpu_count() or 1)
        log(f"[bench] cpu baseline: {th} threads, ~{a.cpu_seconds}s")
        cpu = run_cpu_baseline(a.workload, a.cpu_seconds, th,
                               "f32" if a.grad == "f32-fused" else a.grad)
    out = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(r["ms_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded counter-based generator on the device)",
        "config": {
            "workload": f"{a.workload}: {WORKLOADS[a.workload]['desc']}",
            "params": n,
            "tensors": r["n_tensors"],
            "storage": f"w fp16, g {a.grad[:3]} (loss-scaled), m/v fp32",
            "bytes_per_step": b_step * n,
            "hparams": HP,
            "loss_scale": WORKLOADS[a.workload]["loss_scale"],
            "clipped": r["clipped"],
            "grad_norm": r["grad_norm"],
            "hip_graph_ms_per_step": (round(r["graph_ms"], 4) if r["graph_ms"] is not None
                                      else None),
        },
        "frac_of_peak_hbm": round(gbs / PEAK_HBM_GBS, 4),
        "kernels_ms": {"sumsq": round(r["ms_norm"], 4), "finalize": round(r["ms_finalize"], 4),
                       "adamw": round(r["ms_adamw"], 4), "step_events": round(r["ms_step_events"], 4)},
        "roofline": {
            "kernel": "adamw_kernel",
            "bound": "hbm",
            "achieved": round(adam_gbs, 2),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(adam_gbs / PEAK_HBM_GBS, 4),
            "traffic": traffic,
            "traffic_source": tsrc,
            "algorithmic_bytes_per_launch": b_adamw * n,
        },
        "cpu_baseline": cpu,
    }
    if secondary:
        out["secondary"] = {
            "c3_skipped_step": dict(
                r["skip"], workload="c3: the c2 set with +inf in one fp16 gradient",
                bytes_per_skipped_step=2 * n,
                note="the norm pass reads g (2 B/param) and flags it, the finalize skips and "
                     "halves the loss scale, the AdamW pass exits before any access; the rest "
                     "of the wall clock is that exiting launch's dispatch (kernel trace: "
                     "profiles/adamw_kernel_c3.md)"),
            "c4": c4,
        }
    elif r.get("skip"):
        out["config"]["skipped_steps"] = dict(
            r["skip"], ms_per_applied_step=round(r["ms_step"], 4),
            bytes_per_skipped_step=2 * n,
            note="an inf in one gradient: the norm pass reads g (2 B/param) and flags it, the "
            "finalize skips, the AdamW pass exits before any access")
    if a.grad == "f32-fused":
        out["config"]["fused_norm"] = dict(
            r["fused"], note="ms_per_step: the step after the gradient plan's final "
            "accumulation wrote the norm's units = pair_ms (accumulate + step, wall clock) - "
            "producer_ms (the accumulation, HIP events); plain_*: the same with the plain "
            "accumulation and the step that reads the gradients for its norm")
        out["kernels_ms"]["units_reduce"] = out["kernels_ms"].pop("sumsq")
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
