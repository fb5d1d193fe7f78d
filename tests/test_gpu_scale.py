"""GPU parity at the benchmark configurations' full sizes: the EKO-237M set
(c2), its 5000-step AMP stress trajectory (c3) and the 1.3B scale-up (c4),
checked against the CPU oracle bit for bit (every scalar and every w/m/v
element of the steps run), plus the state/restore and timing entry points."""
import ctypes as C
import os

import numpy as np
import pytest

import oracle
from oracle import harness as H
from ark_amd import _abi
from ark_amd.eko import config_tensors

pytestmark = pytest.mark.gpu

HP = dict(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1, grad_clip=1.0)
THREADS = min(16, os.cpu_count() or 1)


def _opt(ps, scale, **amp_kw):
    from ark_amd.optimizer import AdamConfig, AmpConfig, Optimizer
    cfg = AdamConfig(**HP)
    amp = AmpConfig(**{"loss_scale_init": scale, "loss_scale_max": 2.0 ** 24, **amp_kw})
    return cfg, Optimizer(cfg, ps, amp)


def _full_size_steps(name, sig, scale, steps, seed, sig_at=None):
    """steps fresh-gradient steps on the GPU and the oracle, every scalar and
    every w/m/v element compared after each; sig_at(k) gives step k's
    per-tensor sigmas (default: sig throughout)."""
    specs = config_tensors(name)
    sig_at = sig_at or (lambda k: sig)
    ps = H.gpu_problem(specs, seed, HP["weight_decay"], sig_at(0), scale)
    cfg, opt = _opt(ps, scale)
    ts = H.host_problem(specs, seed, HP["weight_decay"], sig_at(0), scale, nthreads=THREADS)
    ref = oracle.Optimizer(ts, opt.hp, nthreads=THREADS)
    infos = []
    for k in range(steps):
        if k:
            H.gpu_regen_grads(ps, seed, sig_at(k), scale, k)
            H.host_regen_grads(ts, seed, sig_at(k), scale, k, nthreads=THREADS)
        _, gi = opt.step_all(cfg.lr, info=True)
        _, ri = ref.step(cfg.lr)
        assert not H.info_matches(gi, ri), (k, H.info_matches(gi, ri))
        c = H.compare(ps, ts, nthreads=THREADS)
        assert c["w"] == c["m"] == c["v"] == 0, (k, c)
        infos.append(gi)
    opt.close()
    return infos


def test_config2_eko237m_full_size_bit_exact():
    """272 tensors, 236,959,488 params, per-tensor sigma = 10^U(-5,-2),
    loss scale 65536: two steps (fresh gradients), every element compared."""
    specs = config_tensors("c2")
    sig = H.log_uniform_sigmas(len(specs), 20260501)
    infos = _full_size_steps("c2", sig, 65536.0, 2, 20260501)
    assert all(i.applied for i in infos) and infos[-1].state.t == 2


def test_config2_full_size_at_a_scale_that_is_not_a_power_of_two():
    """The same set at loss scale 49152 (1.5 x 2^15): the norm pass then
    unscales each element before squaring instead of taking the squares from
    the fp16 bits, over both its cache-allocating and its streaming blocks
    (tables past ~134M elements have both).  Two steps, every element
    compared."""
    specs = config_tensors("c2")
    sig = H.log_uniform_sigmas(len(specs), 20260503)
    infos = _full_size_steps("c2", sig, 49152.0, 2, 20260503)
    assert all(i.applied for i in infos) and infos[-1].state.t == 2
    assert infos[-1].inv_scale == np.float32(1.0) / np.float32(49152.0)


def test_config2_full_size_both_clip_branches():
    """The c2 benchmark's sigma = 10^U(-5,-2) gives a global norm of about 35.8, so
    every c2 step clips.  The same 272-tensor set with those sigmas scaled to
    put the norm at 0.9, 1.1 and 0.95 x grad_clip on three fresh-gradient
    steps takes both branches of optimizer.rs:145-149 (unclipped, clipped,
    unclipped) at full size, every element compared with the oracle."""
    specs = config_tensors("c2")
    base = H.log_uniform_sigmas(len(specs), 20260501)
    est = float(np.sqrt(sum(s.n * float(x) ** 2 for s, x in zip(specs, base))))
    assert 30.0 < est < 40.0, est
    factors = [0.9, 1.1, 0.95]
    sigs = [[float(x) * f / est for x in base] for f in factors]
    infos = _full_size_steps("c2", None, 65536.0, 3, 20260502, sig_at=lambda k: sigs[k])
    assert [i.applied for i in infos] == [1, 1, 1]
    assert [i.clipped for i in infos] == [0, 1, 0], [i.grad_norm for i in infos]
    for i, f in zip(infos, factors):
        assert abs(i.grad_norm / HP["grad_clip"] - f) < 0.02, (i.grad_norm, f)


def test_config4_scaleup_full_size_bit_exact():
    """218 tensors, 1,279,887,360 params, sigma 1e-3, loss scale 65536: one
    step, every element compared."""
    specs = config_tensors("c4")
    infos = _full_size_steps("c4", [1e-3] * len(specs), 65536.0, 1, 7)
    assert infos[0].applied == 1


def _c3_poke_plan(specs, steps, seed):
    """The c3 injection schedule: on ~0.1 % of steps (seeded) plus the fixed
    steps 1500, 1501 (two in a row) and 2100 (mid-recovery), +inf, -inf or
    NaN at 1-16 seeded positions of seeded tensors.  {step: [(tensor,
    position, fp16 bits)]}."""
    rng = np.random.default_rng(seed)
    bad = np.union1d(np.nonzero(rng.random(steps) < 0.001)[0], [1500, 1501, 2100])
    specials = (0x7C00, 0xFC00, 0x7E00)
    plan = {}
    for k in bad.tolist():
        plan[k] = []
        for _ in range(int(rng.integers(1, 17))):
            ti = int(rng.integers(len(specs)))
            plan[k].append((ti, int(rng.integers(specs[ti].n)), specials[int(rng.integers(3))]))
    return plan


def _sample(specs, ts, seed, embed_stride, w2_stride):
    """The elements a long run follows through every step: every element of
    gamma_final, of every g1 and g2, and of one seeded d x d tensor; a
    seeded strided sample of the embedding and of every layer's w2.
    [(tensor index, element indices)] and the matching oracle HostTensors
    (their own copies, from `ts`)."""
    rng = np.random.default_rng(seed)
    names = [s.name for s in specs]
    square = [i for i, s in enumerate(specs) if s.name.endswith((".wq", ".wk", ".wv", ".wo"))]
    picks = [(names.index("gamma_final"), None), (int(rng.choice(square)), None)]
    picks += [(i, None) for i, s in enumerate(specs) if s.name.endswith((".g1", ".g2"))]
    picks.append((names.index("embed"), embed_stride))
    picks += [(i, w2_stride) for i, s in enumerate(specs) if s.name.endswith(".w2")]
    sample, host = [], []
    for i, stride in picks:
        idx = (np.arange(specs[i].n, dtype=np.int64) if stride is None else
               np.arange(int(rng.integers(stride)), specs[i].n, stride, dtype=np.int64))
        t = ts[i]
        sample.append((i, idx))
        host.append(oracle.HostTensor(t.w[idx].copy(), t.g[idx].copy(), t.m[idx].copy(),
                                      t.v[idx].copy(), t.weight_decay, t.flags))
    return sample, host


def _long_run(name, steps, seed, sig, scale, plan, strides, grad_dtype=_abi.GRAD_F16):
    """`steps` steps of configuration `name` with its gradients fixed from
    step 0 and the injections of `plan` ({step: [(tensor, position, fp16
    bits)]}) planted before each step and removed after it.  Every step's
    scalars -- skip decision, canonical sum of squares, norm, clip
    coefficient, inv_scale, lr_eff, t, loss scale and counters -- are
    compared bit for bit with the oracle's own: its sum of squares over the
    host copy of the gradients once per distinct loss scale, its finite
    check over the poked tensors, its state machine (ark_ref_finalize).  The
    oracle then runs the elementwise update of every applied step, with its
    own scalars, over the elements of _sample(strides), and after the last
    step those w/m/v elements on the device must equal its bits.  The oracle
    side runs on a host thread while the device steps.  grad_dtype: fp16
    (the benchmark configurations) or fp32 gradients (the reference's own
    type; no injections then).  Returns the device step infos."""
    import threading
    import torch
    specs = config_tensors(name)
    lr = HP["lr"]
    assert grad_dtype == _abi.GRAD_F16 or not plan
    ps = H.gpu_problem(specs, seed, HP["weight_decay"], sig, scale, grad_dtype=grad_dtype)
    cfg, opt = _opt(ps, scale)
    ts = H.host_problem(specs, seed, HP["weight_decay"], sig, scale, grad_dtype=grad_dtype,
                        nthreads=THREADS)
    sample, host = _sample(specs, ts, 31, *strides)
    ref_info = [None] * steps
    failure = []

    def oracle_side():
        try:
            st = _abi.State()
            oracle.lib().ark_ref_state_init(opt.hp, st)
            sums = {}
            sub = oracle.Optimizer(host, opt.hp, nthreads=THREADS)
            for k in range(steps):
                if k in plan:
                    hit = sorted({ti for ti, _, _ in plan[k]})
                    poked = [ts[ti].copy() for ti in hit]
                    for ti, pos, bits in plan[k]:
                        poked[hit.index(ti)].g[pos] = bits
                    sq, bad = oracle.sumsq(poked, _abi.GRAD_F16, 1.0, nthreads=THREADS)
                    assert bad, k
                else:
                    scale_k = float(st.loss_scale)
                    if scale_k not in sums:
                        inv = np.float32(1.0) / np.float32(scale_k)
                        sums[scale_k] = oracle.sumsq(ts, grad_dtype, inv, nthreads=THREADS)
                    sq, bad = sums[scale_k]
                    assert not bad, k
                _, ri = oracle.finalize(opt.hp, st, sq, bad, lr)
                if ri.applied:
                    sub.apply_given(lr, st.t, ri)
                ref_info[k] = ri
        except BaseException as e:  # reported on the main thread
            failure.append(e)

    worker = threading.Thread(target=oracle_side)
    worker.start()
    g16 = [ps.g(i).view(torch.int16) for i in range(len(specs))]
    dev_info = []
    for k in range(steps):
        undo = []
        for ti, pos, bits in plan.get(k, ()):
            undo.append((ti, pos, int(g16[ti][pos].item())))
            g16[ti][pos] = int(np.array(bits, np.uint16).view(np.int16))
        _, gi = opt.step_all(lr, info=True)
        dev_info.append(gi)
        for ti, pos, old in reversed(undo):
            g16[ti][pos] = old
    worker.join()
    assert not failure, failure
    for k in range(steps):
        d = H.info_matches(dev_info[k], ref_info[k])
        assert not d, (k, d)
        assert dev_info[k].applied == (k not in plan), k
    assert sum(idx.size for _, idx in sample) > 2_000_000
    for (i, idx), h in zip(sample, host):
        at = torch.from_numpy(idx).cuda()
        w = H.to_host(ps.w(i)[at])
        m = H.to_host(ps.m(i)[at])
        v = H.to_host(ps.v(i)[at])
        assert not H.bits_differ16(w, h.w).any(), (specs[i].name, "w")
        assert not H.bits_differ32(m, h.m).any(), (specs[i].name, "m")
        assert not H.bits_differ32(v, h.v).any(), (specs[i].name, "v")
    opt.close()
    return dev_info


def test_config3_amp_stress_5000_steps_scalars_and_elements():
    """EKO-237M, 5000 steps from scale 65536 (cap 2^24), gradients fixed from
    step 0, with the seeded injections of _c3_poke_plan (five random events
    at this seed, plus the three fixed ones), through _long_run: every
    step's scalars against the oracle's own, and after step 5000 gamma_final,
    every g1/g2, one 768 x 768 tensor and strided samples of the embedding
    (~1.07M) and of every w2 (~38k each) against the oracle's run of those
    elements (2.86M in all)."""
    specs = config_tensors("c3")
    steps, seed = 5000, 3
    plan = _c3_poke_plan(specs, steps, 2156)
    assert sorted(plan) == [15, 287, 813, 1500, 1501, 2100, 2778, 4993]
    dev_info = _long_run("c3", steps, seed, H.log_uniform_sigmas(len(specs), seed), 65536.0,
                         plan, (23, 41))
    scales = [i.state.loss_scale for i in dev_info]
    last = dev_info[-1].state
    assert last.t == steps - 8 and last.skipped_steps == 8
    # 65536 halved by the seven skips up to 2778 to 512; 2000 clean steps
    # later (4778) it doubles to 1024; the skip at 4993 halves it again
    assert min(scales) == 512.0 and scales[4777] == 512.0 and scales[4778] == 1024.0
    assert scales[-1] == 512.0
    assert all(i.clipped for i in dev_info if i.applied)


def test_config2_200_steps_as_the_bench_runs_them():
    """Configuration c2 exactly as bench.py builds it (seed 20260501, per-tensor
    sigma = 10^U(-5,-2) from that seed, loss scale 65536): one fused step
    repeated 200 times on fixed gradients, through _long_run: every step's
    scalars against the oracle's own, and after step 200 2.86M sampled
    elements against the oracle's run of them."""
    specs = config_tensors("c2")
    seed = 20260501
    dev_info = _long_run("c2", 200, seed, H.log_uniform_sigmas(len(specs), seed), 65536.0, {},
                         (23, 41))
    assert all(i.applied and i.clipped for i in dev_info)
    assert dev_info[-1].state.t == 200


def test_config2_fp32_gradients_200_steps():
    """The c2 set with the reference's own gradient type (fp32,
    memory.rs:239-243; the step reads 4 B/param for its norm and AdamW):
    200 steps on fixed gradients N(0, sigma_t) x 65536, through _long_run:
    every step's scalars against the oracle's own and, after step 200,
    2.86M sampled elements against the oracle's run of them."""
    specs = config_tensors("c2")
    seed = 20260504
    dev_info = _long_run("c2", 200, seed, H.log_uniform_sigmas(len(specs), seed), 65536.0, {},
                         (23, 41), grad_dtype=_abi.GRAD_F32)
    assert all(i.applied and i.clipped for i in dev_info)
    assert dev_info[-1].state.t == 200


def test_config4_scaleup_50_steps_scalars_and_elements():
    """Configuration c4 as the bench runs it: the 1.3B set (218 tensors,
    1,279,887,360 params), fp16 gradients N(0, 1e-3) x 65536 fixed from step
    0, 50 fused steps, through _long_run: every step's scalars against the
    oracle's own, and after step 50 gamma_final, every g1/g2, one 2048 x 2048
    tensor and strided samples of the embedding (~1.07M of 65.5M) and of
    every w2 (~37.6k of 11.3M each) against the oracle's run of those
    elements (6.3M in all)."""
    specs = config_tensors("c4")
    dev_info = _long_run("c4", 50, 7, [1e-3] * len(specs), 65536.0, {}, (61, 300))
    assert all(i.applied and i.clipped for i in dev_info)
    assert dev_info[-1].state.t == 50 and dev_info[-1].state.loss_scale == 65536.0


def test_state_set_get_and_restaurar_momentos():
    """restaurar_momentos (optimizer.rs:237-313) on a small EKO set: moments
    copied in checkpoint order, step set; wrong counts or sizes keep the
    step, as the reference does."""
    import torch
    from ark_amd.eko import EkoConfig
    specs = EkoConfig(n_layers=2, d_model=64, hidden=128, vocab=100).tensors()
    ps = H.gpu_problem(specs, 1, 0.1, [1e-3] * len(specs), 1024.0)
    cfg, opt = _opt(ps, 1024.0)
    names = [s.name for s in specs]
    layers = [i for i, s in enumerate(specs) if s.name not in ("embed", "gamma_final")]
    order = [names.index("embed")] + layers + [names.index("gamma_final")]
    rng = np.random.default_rng(0)
    mm = [rng.random(specs[i].n).astype(np.float32) for i in order]
    vv = [rng.random(specs[i].n).astype(np.float32) for i in order]
    assert opt.restaurar_momentos(mm[:-2], vv[:-2], 77) is False       # wrong count
    assert opt.step == 0
    assert opt.restaurar_momentos(mm, vv, 1234) is True                # 1 + 9L + 1
    assert opt.step == 1234
    for k, i in enumerate(order):
        assert np.array_equal(ps.m(i).cpu().numpy(), mm[k])
        assert np.array_equal(ps.v(i).cpu().numpy(), vv[k])
    assert opt.restaurar_momentos(mm[:-1], vv[:-1], 99) is True        # legacy 271-style
    assert opt.step == 99
    bad = list(mm)
    bad[3] = bad[3][:-1]
    assert opt.restaurar_momentos(bad, vv, 5) is False                 # layer size mismatch
    assert opt.step == 99
    opt.set_state(loss_scale=4096.0, clean_steps=1999)
    _, info = opt.step_all(cfg.lr, info=True)
    assert info.state.t == 100 and info.state.loss_scale == 8192.0 and info.state.clean_steps == 0
    opt.close()


def test_timing_counts_every_kernel():
    specs = config_tensors("c1")
    ps = H.gpu_problem(specs, 1, 0.1, [1e-3] * len(specs), 1024.0)
    cfg, opt = _opt(ps, 1024.0)
    opt.set_timing(True)
    for _ in range(300):  # more than one event pool
        opt.step_all(cfg.lr)
    t = opt.get_timing()
    assert t.steps == 300 and t.ms_adamw > 0 and t.ms_norm > 0 and t.ms_finalize > 0
    assert t.ms_step >= t.ms_adamw
    opt.set_timing(False)
    opt.close()


def test_many_handles_create_and_destroy():
    specs = config_tensors("c0")
    ps = H.gpu_problem(specs, 1, 0.1, [1e-3], 1024.0)
    for _ in range(50):
        cfg, opt = _opt(ps, 1024.0)
        opt.step_all(cfg.lr)
        opt.close()


def _loaded_hip_runtime():
    """The HIP runtime this process already uses (torch's), by the path it was
    loaded from, so that dlopen returns that same library."""
    import torch
    torch.cuda.init()
    with open("/proc/self/maps") as f:
        paths = {ln.split()[-1] for ln in f if "libamdhip64.so" in ln}
    assert len(paths) == 1, paths
    hip = C.CDLL(paths.pop())
    hip.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
    hip.hipFree.argtypes = [C.c_void_p]
    return hip


def test_create_rejects_short_or_host_buffers():
    import torch
    from ark_amd._lib import ArkOptError
    from ark_amd.optimizer import AdamConfig, Optimizer, ParamSet
    specs = config_tensors("c0")
    ps = ParamSet(specs, 0.1)
    # A 16-element tensor whose w starts 16 bytes before the end of a 2 MiB
    # hipMalloc allocation (not torch's, whose cached segments can be larger
    # than the tensor), so it runs 16 bytes past it; its g, m and v sit
    # 512 KiB into their arenas, where that overrun cannot reach (the spans
    # are disjoint, so only the allocation check can refuse it).
    hip = _loaded_hip_runtime()
    tail = C.c_void_p()
    assert hip.hipMalloc(C.byref(tail), C.c_size_t(2 << 20)) == 0
    try:
        off = 512 << 10
        tab = (_abi.Tensor * 1)()
        tab[0].w = tail.value + (2 << 20) - 16
        tab[0].g = ps.g(0).data_ptr() + off
        tab[0].m = ps.m(0).data_ptr() + off
        tab[0].v = ps.v(0).data_ptr() + off
        tab[0].n = 16
        with pytest.raises(ArkOptError, match="w .*exceeds its allocation"):
            Optimizer(AdamConfig(), ps, table=tab)
        tab[0].w = tail.value
        Optimizer(AdamConfig(), ps, table=tab).close()  # the same table in bounds is accepted
    finally:
        torch.cuda.synchronize()
        assert hip.hipFree(tail) == 0
    host = np.zeros(16, np.float32)
    tab = ps.table()
    tab[0].m = host.ctypes.data
    with pytest.raises(ArkOptError, match="host memory|not memory known"):
        Optimizer(AdamConfig(), ps, table=tab)
