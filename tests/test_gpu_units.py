"""The step's norm from units written by the gradient producers
(ark_grad_plan_run_final, ark_grad_embed_scatter_final; include/ark_grad.h)
against the same step reading the gradients (ark_opt_step's own norm pass):
the global sum of squares must keep its bits, so every step scalar and every
w/m/v element of the two paths must be identical.  On the full EKO-237M
set both paths are also compared with the oracle's gradient loops and
optimizer (test_eko237m_fp32_gradients_both_paths_against_the_oracle); the
rest compares the two device paths with each other on ragged and unaligned
tables, with non-finite values entering through either producer, and on
misuse, the reading path's own agreement with the oracle being what
tests/test_gpu_parity.py and tests/test_gpu_grad.py establish."""
import numpy as np
import pytest

from ark_amd import _abi, grad
from ark_amd.eko import EKO_237M, EkoConfig, TensorSpec

pytestmark = pytest.mark.gpu

HP = dict(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1, grad_clip=1.0)


def _torch():
    import torch
    assert torch.cuda.is_available(), "GPU test run without a GPU"
    return torch


class _Run:
    """A ParamSet with fp32 gradients, its optimizer and a gradient plan over
    backward outputs `outs` (shared between runs)."""

    def __init__(self, specs, outs, scale, no_unscale=()):
        torch = _torch()
        from ark_amd.optimizer import AdamConfig, AmpConfig, Optimizer, ParamSet
        self.ps = ParamSet(specs, weight_decay=0.1, grad_dtype=_abi.GRAD_F32,
                           no_unscale=no_unscale)
        g = torch.Generator(device="cuda").manual_seed(5)
        for i, s in enumerate(specs):
            self.ps.w(i).copy_((torch.randn(s.n, device="cuda", generator=g) * 0.02).half())
        self.cfg = AdamConfig(**HP)
        self.opt = Optimizer(self.cfg, self.ps, AmpConfig(loss_scale_init=scale,
                                                          loss_scale_max=2.0 ** 24))
        self.plan = grad.GradPlan([(self.ps.g(i), outs[i]) for i in range(len(specs))])

    def step(self, specs, fused, scatter=None):
        """Zero the gradients, accumulate, scatter, step; returns the info."""
        for i in range(len(specs)):
            self.ps.g(i).zero_()
        self.plan.run(final_for=self.opt if fused else None)
        if scatter is not None:
            e, vocab, d, tokens, dx0 = scatter
            grad.embed_scatter(self.ps.g(e).view(vocab, d), tokens, dx0,
                               final_for=self.opt if fused else None)
        _, info = self.opt.step_all(self.cfg.lr, info=True)
        return info

    def close(self):
        self.plan.close()
        self.opt.close()


def _same(a, b, specs):
    torch = _torch()
    for i in range(len(specs)):
        for f in ("w", "m", "v"):
            x, y = getattr(a.ps, f)(i), getattr(b.ps, f)(i)
            assert torch.equal(x.view(torch.int16 if f == "w" else torch.int32),
                               y.view(torch.int16 if f == "w" else torch.int32)), (i, f)


def _info_eq(x, y):
    """Step scalars equal; floats compared as bits, NaN matching NaN."""
    def key(i):
        f = [np.float64(i.grad_sumsq), np.float32(i.grad_norm), np.float32(i.clip_coef)]
        return (i.applied, i.clipped) + tuple("nan" if np.isnan(v) else v.tobytes() for v in f)
    assert key(x) == key(y), (key(x), key(y))
    assert x.state.as_dict() == y.state.as_dict()


def _outs(specs, seed, sigma, scale):
    torch = _torch()
    g = torch.Generator(device="cuda").manual_seed(seed)
    return [torch.randn(s.n, device="cuda", generator=g) * (sigma * scale) for s in specs]


def test_eko237m_units_step_matches_the_reading_step():
    """All 272 EKO-237M tensors (d 768: the scatter's rows are whole units),
    a 2 x 2048-token Zipf scatter, gamma_final kept scaled (the reference's
    quirk flag): five fresh-gradient steps -- two clipped, one with an inf in
    a layer's backward output (skipped), one with a NaN entering through dx0
    (skipped), one unclipped."""
    torch = _torch()
    specs = EKO_237M.tensors()
    names = [s.name for s in specs]
    e = names.index("embed")
    scale = 65536.0
    outs = _outs(specs, 11, 1e-4, scale)
    runs = [_Run(specs, outs, scale, no_unscale=("gamma_final",)) for _ in range(2)]
    rng = np.random.default_rng(3)
    vocab, d, n = 32000, 768, 4096
    for k, (sig, bad_out, bad_dx) in enumerate([(1e-4, False, False), (1e-2, False, False),
                                                (1e-4, True, False), (1e-4, False, True),
                                                (3e-5, False, False)]):
        for o in outs:
            o.normal_(0.0, sig * scale)
        if bad_out:
            outs[names.index("l7.w2")][12345] = float("inf")
        tokens = torch.from_numpy(((rng.zipf(1.2, n) - 1) % vocab).astype(np.int32)).cuda()
        dx0 = torch.randn(n, d, device="cuda") * (sig * scale)
        if bad_dx:
            dx0[100, 5] = float("nan")
        infos = [r.step(specs, fused, (e, vocab, d, tokens, dx0))
                 for r, fused in zip(runs, (False, True))]
        _info_eq(infos[0], infos[1])
        assert infos[0].applied == (0 if (bad_out or bad_dx) else 1), k
        _same(runs[0], runs[1], specs)
    assert infos[0].state.t == 3
    for r in runs:
        r.close()


def test_eko237m_fp32_gradients_both_paths_against_the_oracle():
    """The reference's own gradient type (fp32, memory.rs:239-243) at full
    size: all 272 EKO-237M tensors, gradients zeroed (training.rs:248), then
    two accumulations of seeded backward outputs (bridge.m:910-915,
    :931-947) -- the second through ark_grad_plan_run_final on the units
    path -- and a 4096-token Zipf scatter at d 768 (bridge.m:922-928) --
    ark_grad_embed_scatter_final on the units path -- then one step.  Two
    fresh-gradient steps, the first clipped and the second not
    (optimizer.rs:145-149).  Each path's gradients, step scalars and every
    w/m/v element are compared bit for bit with the oracle's loops and
    optimizer on the host (training.rs:289-314), not only with each
    other."""
    torch = _torch()
    import oracle
    from ark_amd import synth
    from oracle import harness as H
    specs = EKO_237M.tensors()
    e = [s.name for s in specs].index("embed")
    vocab, d, n_tok = 32000, 768, 4096
    seed, scale, lr = 23, 65536.0, HP["lr"]
    base = synth.log_uniform_sigmas(len(specs), seed)
    est = float(np.sqrt(sum(s.n * float(x) ** 2 for s, x in zip(specs, base))))
    # step 0 as drawn (norm ~ 50: clips); step 1 scaled to a norm of ~0.6
    sigs = [base, [float(x) * 0.4 / est for x in base]]
    ps = [synth.problem(specs, seed, HP["weight_decay"], base, scale,
                        grad_dtype=_abi.GRAD_F32) for _ in range(2)]
    from ark_amd.optimizer import AdamConfig, AmpConfig, Optimizer
    cfg = AdamConfig(**HP)
    opts = [Optimizer(cfg, p, AmpConfig(loss_scale_init=scale, loss_scale_max=2.0 ** 24))
            for p in ps]
    outs = [torch.empty(s.n, dtype=torch.float32, device="cuda") for s in specs]
    plans = [grad.GradPlan([(p.g(i), outs[i]) for i in range(len(specs))]) for p in ps]
    ts = H.host_problem(specs, seed, HP["weight_decay"], base, scale,
                        grad_dtype=_abi.GRAD_F32, nthreads=8)
    ref = oracle.Optimizer(ts, opts[0].hp, nthreads=8)
    rng = np.random.default_rng(seed)
    for k in range(2):
        tokens = ((rng.zipf(1.2, n_tok) - 1) % vocab).astype(np.uint32)
        dx0 = (rng.standard_normal((n_tok, d)) * (sigs[k][e] * scale)).astype(np.float32)
        tok_d = torch.from_numpy(tokens.view(np.int32)).cuda()
        dx0_d = torch.from_numpy(dx0).cuda()
        for p in ps:
            for i in range(len(specs)):
                p.g(i).zero_()
        host_out = []
        for a in range(2):  # two accumulations, the backward outputs regenerated between
            st = 100 + 2 * k + a
            for i, s in enumerate(specs):
                ss = synth.grad_sigma_scale(sigs[k][i], scale)
                synth.normal_f32(outs[i], seed, i, st, ss)
            host_out.append(st)
            for p, plan, opt, fused in zip(ps, plans, opts, (False, True)):
                plan.run(final_for=opt if (fused and a == 1) else None)
        for p, opt, fused in zip(ps, opts, (False, True)):
            grad.embed_scatter(p.g(e).view(vocab, d), tok_d, dx0_d,
                               final_for=opt if fused else None)
        infos = [opt.step_all(lr, info=True)[1] for opt in opts]

        def host_grads(i):
            t = ts[i]
            t.g[:] = 0.0
            for st in host_out:
                oracle.grad_accumulate(t.g, oracle.synth_normal_f32(
                    t.n, seed, i, st, synth.grad_sigma_scale(sigs[k][i], scale)))
        H._pmap(host_grads, range(len(specs)), 8)
        oracle.embed_scatter(ts[e].g.reshape(vocab, d), tokens, dx0)
        _, ri = ref.step(lr)
        assert ri.applied == 1 and ri.clipped == (1 if k == 0 else 0), (k, ri.grad_norm)
        for name, p, gi in zip(("reading", "units"), ps, infos):
            diff = H.info_matches(gi, ri)
            assert not diff, (k, name, diff)
            c = H.compare(p, ts, nthreads=8)
            assert c["w"] == c["m"] == c["v"] == 0, (k, name, c)
        # the reading path's gradients are the oracle's loops' bit for bit
        # (the units path's are the same buffers' values; its step did not read them)
        for i in (e, 1, len(specs) - 1):
            assert np.array_equal(H.to_host(ps[0].g(i)).view(np.uint32),
                                  ts[i].g.view(np.uint32)), (k, specs[i].name)
    for plan in plans:
        plan.close()
    for opt in opts:
        opt.close()


def test_ragged_unaligned_tables_and_small_norm_blocks():
    """Tensors of 1, 255, 256, 257, 4095, 4097 and 9000 elements (units
    partly and wholly past a segment's end), a backward output that is only
    4-byte aligned (the scalar path), a no-unscale tensor, and tables small
    enough that the norm blocks hold 1, 2 or 4 segments."""
    torch = _torch()
    for sizes in ([1, 255, 256, 257, 4095, 4097, 9000], [5000] * 3, [4096] * 40, [300] * 200):
        specs = [TensorSpec(f"t{i}", (n,), True, False) for i, n in enumerate(sizes)]
        outs = _outs(specs, len(sizes), 1e-3, 1024.0)
        base = torch.randn(sizes[0] + 1, device="cuda")
        outs[0] = base[1:]  # 4-byte aligned only
        runs = [_Run(specs, outs, 1024.0, no_unscale=(specs[-1].name,)) for _ in range(2)]
        for k in range(3):
            infos = [r.step(specs, fused) for r, fused in zip(runs, (False, True))]
            _info_eq(infos[0], infos[1])
            _same(runs[0], runs[1], specs)
            for o in outs:
                o.mul_(1.5)
        for r in runs:
            r.close()


@pytest.mark.parametrize("case", range(16))
def test_random_tables_fused_equals_reading(case):
    """Seeded random fp32-gradient tables with an embedding of random width
    (rows whole units when it is a multiple of 256, straddling units
    otherwise) and a random token scatter: three steps with fresh backward
    outputs, the step after the final calls equal, bit for bit, to the step
    that reads the gradients."""
    torch = _torch()
    rng = np.random.default_rng(500 + case)
    vocab = int(rng.choice([3, 100, 1000, 5000]))
    d = int(rng.choice([1, 64, 256, 300, 512, 768]))
    specs = [TensorSpec("embed", (vocab, d), True, False)]
    for i in range(int(rng.integers(0, 8))):
        n = int(rng.choice([1, 255, 256, 257, 4095, 4096, 4097, 12345, int(rng.integers(1, 30000))]))
        specs.append(TensorSpec(f"t{i}", (n,), bool(rng.random() < 0.8), False))
    scale = float(2.0 ** int(rng.integers(0, 17)))
    no_unscale = tuple(s.name for s in specs[1:] if rng.random() < 0.2)
    outs = _outs(specs, 600 + case, 1e-3, scale)
    runs = [_Run(specs, outs, scale, no_unscale=no_unscale) for _ in range(2)]
    batch = int(rng.choice([0, 1, 100, 4096, 5000]))
    for k in range(3):
        for o in outs:
            o.normal_(0.0, float(10.0 ** rng.uniform(-5, -1)) * scale)
        tokens = torch.from_numpy(rng.integers(0, vocab + 3, batch).astype(np.int32)).cuda()
        dx0 = torch.randn(batch, d, device="cuda") * scale * 1e-3
        infos = [r.step(specs, fused, (0, vocab, d, tokens, dx0))
                 for r, fused in zip(runs, (False, True))]
        _info_eq(infos[0], infos[1])
        _same(runs[0], runs[1], specs)
    for r in runs:
        r.close()


def test_units_are_discarded_when_the_loss_scale_or_gradients_change():
    """After the final accumulation: ark_opt_set_state and
    ark_opt_record_overflow discard the units (the loss scale they were
    unscaled by changes), so the next step reads the gradients, here
    deliberately changed after the units were written; and a step consumes
    the units, so the one after reads again."""
    torch = _torch()
    specs = EkoConfig(n_layers=1, d_model=256, hidden=512, vocab=100).tensors()
    outs = _outs(specs, 2, 1e-3, 1024.0)
    a, b = (_Run(specs, outs, 1024.0) for _ in range(2))
    for r in (a, b):
        for i in range(len(specs)):
            r.ps.g(i).zero_()
    a.plan.run(final_for=a.opt)
    b.plan.run()
    for r in (a, b):
        r.ps.g(0).mul_(3.0)  # changed behind the units' back
    a.opt.set_state()  # the state as it is
    ia = a.opt.step_all(a.cfg.lr, info=True)[1]
    ib = b.opt.step_all(b.cfg.lr, info=True)[1]
    _info_eq(ia, ib)
    _same(a, b, specs)
    for r in (a, b):
        for i in range(len(specs)):
            r.ps.g(i).zero_()
    a.plan.run(final_for=a.opt)
    b.plan.run()
    a.opt.record_overflow()
    b.opt.record_overflow()
    for r in (a, b):
        r.ps.g(1).add_(1.0)
    ia = a.opt.step_all(a.cfg.lr, info=True)[1]
    ib = b.opt.step_all(b.cfg.lr, info=True)[1]
    _info_eq(ia, ib)
    _same(a, b, specs)
    a.close(), b.close()


@pytest.mark.parametrize("route", ["accumulate", "plan", "scatter", "scatter_noalloc", "dequant",
                                   "codec_plan", "ckpt_unpack", "adam_dropin"])
def test_library_gradient_writes_after_the_final_calls_drop_the_units(route):
    """After the final accumulation, a further write to a gradient through
    the library's other calls (ark_grad_accumulate, ark_grad_plan_run,
    ark_grad_embed_scatter and its no-allocation form, the codec's
    dequantisation and plan, a checkpoint unpack, a single-tensor Adam step
    whose m is that buffer) makes the next step read the gradients instead
    of the units the final call wrote: the step equals, bit for bit, that of
    a twin problem that never had units."""
    from ark_amd import ckpt, codec
    from ark_amd._lib import lib as lib_
    torch = _torch()
    specs = EkoConfig(n_layers=1, d_model=256, hidden=512, vocab=100).tensors()
    e = [s.name for s in specs].index("embed")
    outs = _outs(specs, 6, 1e-3, 1024.0)
    extra = _outs(specs, 7, 1e-2, 1024.0)
    tokens = torch.tensor([3, 7, 3, 99, 150], dtype=torch.int32, device="cuda")
    dx0 = torch.randn(5, 256, device="cuda", generator=torch.Generator(device="cuda")
                      .manual_seed(8)) * 10.0
    a, b = (_Run(specs, outs, 1024.0) for _ in range(2))
    for r in (a, b):
        for i in range(len(specs)):
            r.ps.g(i).zero_()
    a.plan.run(final_for=a.opt)  # a's units now describe these gradients
    b.plan.run()
    for r in (a, b):
        if route == "accumulate":
            grad.accumulate(r.ps.g(1), extra[1])
        elif route == "plan":
            r.plan.run()
        elif route == "dequant":
            codec.dequant_f16_to_f32(extra[1].half(), r.ps.g(1))
        elif route == "codec_plan":
            src = extra[1].half()
            cp = codec.CodecPlan([(src, r.ps.g(1))], "f16_to_f32")
            cp.run()
            torch.cuda.synchronize()
            cp.close()
        elif route == "ckpt_unpack":
            image = torch.empty(ckpt.image_bytes([extra[1]]), dtype=torch.uint8, device="cuda")
            ckpt.pack([extra[1]], image, 1, 1)
            ckpt.unpack(image, [r.ps.g(1)])
        elif route == "adam_dropin":
            # the gradient buffer used as another tensor's first moment
            n = r.ps.g(1).numel()
            w = torch.zeros(n, dtype=torch.float16, device="cuda")
            v = torch.zeros(n, device="cuda")
            assert lib_().ark_hip_adam_step_f16(w.data_ptr(), extra[1].data_ptr(),
                                                r.ps.g(1).data_ptr(), v.data_ptr(), n,
                                                3e-4, 0.9, 0.95, 1e-8, 0.0, 1,
                                                torch.cuda.current_stream().cuda_stream) == 0
        else:
            grad.embed_scatter(r.ps.g(e).view(100, 256), tokens, dx0,
                               noalloc=(route == "scatter_noalloc"))
    ia = a.opt.step_all(a.cfg.lr, info=True)[1]
    ib = b.opt.step_all(b.cfg.lr, info=True)[1]
    _info_eq(ia, ib)
    _same(a, b, specs)
    a.close(), b.close()


def test_final_calls_refuse_mismatched_handles():
    torch = _torch()
    from ark_amd._lib import ArkOptError, lib
    from ark_amd.optimizer import AdamConfig, AmpConfig, Optimizer, ParamSet
    specs = EkoConfig(n_layers=1, d_model=256, hidden=512, vocab=100).tensors()
    e = [s.name for s in specs].index("embed")
    outs = _outs(specs, 4, 1e-3, 1024.0)
    r = _Run(specs, outs, 1024.0)
    tokens = torch.zeros(10, dtype=torch.int32, device="cuda")
    dx0 = torch.ones(10, 256, device="cuda")
    emb = r.ps.g(e).view(100, 256)
    # the scatter's final form needs a final accumulation since the last step
    with pytest.raises(ArkOptError, match="final accumulation"):
        grad.embed_scatter(emb, tokens, dx0, final_for=r.opt)
    # ... unless its rows cannot be units (d % 256 != 0): then it only scatters,
    # as often as asked, and the step reads the gradients
    ps5 = ParamSet([TensorSpec("e", (50, 20), True, False)], 0.1, grad_dtype=_abi.GRAD_F32)
    o5 = Optimizer(AdamConfig(**HP), ps5, AmpConfig())
    t5 = torch.tensor([1, 3, 1], dtype=torch.int32, device="cuda")
    x5 = torch.ones(3, 20, device="cuda")
    for _ in range(2):
        grad.embed_scatter(ps5.g(0).view(50, 20), t5, x5, final_for=o5)
    torch.cuda.synchronize()
    assert ps5.g(0).view(50, 20)[1].tolist() == [4.0] * 20
    o5.close()
    # a plan over other buffers, or over a subset, is not the handle's table
    other = grad.GradPlan([(outs[i], outs[i].clone()) for i in range(len(specs))])
    with pytest.raises(ArkOptError, match="is not tensor 0's gradient"):
        other.run(final_for=r.opt)
    part = grad.GradPlan([(r.ps.g(i), outs[i]) for i in range(len(specs) - 1)])
    with pytest.raises(ArkOptError, match="ends before tensor"):
        part.run(final_for=r.opt)
    # an fp16-gradient handle has no units
    ps16 = ParamSet(specs, weight_decay=0.1)
    o16 = Optimizer(AdamConfig(**HP), ps16, AmpConfig())
    with pytest.raises(ArkOptError, match="fp32 gradients"):
        r.plan.run(final_for=o16)
    # a gradient that is no tensor of the table
    r.plan.run(final_for=r.opt)
    with pytest.raises(ArkOptError, match="no tensor of the optimizer table"):
        grad.embed_scatter(outs[e].view(100, 256), tokens, dx0, final_for=r.opt)
    assert lib().ark_grad_plan_run_final(None, r.opt.handle) == _abi.EINVAL
    assert lib().ark_grad_plan_run_final(r.plan._h, None) == _abi.EINVAL
    torch.cuda.synchronize()
    other.close(), part.close(), o16.close(), r.close()
