"""The optimizer step captured in a HIP graph (through torch.cuda.CUDAGraph):
ark_opt_step without an info read-back only queues kernels on the handle's
stream (no host wait, no memset, no allocation), so a caller can capture it
once and replay it.  Every replay is checked against an eager step of an
identical problem, with eager work (new gradients, a state read) between
replays, including a replay that must skip on a non-finite gradient."""
import pytest

from oracle import harness as H
from ark_amd.eko import config_tensors

pytestmark = pytest.mark.gpu


def _torch():
    import torch
    assert torch.cuda.is_available(), "GPU test run without a GPU"
    return torch


@pytest.mark.parametrize("name", ["c0", "c1"])
def test_step_replays_match_eager(name):
    torch = _torch()
    from ark_amd.optimizer import AdamConfig, AmpConfig, Optimizer
    specs = config_tensors(name)
    sig = [1e-3] * len(specs)
    scale, seed, lr = 1024.0, 21, 3e-4
    cfg = AdamConfig(lr=lr, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1, grad_clip=1.0)
    amp = AmpConfig(loss_scale_init=scale, loss_scale_max=2.0 ** 24)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        pg = H.gpu_problem(specs, seed, cfg.weight_decay, sig, scale)
        pe = H.gpu_problem(specs, seed, cfg.weight_decay, sig, scale)
        og, oe = Optimizer(cfg, pg, amp), Optimizer(cfg, pe, amp)
    s.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        og.step_all(lr)
    for k in range(6):
        with torch.cuda.stream(s):
            if k:
                H.gpu_regen_grads(pg, seed, sig, scale, k)
                H.gpu_regen_grads(pe, seed, sig, scale, k)
            if k == 3:  # one non-finite gradient: both must skip
                for p in (pg, pe):
                    p.g(0).view(torch.int16)[5] = 0x7C00
            g.replay()
            oe.step_all(lr)
        s.synchronize()
        sg, se = og.get_state(), oe.get_state()
        for f in ("t", "loss_scale", "clean_steps", "consecutive_nonfinite", "skipped_steps"):
            assert getattr(sg, f) == getattr(se, f), (k, f)
        assert sg.skipped_steps == (1 if k >= 3 else 0)
        for i in range(len(specs)):
            for a, b in ((pg.w(i), pe.w(i)), (pg.m(i), pe.m(i)), (pg.v(i), pe.v(i))):
                it = torch.int16 if a.element_size() == 2 else torch.int32
                assert torch.equal(a.view(it), b.view(it)), (k, i)
    og.close(), oe.close()


def _same(pa, pb, n, what):
    torch = _torch()
    for i in range(n):
        for a, b in ((pa.w(i), pb.w(i)), (pa.m(i), pb.m(i)), (pa.v(i), pb.v(i))):
            it = torch.int16 if a.element_size() == 2 else torch.int32
            assert torch.equal(a.view(it), b.view(it)), (what, i)


def test_lr_from_a_device_scalar_follows_a_schedule_in_replays():
    """ark_opt_step_lr_dev reads lr from a device scalar when the step runs:
    eagerly it matches ark_opt_step with the same host lr bit for bit, and
    one captured call replayed with the scalar rewritten (outside the graph)
    before each replay follows a warmup-then-cosine schedule (lr_now,
    optimizer.rs:80-92) exactly as eager steps with host lrs do."""
    torch = _torch()
    from ark_amd.optimizer import AdamConfig, AmpConfig, Optimizer
    specs = config_tensors("c1")
    sig = [1e-3] * len(specs)
    scale, seed = 1024.0, 33
    cfg = AdamConfig(lr=6e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1, grad_clip=1.0,
                     warmup_steps=10)
    amp = AmpConfig(loss_scale_init=scale, loss_scale_max=2.0 ** 24)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        pg = H.gpu_problem(specs, seed, cfg.weight_decay, sig, scale)
        pe = H.gpu_problem(specs, seed, cfg.weight_decay, sig, scale)
        og, oe = Optimizer(cfg, pg, amp), Optimizer(cfg, pe, amp)
        lr_dev = torch.zeros(1, dtype=torch.float32, device="cuda")
    s.synchronize()
    # eager: the device scalar and the host value give the same step
    with torch.cuda.stream(s):
        lr_dev.fill_(og.lr_now(1))
        og.step_lr_dev(lr_dev)
        oe.step_all(oe.lr_now(1))
    s.synchronize()
    _same(pg, pe, len(specs), "eager")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        og.step_lr_dev(lr_dev)
    for k in range(2, 8):
        lr = oe.lr_now(k)
        with torch.cuda.stream(s):
            H.gpu_regen_grads(pg, seed, sig, scale, k)
            H.gpu_regen_grads(pe, seed, sig, scale, k)
            lr_dev.fill_(lr)
            g.replay()
            oe.step_all(lr)
        s.synchronize()
        assert og.get_state().t == oe.get_state().t == k
        _same(pg, pe, len(specs), k)
    assert len({oe.lr_now(k) for k in range(2, 8)}) == 6  # the lr changed on every replay
    og.close(), oe.close()


def test_a_non_finite_device_lr_leaves_everything_as_it_was():
    torch = _torch()
    from ark_amd import _abi
    from ark_amd._lib import ArkOptError
    from ark_amd.optimizer import AdamConfig, AmpConfig, Optimizer
    specs = config_tensors("c0")
    p = H.gpu_problem(specs, 3, 0.1, [1e-3], 1024.0)
    o = Optimizer(AdamConfig(), p, AmpConfig(loss_scale_init=1024.0))
    before = [x.clone() for x in (p.w(0), p.m(0), p.v(0))]
    st0 = o.get_state().as_dict()
    lr_dev = torch.tensor([float("nan")], device="cuda")
    with pytest.raises(ArkOptError, match="not finite"):
        o.step_lr_dev(lr_dev, info=True)
    torch.cuda.synchronize()
    assert o.get_state().as_dict() == st0
    for a, b in zip((p.w(0), p.m(0), p.v(0)), before):
        assert torch.equal(a, b)
    lr_dev.fill_(3e-4)
    rc, info = o.step_lr_dev(lr_dev, info=True)
    assert rc == _abi.OK and info.applied == 1 and info.lr == pytest.approx(3e-4)
    o.close()


def test_final_accumulation_and_step_captured_together():
    """The gradient plan's final accumulation (which also writes the norm's
    units) and the step on fp32 gradients captured in one graph, replayed
    over fresh backward outputs with the lr rewritten in its device scalar
    before each replay: every replay leaves the same w, m, v, gradient and
    state bits as the same two calls made eagerly on an identical problem.
    Capture records no host-side decision that a replay would get wrong:
    the accumulation marks the units fresh and the captured step consumes
    them, both inside the graph."""
    torch = _torch()
    from ark_amd import _abi, synth
    from ark_amd.grad import GradPlan
    from ark_amd.optimizer import AdamConfig, AmpConfig, Optimizer
    specs = config_tensors("c1")
    sig = [1e-3] * len(specs)
    scale, seed = 256.0, 41
    cfg = AdamConfig(lr=6e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1, grad_clip=1.0,
                     warmup_steps=10)
    amp = AmpConfig(loss_scale_init=scale, loss_scale_max=2.0 ** 24)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        pa = H.gpu_problem(specs, seed, cfg.weight_decay, sig, scale, grad_dtype=_abi.GRAD_F32)
        pb = H.gpu_problem(specs, seed, cfg.weight_decay, sig, scale, grad_dtype=_abi.GRAD_F32)
        oa, ob = Optimizer(cfg, pa, amp, stream=s), Optimizer(cfg, pb, amp, stream=s)
        outs_a = [torch.empty_like(pa.g(i)) for i in range(len(specs))]
        outs_b = [torch.empty_like(pb.g(i)) for i in range(len(specs))]
        plan_a = GradPlan(list(zip([pa.g(i) for i in range(len(specs))], outs_a)), stream=s)
        plan_b = GradPlan(list(zip([pb.g(i) for i in range(len(specs))], outs_b)), stream=s)
        lr_dev = torch.zeros(1, dtype=torch.float32, device="cuda")

    def backward_outputs(k):
        for i in range(len(specs)):
            ss = synth.grad_sigma_scale(sig[i], scale)
            synth.normal_f32(outs_a[i], seed + 7, i, k, ss)
            synth.normal_f32(outs_b[i], seed + 7, i, k, ss)

    with torch.cuda.stream(s):
        backward_outputs(0)
    s.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        plan_a.run(final_for=oa)
        oa.step_lr_dev(lr_dev)
    # capture ran no kernel: both problems are still at step 0
    assert oa.get_state().t == ob.get_state().t == 0
    lrs = set()
    for k in range(1, 7):
        lr = ob.lr_now(k)
        lrs.add(lr)
        with torch.cuda.stream(s):
            backward_outputs(k)
            lr_dev.fill_(lr)
            g.replay()
            plan_b.run(final_for=ob)
            ob.step_all(lr)
        s.synchronize()
        sa, sb = oa.get_state(), ob.get_state()
        assert sa.as_dict() == sb.as_dict() and sa.t == k, (k, sa.as_dict(), sb.as_dict())
        _same(pa, pb, len(specs), k)
        for i in range(len(specs)):
            assert torch.equal(pa.g(i).view(torch.int32), pb.g(i).view(torch.int32)), (k, i)
    assert len(lrs) == 6  # the warmup changes lr on every replay
    plan_a.close(), plan_b.close()
    oa.close(), ob.close()
