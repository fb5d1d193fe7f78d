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
