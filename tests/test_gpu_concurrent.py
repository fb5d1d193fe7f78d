"""Handles are independent: two optimizer handles bound to two streams,
stepped in an interleaved order with no host wait between them (so their
kernels may overlap on the device), each give exactly the oracle's result
for their own problem.  Also a codec plan and a gradient plan running on a
third stream meanwhile."""
import pytest

import oracle
from oracle import harness as H
from ark_amd.eko import EkoConfig

pytestmark = pytest.mark.gpu


def test_two_handles_on_two_streams():
    import torch
    assert torch.cuda.is_available(), "GPU test run without a GPU"
    from ark_amd import codec, grad
    from ark_amd.optimizer import AdamConfig, AmpConfig, Optimizer
    cfg = AdamConfig(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1, grad_clip=1.0)
    amp = AmpConfig(loss_scale_init=1024.0, loss_scale_max=2.0 ** 24, scale_up_every=2)
    specs = [EkoConfig(n_layers=2, d_model=64, hidden=96, vocab=500).tensors(),
             EkoConfig(n_layers=1, d_model=128, hidden=256, vocab=777).tensors()]
    seeds = [31, 32]
    sig = [[1e-3] * len(s) for s in specs]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    ps, opts, ts, refs = [], [], [], []
    for i in range(2):
        with torch.cuda.stream(streams[i]):
            p = H.gpu_problem(specs[i], seeds[i], cfg.weight_decay, sig[i], 1024.0)
            ps.append(p)
            opts.append(Optimizer(cfg, p, amp))
        t = H.host_problem(specs[i], seeds[i], cfg.weight_decay, sig[i], 1024.0)
        ts.append(t)
        refs.append(oracle.Optimizer(t, opts[i].hp))
    torch.cuda.synchronize()
    # a third stream keeps the device busy with other library work meanwhile
    s3 = torch.cuda.Stream()
    with torch.cuda.stream(s3):
        a16 = torch.randn(1 << 20, device="cuda").half()
        a32 = torch.empty(1 << 20, device="cuda")
        dq = codec.CodecPlan([(a16, a32)], "f16_to_f32")
        x = torch.randn(1 << 20, device="cuda")
        y = torch.randn(1 << 20, device="cuda")
        gp = grad.GradPlan([(x, y)])
    torch.cuda.synchronize()
    for k in range(6):
        for i in (0, 1) if k % 2 else (1, 0):
            with torch.cuda.stream(streams[i]):
                if k:
                    H.gpu_regen_grads(ps[i], seeds[i], sig[i], 1024.0, k)
                opts[i].step_all(cfg.lr)
        with torch.cuda.stream(s3):
            dq.run()
            gp.run()
    torch.cuda.synchronize()
    for i in range(2):
        for k in range(6):
            if k:
                H.host_regen_grads(ts[i], seeds[i], sig[i], 1024.0, k)
            refs[i].step(cfg.lr)
        st = opts[i].get_state()
        assert st.t == refs[i].state.t and st.loss_scale == refs[i].state.loss_scale
        c = H.compare(ps[i], ts[i])
        assert c["w"] == c["m"] == c["v"] == 0, (i, c)
        opts[i].close()
    dq.close(), gp.close()
