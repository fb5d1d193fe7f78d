"""The rows together, in the order the reference's Trainer::train_step and
its checkpointing call them (training.rs:162-186, :228-326, :536-604;
objc/bridge.m:902-948): per step the gradients are zeroed (:248), the
backward outputs accumulated and the tokens scattered into the embedding
gradient (ark_grad_*), the fused step runs on the fp32 gradients
(ark_opt_step), and the updated fp16 weights are dequantised for the next
forward (ark_codec_*); a checkpoint is written mid-run and loaded into
fresh buffers at the end.  The CPU oracle runs the same chain; every
gradient, weight, moment, dequantised weight and checkpoint byte matches."""
import numpy as np
import pytest

import oracle
from oracle import ckpt as K
from oracle import harness as H
from ark_amd.eko import EkoConfig

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("d_model,fused", [(64, False), (256, True), (64, True)])
def test_training_steps_through_every_row(tmp_path, d_model, fused):
    """fused: the last accumulation and the scatter also write the norm's
    units (ark_grad_plan_run_final, ark_grad_embed_scatter_final), so the
    step reads no gradient; at d_model 64 the embedding rows do not align
    with the units and the step reads the gradients again."""
    import torch
    assert torch.cuda.is_available(), "GPU test run without a GPU"
    from ark_amd import _abi, ckpt, codec, grad
    from ark_amd.optimizer import AdamConfig, AmpConfig, Optimizer, ParamSet

    mc = EkoConfig(n_layers=2, d_model=d_model, hidden=96, vocab=300)
    specs = mc.tensors()
    e = [s.name for s in specs].index("embed")
    rng = np.random.default_rng(2024)
    scale = 2048.0
    cfg = AdamConfig(lr=1e-3, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1, grad_clip=1.0)
    amp = AmpConfig(loss_scale_init=scale, loss_scale_max=2.0 ** 24, scale_up_every=2)

    ps = ParamSet(specs, weight_decay=0.1, grad_dtype=_abi.GRAD_F32)
    w0 = [(rng.standard_normal(s.n) * 0.02).astype(np.float16).view(np.uint16) for s in specs]
    for i in range(len(specs)):
        ps.w(i).copy_(torch.from_numpy(w0[i].view(np.int16)).view(torch.float16))
    opt = Optimizer(cfg, ps, amp)
    temps = [torch.empty(s.n, dtype=torch.float32, device="cuda") for s in specs]
    dq = codec.CodecPlan([(ps.w(i), temps[i]) for i in range(len(specs))], "f16_to_f32")
    outs_dev = [torch.empty(s.n, dtype=torch.float32, device="cuda") for s in specs]
    gp = grad.GradPlan([(ps.g(i), outs_dev[i]) for i in range(len(specs))])

    host = [oracle.HostTensor(w0[i].copy(), np.zeros(s.n, np.float32), np.zeros(s.n, np.float32),
                              np.zeros(s.n, np.float32), 0.1 if s.decay else 0.0)
            for i, s in enumerate(specs)]
    ref = oracle.Optimizer(host, opt.hp)
    mid = str(tmp_path / "mid.ark")
    for k in range(5):
        outs = [(rng.standard_normal(s.n) * 1e-3 * scale).astype(np.float32) for s in specs]
        tokens = ((rng.zipf(1.3, 256) - 1) % (mc.vocab + 4)).astype(np.uint32)
        dx0 = (rng.standard_normal((256, mc.d_model)) * 1e-3 * scale).astype(np.float32)
        if k == 2:
            outs[3][7] = np.inf  # a non-finite gradient: the step is skipped
        # device
        for i in range(len(specs)):
            ps.g(i).zero_()                                        # training.rs:248
            outs_dev[i].copy_(torch.from_numpy(outs[i]))
        gp.run(final_for=opt if fused else None)                   # bridge.m:910-915, :931-947
        grad.embed_scatter(ps.g(e).view(mc.vocab, mc.d_model),     # bridge.m:922-928
                           torch.from_numpy(tokens.view(np.int32)).cuda(),
                           torch.from_numpy(dx0).cuda(), final_for=opt if fused else None)
        _, gi = opt.step_all(cfg.lr, info=True)                    # training.rs:289-326
        dq.run()                                                   # training.rs:162-186
        # host
        for i, t in enumerate(host):
            t.g[:] = 0.0
            oracle.grad_accumulate(t.g, outs[i])
        oracle.embed_scatter(host[e].g.reshape(mc.vocab, mc.d_model), tokens, dx0)
        _, ri = ref.step(cfg.lr)
        assert not H.info_matches(gi, ri), k
        assert gi.applied == (0 if k == 2 else 1)
        torch.cuda.synchronize()
        for i, t in enumerate(host):
            np.testing.assert_array_equal(ps.g(i).cpu().numpy().view(np.uint32),
                                          t.g.view(np.uint32))
            np.testing.assert_array_equal(temps[i].cpu().numpy().view(np.uint32),
                                          oracle.f16_to_f32(t.w).view(np.uint32))
        c = H.compare(ps, host)
        assert c["w"] == c["m"] == c["v"] == 0, (k, c)
        if k == 3:                                                 # training.rs:536-604
            ckpt.save_params(mid, ps, opt, global_step=k)
            snap = [H.to_host(x).copy() for x in ckpt.param_tensors(ps)]
            want = (K.write_v4(k, ref.state.t, _file_order(specs, mc.n_layers, host))
                    + K.amp_trailer(bytes(ref.state)))
            assert open(mid, "rb").read() == want
    # resume the mid-run checkpoint into fresh buffers and a fresh handle
    qs = ParamSet(specs, weight_decay=0.1, grad_dtype=_abi.GRAD_F32)
    o2 = Optimizer(cfg, qs, amp)
    info, st = ckpt.load_params(mid, qs, o2)
    assert info.global_step == 3 and info.has_amp and o2.get_state().t == st.t
    for a, b in zip(snap, ckpt.param_tensors(qs)):
        np.testing.assert_array_equal(H.to_host(b).view(a.dtype), a)
    opt.close(), o2.close(), dq.close(), gp.close()


def _file_order(specs, n_layers, host):
    """The oracle's w/m/v in guardar_checkpoint's order (embed w, m, v; per
    layer 9 w, 9 m, 9 v; gamma_final w, m, v)."""
    idx = {s.name: i for i, s in enumerate(specs)}
    names = ["wq", "wk", "wv", "wo", "w1", "w2", "w3", "g1", "g2"]
    emb, gam = host[idx["embed"]], host[idx["gamma_final"]]
    out = [emb.w, emb.m, emb.v]
    for layer in range(n_layers):
        ids = [idx[f"l{layer}.{n}"] for n in names]
        out += [host[i].w for i in ids] + [host[i].m for i in ids] + [host[i].v for i in ids]
    return out + [gam.w, gam.m, gam.v]
