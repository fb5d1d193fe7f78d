"""Randomised GPU parity of the optimizer step: seeded random tensor tables
(sizes from 1 element to several segments, exact multiples of the 4096
segment and the 256-element row, element offsets that break 16-byte
alignment), fp16 or fp32 gradients, the no-unscale flag, random
hyperparameters, loss scales and clip thresholds, and occasional inf/NaN
gradients; three steps each, every scalar and every w/m/v bit against the
CPU oracle."""
import ctypes as C

import numpy as np
import pytest

import oracle
from oracle import harness as H
from ark_amd import _abi

pytestmark = pytest.mark.gpu

SIZES = [1, 3, 255, 256, 257, 1000, 4095, 4096, 4097, 8192, 12345, 3 * 4096 + 256]


def _torch():
    import torch
    assert torch.cuda.is_available(), "GPU test run without a GPU"
    return torch


def _bits16(t):
    torch = _torch()
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def _bits32(t):
    torch = _torch()
    return t.view(torch.int32).cpu().numpy().view(np.uint32)


@pytest.mark.parametrize("case", range(60))
def test_random_tables_match_oracle(case):
    torch = _torch()
    from ark_amd._lib import check, lib
    rng = np.random.default_rng(1000 + case)
    gdt = _abi.GRAD_F16 if case % 3 else _abi.GRAD_F32
    nt = int(rng.integers(1, 9))
    sizes = [int(rng.choice(SIZES)) if rng.random() < 0.7 else int(rng.integers(1, 30000))
             for _ in range(nt)]
    scale = float(2.0 ** rng.integers(0, 17))
    hp = oracle.default_hparams()
    hp.beta1 = float(np.float32(rng.choice([0.0, 0.5, 0.9, 0.99])))
    hp.beta2 = float(np.float32(rng.choice([0.0, 0.95, 0.999])))
    hp.eps = float(np.float32(rng.choice([1e-8, 1e-6, 1e-3])))
    hp.grad_clip = float(np.float32(rng.choice([0.05, 1.0, 1e30])))
    hp.loss_scale_init = scale
    hp.loss_scale_max = 2.0 ** 24
    hp.scale_up_every = int(rng.integers(1, 4))
    hp.grad_dtype = gdt
    lr = float(np.float32(rng.choice([1e-4, 3e-4, 1e-2])))

    gnp = np.float16 if gdt == _abi.GRAD_F16 else np.float32
    gtorch = torch.float16 if gdt == _abi.GRAD_F16 else torch.float32
    dev, host, keep = [], [], []
    for i, n in enumerate(sizes):
        off = int(rng.integers(0, 8))  # elements: breaks 16-byte alignment for off % 8 != 0
        w = (rng.standard_normal(n) * 0.05).astype(np.float16).view(np.uint16)
        m = (rng.standard_normal(n) * 1e-3).astype(np.float32)
        v = np.abs(rng.standard_normal(n) * 1e-6).astype(np.float32)
        wd = float(np.float32(rng.choice([0.0, 0.01, 0.1])))
        flags = _abi.TENSOR_NO_UNSCALE if rng.random() < 0.15 else 0
        bw = torch.zeros(n + off, dtype=torch.float16, device="cuda")
        bg = torch.zeros(n + off, dtype=gtorch, device="cuda")
        bm = torch.zeros(n + off, dtype=torch.float32, device="cuda")
        bv = torch.zeros(n + off, dtype=torch.float32, device="cuda")
        tw, tg, tm, tv = bw[off:], bg[off:], bm[off:], bv[off:]
        tw.copy_(torch.from_numpy(w.view(np.int16)).view(torch.float16))
        tm.copy_(torch.from_numpy(m))
        tv.copy_(torch.from_numpy(v))
        keep += [bw, bg, bm, bv]
        dev.append((tw, tg, tm, tv, wd, flags))
        host.append(oracle.HostTensor(w.copy(), np.zeros(n, np.uint16 if gdt == _abi.GRAD_F16
                                                         else np.float32),
                                      m.copy(), v.copy(), wd, flags))
    tab = (_abi.Tensor * nt)()
    for i, (tw, tg, tm, tv, wd, flags) in enumerate(dev):
        tab[i] = _abi.Tensor(tw.data_ptr(), tg.data_ptr(), tm.data_ptr(), tv.data_ptr(),
                             tw.numel(), wd, flags)
    h = C.c_void_p()
    check(lib().ark_opt_create(tab, nt, C.byref(hp), C.c_void_p(torch.cuda.current_stream()
                                                                   .cuda_stream), C.byref(h)))
    ref = oracle.Optimizer(host, hp)
    try:
        for k in range(3):
            for i, n in enumerate(sizes):
                sig = float(10.0 ** rng.uniform(-5, -1))
                g = (rng.standard_normal(n) * sig * scale).astype(gnp)
                if rng.random() < 0.08:
                    g[int(rng.integers(0, n))] = rng.choice([np.inf, -np.inf, np.nan])
                dev[i][1].copy_(torch.from_numpy(g))
                host[i].g[:] = g.view(host[i].g.dtype)
            gi = _abi.StepInfo()
            rc = lib().ark_opt_step(h, lr, C.byref(gi))
            rrc, ri = ref.step(lr)
            assert rc == rrc, (k, rc, rrc)
            d = H.info_matches(gi, ri)
            assert not d, f"step {k}: {d}"
            for i in range(nt):
                tw, tg, tm, tv = dev[i][:4]
                assert not np.any(H.bits_differ16(_bits16(tw), host[i].w)), (k, i, "w")
                assert not np.any(H.bits_differ32(_bits32(tm).view(np.float32), host[i].m)), (k, i, "m")
                assert not np.any(H.bits_differ32(_bits32(tv).view(np.float32), host[i].v)), (k, i, "v")
    finally:
        lib().ark_opt_destroy(h)


def test_thousands_of_tiny_tensors():
    """3000 tensors of 1-300 elements: every segment ragged, every norm block
    mixed, a 3000-entry descriptor table; plus one tensor past a segment
    boundary.  Three steps against the oracle."""
    torch = _torch()
    from ark_amd.eko import TensorSpec
    from ark_amd.optimizer import AdamConfig, AmpConfig, Optimizer
    rng = np.random.default_rng(77)
    sizes = [int(x) for x in rng.integers(1, 301, 3000)] + [4096 + 17]
    specs = [TensorSpec(f"t{i}", (n,), bool(i % 5), False) for i, n in enumerate(sizes)]
    sig = [float(10.0 ** rng.uniform(-4, -2)) for _ in specs]
    cfg = AdamConfig(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1, grad_clip=0.5)
    amp = AmpConfig(loss_scale_init=4096.0, loss_scale_max=2.0 ** 24)
    ps = H.gpu_problem(specs, 8, cfg.weight_decay, sig, 4096.0)
    ts = H.host_problem(specs, 8, cfg.weight_decay, sig, 4096.0)
    opt = Optimizer(cfg, ps, amp)
    ref = oracle.Optimizer(ts, opt.hp, nthreads=8)
    for k in range(3):
        if k:
            H.gpu_regen_grads(ps, 8, sig, 4096.0, k)
            H.host_regen_grads(ts, 8, sig, 4096.0, k)
        _, gi = opt.step_all(cfg.lr, info=True)
        _, ri = ref.step(cfg.lr)
        assert not H.info_matches(gi, ri), k
    c = H.compare(ps, ts)
    assert c["w"] == c["m"] == c["v"] == 0, c
    opt.close()
