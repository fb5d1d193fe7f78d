"""Committed golden fixtures (tests/golden/oracle_steps.json, written by
tests/golden/make_golden.py): the CPU oracle must reproduce them (CPU test),
and the HIP path must match them bit for bit (GPU test)."""
import hashlib
import json
import os

import numpy as np
import pytest

import oracle
from oracle import harness as H
from ark_amd.eko import config_tensors
from ark_amd.optimizer import AdamConfig, AmpConfig, hparams

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "oracle_steps.json")))


def _encode(info):
    d = info.as_dict()
    d["grad_sumsq"] = float(d["grad_sumsq"]).hex()
    for f in ("grad_norm", "clip_coef", "inv_scale", "lr", "lr_eff"):
        d[f] = float(np.float32(d[f])).hex()
    d["state"]["loss_scale"] = float(d["state"]["loss_scale"]).hex()
    return d


def _digest(arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


@pytest.mark.parametrize("name", sorted(GOLD))
def test_oracle_reproduces_golden(name):
    g = GOLD[name]
    c = g["config"]
    specs = config_tensors(name)
    sig = [c["sigma"]] * len(specs)
    cfg = AdamConfig(**g["hparams"])
    hp = hparams(cfg, AmpConfig(loss_scale_init=c["scale"], loss_scale_max=2.0 ** 24))
    ts = H.host_problem(specs, c["seed"], cfg.weight_decay, sig, c["scale"])
    ref = oracle.Optimizer(ts, hp, nthreads=8)
    for k, want in enumerate(g["steps"]):
        if k:
            H.host_regen_grads(ts, c["seed"], sig, c["scale"], k)
        _, info = ref.step(cfg.lr)
        assert _encode(info) == want["info"], k
        for a in ("w", "m", "v"):
            assert _digest([getattr(t, a) for t in ts]) == want["sha256"][a], (k, a)


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(GOLD))
def test_gpu_matches_golden(name):
    import torch
    from ark_amd.optimizer import Optimizer
    assert torch.cuda.is_available()
    g = GOLD[name]
    c = g["config"]
    specs = config_tensors(name)
    sig = [c["sigma"]] * len(specs)
    cfg = AdamConfig(**g["hparams"])
    amp = AmpConfig(loss_scale_init=c["scale"], loss_scale_max=2.0 ** 24)
    ps = H.gpu_problem(specs, c["seed"], cfg.weight_decay, sig, c["scale"])
    opt = Optimizer(cfg, ps, amp)
    for k, want in enumerate(g["steps"]):
        if k:
            H.gpu_regen_grads(ps, c["seed"], sig, c["scale"], k)
        _, info = opt.step_all(cfg.lr, info=True)
        assert _encode(info) == want["info"], k
        for a in ("w", "m", "v"):
            arrays = [H.to_host(getattr(ps, a)(i)) for i in range(len(specs))]
            assert _digest(arrays) == want["sha256"][a], (k, a)
    opt.close()
