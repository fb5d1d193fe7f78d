"""Write tests/golden/oracle_steps.json: per-step scalars and SHA-256 digests
of w, m, v produced by the CPU oracle for configurations c0 and c1 (seeded
synthetic inputs from the counter-based generator).  The CPU test
regenerates them to catch oracle regressions; the GPU test compares the HIP
path's arrays against the same digests.

Usage: python tests/golden/make_golden.py
"""
import hashlib
import json
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

import numpy as np  # noqa: E402

import oracle  # noqa: E402
from oracle import harness as H  # noqa: E402
from ark_amd.eko import config_tensors  # noqa: E402
from ark_amd.optimizer import AdamConfig, AmpConfig, hparams  # noqa: E402

CASES = {
    "c0": dict(seed=11, sigma=1e-3, scale=1024.0, steps=10),
    "c1": dict(seed=5, sigma=1e-3, scale=1024.0, steps=5),
}
HP = dict(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1, grad_clip=1.0)


def digest(ts):
    out = {}
    for k in ("w", "m", "v"):
        h = hashlib.sha256()
        for t in ts:
            h.update(np.ascontiguousarray(getattr(t, k)).tobytes())
        out[k] = h.hexdigest()
    return out


def run_case(name, c):
    specs = config_tensors(name)
    sig = [c["sigma"]] * len(specs)
    cfg = AdamConfig(**HP)
    hp = hparams(cfg, AmpConfig(loss_scale_init=c["scale"], loss_scale_max=2.0 ** 24))
    ts = H.host_problem(specs, c["seed"], cfg.weight_decay, sig, c["scale"])
    ref = oracle.Optimizer(ts, hp, nthreads=8)
    steps = []
    for k in range(c["steps"]):
        if k:
            H.host_regen_grads(ts, c["seed"], sig, c["scale"], k)
        _, info = ref.step(cfg.lr)
        d = info.as_dict()
        d["grad_sumsq"] = float(d["grad_sumsq"]).hex()
        for f in ("grad_norm", "clip_coef", "inv_scale", "lr", "lr_eff"):
            d[f] = float(np.float32(d[f])).hex()
        d["state"]["loss_scale"] = float(d["state"]["loss_scale"]).hex()
        steps.append({"info": d, "sha256": digest(ts)})
    return {"config": c, "hparams": HP, "steps": steps}


def main():
    out = {name: run_case(name, c) for name, c in CASES.items()}
    dst = os.path.join(os.path.dirname(os.path.abspath(__file__)), "oracle_steps.json")
    json.dump(out, open(dst, "w"), indent=1)
    print("wrote", dst)


if __name__ == "__main__":
    main()
