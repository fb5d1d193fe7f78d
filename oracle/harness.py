"""TEST INFRASTRUCTURE ONLY: matched GPU / CPU-oracle problems for the parity
tests, __graft_entry__.smoke() and bench.py's cpu_baseline leg.

A problem is a list of TensorSpec (ark_amd.eko) with seeded inputs built by
the same counter-based generator on both sides (ark_amd.synth on the GPU,
oracle.synth_* on the CPU), so both start from identical bits; the stream
constants and the sigma draw are ark_amd.synth's.
"""
import numpy as np

import oracle
from ark_amd import _abi
from ark_amd.synth import (F16_ONE, W_SIGMA, WEIGHT_STEP, grad_sigma_scale,  # noqa: F401
                           log_uniform_sigmas)
from ark_amd.synth import problem as gpu_problem  # noqa: F401
from ark_amd.synth import regen_grads as gpu_regen_grads  # noqa: F401


def f32(x):
    return float(np.float32(x))


# ---- host side ----------------------------------------------------------------

def _pmap(fn, items, nthreads):
    """Map over items on a thread pool (the oracle's C calls release the GIL)."""
    if nthreads <= 1:
        return [fn(x) for x in items]
    from concurrent.futures import ThreadPoolExecutor
    with ThreadPoolExecutor(nthreads) as ex:
        return list(ex.map(fn, items))


def host_problem(specs, seed, weight_decay, sigmas, loss_scale, step=0,
                 grad_dtype=_abi.GRAD_F16, no_unscale=(), nthreads=1):
    def make(i):
        s = specs[i]
        if s.gain:
            w = np.full(s.n, F16_ONE, np.uint16)
        else:
            w = oracle.synth_normal_f16(s.n, seed, i, WEIGHT_STEP, W_SIGMA)
        if grad_dtype == _abi.GRAD_F16:
            g = oracle.synth_normal_f16(s.n, seed, i, step, grad_sigma_scale(sigmas[i], loss_scale))
        else:
            g = oracle.synth_normal_f32(s.n, seed, i, step, grad_sigma_scale(sigmas[i], loss_scale))
        m = np.zeros(s.n, np.float32)
        v = np.zeros(s.n, np.float32)
        return oracle.HostTensor(w, g, m, v, weight_decay if s.decay else 0.0,
                                 _abi.TENSOR_NO_UNSCALE if s.name in no_unscale else 0)
    return _pmap(make, range(len(specs)), nthreads)


def host_regen_grads(ts, seed, sigmas, loss_scale, step, grad_dtype=_abi.GRAD_F16,
                     nthreads=1):
    def regen(i):
        t = ts[i]
        ss = grad_sigma_scale(sigmas[i], loss_scale)
        if grad_dtype == _abi.GRAD_F16:
            t.g[:] = oracle.synth_normal_f16(t.n, seed, i, step, ss)
        else:
            t.g[:] = oracle.synth_normal_f32(t.n, seed, i, step, ss)
    _pmap(regen, range(len(ts)), nthreads)


# ---- comparisons -------------------------------------------------------------

def to_host(t):
    """torch tensor on the GPU -> numpy array with the same bits."""
    import torch
    if t.dtype == torch.float16:
        return t.view(torch.int16).cpu().numpy().view(np.uint16)
    return t.cpu().numpy()


def compare(ps, ts, idx=None, nthreads=1):
    """Bitwise mismatch counts of w, m, v (NaNs compare equal to NaNs)."""
    out = {"w": 0, "m": 0, "v": 0, "n": 0}
    idx = list(range(len(ts)) if idx is None else idx)
    host = [(to_host(ps.w(i)), to_host(ps.m(i)), to_host(ps.v(i))) for i in idx]

    def count(k):
        i = idx[k]
        gw, gm, gv = host[k]
        t = ts[i]
        return (int(np.sum(bits_differ16(gw, t.w))), int(np.sum(bits_differ32(gm, t.m))),
                int(np.sum(bits_differ32(gv, t.v))), t.n)
    for w, m, v, n in _pmap(count, range(len(idx)), nthreads):
        out["w"] += w
        out["m"] += m
        out["v"] += v
        out["n"] += n
    return out


def bits_differ16(a, b):
    a = np.asarray(a, np.uint16)
    b = np.asarray(b, np.uint16)
    na = (a & 0x7FFF) > 0x7C00
    nb = (b & 0x7FFF) > 0x7C00
    return np.where(na | nb, na != nb, a != b)


def bits_differ32(a, b):
    a = np.asarray(a, np.float32).view(np.uint32)
    b = np.asarray(b, np.float32).view(np.uint32)
    na = (a & 0x7FFFFFFF) > 0x7F800000
    nb = (b & 0x7FFFFFFF) > 0x7F800000
    return np.where(na | nb, na != nb, a != b)


def info_matches(a, b):
    """Every scalar of two StepInfo structs bit for bit (sumsq included)."""
    da, db = a.as_dict(), b.as_dict()
    diffs = {}
    for k in da:
        if k == "state":
            for kk in da[k]:
                if da[k][kk] != db[k][kk]:
                    diffs[f"state.{kk}"] = (da[k][kk], db[k][kk])
        elif isinstance(da[k], float):
            if np.float64(da[k]).tobytes() != np.float64(db[k]).tobytes() and not (
                    np.isnan(da[k]) and np.isnan(db[k])):
                diffs[k] = (da[k], db[k])
        elif da[k] != db[k]:
            diffs[k] = (da[k], db[k])
    return diffs
