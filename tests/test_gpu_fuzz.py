"""Randomised GPU parity of the optimizer step (ark_opt_step) against the
CPU oracle, bit for bit, on tables and hyperparameters no fixed
configuration covers together.

Each of 60 cases draws, from its own seed:
  * 1-9 tensors with sizes from empty and single elements through exact
    multiples of the 256-element row and the 4096-element segment and
    ragged segment counts to ~40k elements, each at its own element offset
    (0-7) in separate allocations, so 16-byte alignment breaks;
  * per-tensor weight decay and the NO_UNSCALE flag (the gamma_final quirk);
  * fp16 (loss-scaled) or fp32 gradients;
  * beta1, beta2 (fixed and continuous values, 0 included), eps (0
    included), grad_clip (tiny to never), the initial loss scale,
    scale_up_every and the early-stop limit;
  * starting m (signed) and v (non-negative), fp16 weights with some
    subnormals and some gains of 1.0;
and runs five steps with fresh gradients and a fresh lr each; gradient
scales reach fp16 overflow (inf: a skipped step), and an inf, -inf or NaN is
sometimes planted.  Every step's status and scalars and every w/m/v element
are compared (optimizer.rs:126-228, training.rs:289-326, opti.s:192-360).
The twenty fp16 cases run again at 1.5 times their drawn loss scale, so the
norm pass's path for scales that are not powers of two is compared too.
A CPU test replays every case through the oracle alone and checks that the
sweep reaches each of those outcomes.  A last test steps 3001 tensors, most
of them tiny."""
import numpy as np
import pytest

import oracle
from oracle import harness as H
from ark_amd import _abi

SIZES = [0, 1, 3, 255, 256, 257, 1000, 4095, 4096, 4097, 8192, 12345, 3 * 4096 + 256, 40000]


def _torch():
    import torch
    assert torch.cuda.is_available(), "GPU test run without a GPU"
    return torch


def _f16_bits(rng, n, sigma):
    x = (rng.standard_normal(n) * sigma).astype(np.float16)
    return x.view(np.uint16).copy()


def _draw_grads(rng, n, grad_dtype, scale):
    sigma = 10.0 ** rng.uniform(-7, -1) * scale
    if rng.random() < 0.15:
        sigma = 10.0 ** rng.uniform(3, 6)  # reaches fp16's range: inf, a skipped step
    if grad_dtype == _abi.GRAD_F16:
        with np.errstate(over="ignore"):
            g = _f16_bits(rng, n, sigma)
    else:
        g = (rng.standard_normal(n) * sigma).astype(np.float32)
    if n and rng.random() < 0.08:
        bad = np.array([rng.choice([np.inf, -np.inf, np.nan])], np.float32)
        g[int(rng.integers(n))] = (bad.astype(np.float16).view(np.uint16)[0]
                                   if grad_dtype == _abi.GRAD_F16 else bad[0])
    return g


CASES = 60


def draw_case(case, scale_mul=1.0):
    """The case's hyperparameters, tensors (host arrays and element offsets)
    and its per-step gradients and lrs, all from the case's seed; the drawn
    initial loss scale (a power of two) times scale_mul."""
    from ark_amd.optimizer import AdamConfig, AmpConfig
    rng = np.random.default_rng(1000 + case)
    grad_dtype = _abi.GRAD_F16 if case % 3 else _abi.GRAD_F32
    ntens = int(rng.integers(1, 10))
    scale = float(2.0 ** int(rng.integers(0, 17))) * scale_mul
    cfg = AdamConfig(lr=3e-4,
                     beta1=float(np.float32(rng.choice([0.0, 0.5, 0.9, rng.uniform(0, 0.999)]))),
                     beta2=float(np.float32(rng.choice([0.0, 0.95, 0.999,
                                                        rng.uniform(0.5, 0.99999)]))),
                     eps=float(rng.choice([0.0, 1e-8, 1e-6, 1e-3])),
                     weight_decay=0.0,
                     grad_clip=float(rng.choice([1e-3, 0.5, 1.0, 10.0, 1e30])))
    amp = AmpConfig(loss_scale_init=scale, loss_scale_max=2.0 ** 24,
                    scale_up_every=int(rng.choice([1, 2, 3, 2000])),
                    max_consecutive_nonfinite=int(rng.choice([1, 2, 200])))
    tensors = []
    for _ in range(ntens):
        n = int(rng.choice(SIZES)) if rng.random() < 0.7 else int(rng.integers(1, 30000))
        off = int(rng.integers(0, 8))
        wd = float(np.float32(rng.choice([0.0, 0.01, 0.1, rng.uniform(0, 0.5)])))
        flags = _abi.TENSOR_NO_UNSCALE if rng.random() < 0.2 else 0
        w = _f16_bits(rng, n, 0.05)
        if n and rng.random() < 0.3:  # some subnormal weights
            k = max(1, n // 50)
            w[rng.integers(n, size=k)] = rng.integers(1, 0x400, size=k)
        if rng.random() < 0.15:
            w[:] = 0x3C00  # a gain, initialised to 1.0
        m = (rng.standard_normal(n) * 1e-3).astype(np.float32)
        v = (np.abs(rng.standard_normal(n)) * 1e-6).astype(np.float32)
        tensors.append(dict(n=n, off=off, wd=wd, flags=flags, w=w, m=m, v=v))
    steps = []
    for _ in range(5):
        grads = [_draw_grads(rng, t["n"], grad_dtype, scale) for t in tensors]
        steps.append((grads, float(np.float32(10.0 ** rng.uniform(-6, -2)))))
    return grad_dtype, cfg, amp, tensors, steps


def _host_tensors(tensors, steps):
    return [oracle.HostTensor(t["w"].copy(), steps[0][0][i].copy(), t["m"].copy(),
                              t["v"].copy(), t["wd"], t["flags"])
            for i, t in enumerate(tensors)]


@pytest.mark.gpu
@pytest.mark.parametrize("case", range(CASES))
def test_random_tables_and_hyperparameters(case):
    _run_case(case)


@pytest.mark.gpu
@pytest.mark.parametrize("case", range(1, CASES, 3))
def test_random_fp16_cases_at_scales_that_are_not_powers_of_two(case):
    """The fp16-gradient cases again with 1.5 times the drawn loss scale: the
    norm pass then unscales each element before squaring instead of taking
    the squares from the fp16 bits, and tests each element for inf/NaN."""
    _run_case(case, scale_mul=1.5)


def _run_case(case, scale_mul=1.0):
    torch = _torch()
    from ark_amd.optimizer import Optimizer
    grad_dtype, cfg, amp, tensors, steps = draw_case(case, scale_mul)
    gdt = torch.int16 if grad_dtype == _abi.GRAD_F16 else torch.float32
    as_torch = lambda a: torch.from_numpy(a.view(np.int16) if a.dtype == np.uint16 else a)
    bufs, arr = [], (_abi.Tensor * len(tensors))()
    for i, t in enumerate(tensors):
        n, off = t["n"], t["off"]
        # each array in its own allocation, the tensor at element offset off
        dw = torch.zeros(n + off + 8, dtype=torch.int16, device="cuda")
        dg = torch.zeros(n + off + 8, dtype=gdt, device="cuda")
        dm = torch.zeros(n + off + 8, dtype=torch.float32, device="cuda")
        dv = torch.zeros(n + off + 8, dtype=torch.float32, device="cuda")
        dw[off:off + n] = as_torch(t["w"])
        dg[off:off + n] = as_torch(steps[0][0][i])
        dm[off:off + n] = as_torch(t["m"])
        dv[off:off + n] = as_torch(t["v"])
        bufs.append((dw, dg, dm, dv, off, n))
        arr[i].w, arr[i].g = dw.data_ptr() + 2 * off, dg.data_ptr() + dg.element_size() * off
        arr[i].m, arr[i].v = dm.data_ptr() + 4 * off, dv.data_ptr() + 4 * off
        arr[i].n, arr[i].weight_decay, arr[i].flags = n, t["wd"], t["flags"]
    hosts = _host_tensors(tensors, steps)
    torch.cuda.synchronize()
    opt = Optimizer(cfg, _GradDtype(grad_dtype), amp, table=arr)
    ref = oracle.Optimizer(hosts, opt.hp)
    for k, (grads, lr) in enumerate(steps):
        if k:
            for (dw, dg, dm, dv, off, n), t, g in zip(bufs, hosts, grads):
                t.g[:] = g
                dg[off:off + n] = as_torch(g)
        rc, gi = opt.step_all(lr, info=True)
        rrc, ri = ref.step(lr)
        assert rc == rrc, (case, k, rc, rrc)
        d = H.info_matches(gi, ri)
        assert not d, (case, k, d)
        for i, ((dw, dg, dm, dv, off, n), t) in enumerate(zip(bufs, hosts)):
            gw = dw[off:off + n].cpu().numpy().view(np.uint16)
            assert not np.any(H.bits_differ16(gw, t.w)), (case, k, i, "w")
            assert not np.any(H.bits_differ32(dm[off:off + n].cpu().numpy(), t.m)), (case, k, i)
            assert not np.any(H.bits_differ32(dv[off:off + n].cpu().numpy(), t.v)), (case, k, i)
    opt.close()


def test_the_sweep_reaches_every_outcome():
    """On the CPU, through the oracle alone: the cases' steps include
    applied steps that clip and that do not, skipped steps, an early stop,
    growth of the loss scale, both gradient types, unaligned tensors, empty
    tensors and NO_UNSCALE tensors, so the GPU sweep compares all of them."""
    from ark_amd.optimizer import hparams
    seen = set()
    for case in range(CASES):
        grad_dtype, cfg, amp, tensors, steps = draw_case(case)
        hosts = _host_tensors(tensors, steps)
        ref = oracle.Optimizer(hosts, hparams(cfg, amp, grad_dtype))
        scale0 = amp.loss_scale_init
        for k, (grads, lr) in enumerate(steps):
            for t, g in zip(hosts, grads):
                t.g[:] = g
            rc, info = ref.step(lr)
            if rc == _abi.EARLY_STOP:
                seen.add("early stop")
            elif info.applied:
                seen.add("clipped" if info.clipped else "unclipped")
            else:
                seen.add("skipped")
            if info.state.loss_scale > scale0:
                seen.add("growth")
        seen.add(f"grad {grad_dtype}")
        for t in tensors:
            if t["off"]:
                seen.add("unaligned")
            if t["n"] == 0:
                seen.add("empty")
            if t["flags"]:
                seen.add("no unscale")
    want = {"clipped", "unclipped", "skipped", "early stop", "growth", "unaligned", "empty",
            "no unscale", f"grad {_abi.GRAD_F16}", f"grad {_abi.GRAD_F32}"}
    assert want <= seen, want - seen


@pytest.mark.gpu
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


class _GradDtype:
    """Stands in for a ParamSet where only the gradient dtype is read."""

    def __init__(self, grad_dtype):
        self.grad_dtype = grad_dtype
