"""ark_hip_grad_clip, the drop-in for ark_asm_grad_clip (opti.s:369-432,
ffi.rs:111-115, :206-220), against the oracle's form of the same call
(tests/test_oracle_grad_clip.py pins it against the instruction sequence):
the reported norm and every value after the call bit for bit, clipped and
not, over sizes from one value to the 24.6M-value embedding gradient and
past 67M values (the partials folded before the finalize), at unaligned
addresses, with inf, NaN and the compare's edge cases, and queued without
waiting."""
import numpy as np
import pytest

import oracle
from oracle import harness as H
from ark_amd import optimizer

pytestmark = pytest.mark.gpu
F32 = np.float32


def _torch():
    import torch
    assert torch.cuda.is_available(), "GPU test run without a GPU"
    return torch


def _check(h, thr, offset=0, wait=True):
    """h (float32 numpy) through the GPU call at `offset` floats into its
    buffer, and through the oracle; every bit must agree."""
    torch = _torch()
    buf = torch.empty(h.size + offset, dtype=torch.float32, device="cuda")
    dev = buf[offset:]
    dev.copy_(torch.from_numpy(h))
    norm = optimizer.grad_clip_global(dev, float(thr), wait=wait)
    torch.cuda.synchronize()
    want = h.copy()
    wn = oracle.grad_clip(want, F32(thr), nthreads=8)
    got = dev.cpu().numpy()
    if wait:
        assert not H.bits_differ32(np.array([norm], F32), np.array([wn], F32)).any(), (norm, wn)
    bad = np.nonzero(H.bits_differ32(got, want))[0]
    assert bad.size == 0, f"{bad.size} values differ, first at {bad[0]}: {got[bad[0]]} vs {want[bad[0]]}"
    return wn


@pytest.mark.parametrize("n", [1, 3, 4, 5, 2047, 4095, 4096, 4097, 8191, 8192, 8193, 100003,
                               1572864, 24576000])
def test_matches_the_oracle_clipped_and_not(n):
    rng = np.random.default_rng(n)
    h = (rng.standard_normal(n) * 10.0 ** rng.uniform(-5, 1, n)).astype(F32)
    norm = _check(h, 1e30)  # not clipped
    assert 0.0 < norm < 1e30
    _check(h, norm * 0.25)  # clipped


@pytest.mark.parametrize("n", [67108864 + 1, 70000000])
def test_past_the_fold_threshold(n):
    """More than 8192 partials (over 67,108,864 values): folded in groups of
    64 first, as the step folds its own."""
    rng = np.random.default_rng(n)
    h = (rng.standard_normal(n) * 1e-3).astype(F32)
    norm = _check(h, 1e30)
    _check(h, norm * 0.5)


@pytest.mark.parametrize("offset", [1, 2, 3])
def test_unaligned_addresses(offset):
    rng = np.random.default_rng(offset)
    h = (rng.standard_normal(50001) * 0.1).astype(F32)
    _check(h, 1.0, offset=offset)


def test_special_values():
    rng = np.random.default_rng(9)
    base = (rng.standard_normal(20000) * 0.01).astype(F32)
    inf = base.copy()
    inf[12345] = np.inf  # norm inf: coefficient 0, the inf itself to NaN
    assert _check(inf, 1.0) == np.inf
    nan = base.copy()
    nan[7] = np.nan  # norm NaN: unordered, nothing changes
    assert np.isnan(_check(nan, 1.0))
    both = base.copy()
    both[3], both[19999] = np.inf, np.nan
    assert np.isnan(_check(both, 1.0))
    exact = np.array([0.5, -0.5, 0.5, 0.5] * 4, F32)  # norm exactly 2
    assert _check(exact, 2.0) == 2.0
    _check(exact, np.nextafter(F32(2.0), F32(0.0)))
    _check(base, float("nan"))
    _check(np.zeros(1000, F32), -1.0)  # 0 > -1 clips with -1 / 0 = -inf: NaN
    _check(np.zeros(1000, F32), 0.0)   # 0 > 0 does not clip
    big = np.full(10, 3e19, F32)       # squares past fp32 range: norm inf
    assert _check(big, 1.0) == np.inf


def test_queued_without_waiting_and_empty():
    torch = _torch()
    rng = np.random.default_rng(4)
    h = (rng.standard_normal(300000) * 0.1).astype(F32)
    _check(h, 1.0, wait=False)
    empty = torch.empty(0, dtype=torch.float32, device="cuda")
    assert optimizer.grad_clip(empty, 1.0) == 0.0
    assert optimizer.grad_clip_global(empty, -1.0) == 0.0


def test_eko237m_gradients_one_call_per_tensor():
    """The reference's usage (ffi.rs:206-213): one call per gradient slice,
    here every one of EKO-237M's 272 fp32 gradient buffers of a ParamSet, each
    against the oracle; about half clip at 1.0."""
    torch = _torch()
    from ark_amd import _abi, synth
    from ark_amd.eko import config_tensors
    specs = config_tensors("c2")
    sig = synth.log_uniform_sigmas(len(specs), 31)
    ps = synth.problem(specs, 31, 0.1, sig, 1.0, grad_dtype=_abi.GRAD_F32)
    torch.cuda.synchronize()
    host = [ps.g(i).cpu().numpy() for i in range(len(specs))]
    clipped = 0
    for i in range(len(specs)):
        norm = optimizer.grad_clip_global(ps.g(i), 1.0)
        want = host[i].copy()
        wn = oracle.grad_clip(want, F32(1.0), nthreads=8)
        assert np.float32(norm).view(np.uint32) == np.float32(wn).view(np.uint32), specs[i].name
        assert np.array_equal(ps.g(i).cpu().numpy().view(np.uint32), want.view(np.uint32)), i
        clipped += wn > 1.0
    assert 0 < clipped < len(specs)


def random_case(case):
    """Seeded random call `case`: sizes from 1 to ~3M values (ragged blocks,
    n % 4 tails, a few past one 8192-value block), magnitudes 10^U(-30, 15)
    per call with a spread inside it, thresholds around the norm or special
    (0, negative, inf, NaN), and now and then an inf or NaN planted.
    Returns (values, threshold, misalignment in floats)."""
    rng = np.random.default_rng(9000 + case)
    r = rng.random()
    n = (int(rng.integers(1, 9)) if r < 0.15 else int(rng.integers(8185, 8200)) if r < 0.3
         else int(rng.integers(9, 300000)) if r < 0.8 else int(rng.integers(300000, 3000000)))
    scale = 10.0 ** rng.uniform(-30, 15)
    h = (rng.standard_normal(n) * scale * 10.0 ** rng.uniform(-3, 3, n)).astype(F32)
    if rng.random() < 0.2:
        h[int(rng.integers(n))] = rng.choice([np.inf, -np.inf, np.nan])
    probe = oracle.grad_clip(h.copy(), F32(np.inf), nthreads=8)  # the norm, nothing clipped
    t = rng.random()
    thr = (float(probe) * float(rng.uniform(0.1, 2.0)) if t < 0.7 and np.isfinite(probe)
           else float(rng.choice([0.0, -1.0, np.inf, np.nan, 1.0])))
    return h, thr, int(rng.integers(0, 4))


@pytest.mark.parametrize("case", range(30))
def test_seeded_random_calls(case):
    """random_case(case) on the device at its misalignment; every result bit
    against the oracle (tests/test_oracle_grad_clip.py checks on the CPU
    that the cases reach every outcome)."""
    h, thr, offset = random_case(case)
    _check(h, thr, offset=offset)
