"""lr_now (optimizer.rs:80-92) pinned over its whole domain, on the CPU.

The schedule's only non-basic operation is `f32::cos` (optimizer.rs:89).
Both host mirrors (ark_amd/optimizer.py:cos_f32 and ark::host::lr_now in
ark_amd/host/ark_host.hpp) take it as the correctly rounded fp32 cosine.
These tests show that this is what they compute on every argument the
schedule can produce, x = fp32(fp32(pi) * min(d / 800000, 1)) for
d = 0..800000: libm's double cos is rounded once, and each result is
accepted only when rounding is unambiguous (the double lies more than two
of its ulps from an fp32 rounding boundary) or a 60-digit decimal cosine
settles it.  The two mirrors then agree bit for bit on every step."""
import math
import os
import subprocess
from decimal import Decimal, localcontext
from fractions import Fraction

import numpy as np
import pytest

from ark_amd.optimizer import AdamConfig, cos_f32, lr_now

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LR_TABLE = os.path.join(ROOT, "tests", "cpp", "_build", "lr_table")

F32 = np.float32
TOTAL_DECAY = 800_000
PI_DIGITS = "3.14159265358979323846264338327950288419716939937510582097494459"


def schedule_args():
    """Every cosine argument lr_now makes, in the reference's fp32 order."""
    d = np.arange(TOTAL_DECAY + 1, dtype=np.float32)
    progress = np.minimum(d / F32(TOTAL_DECAY), F32(1.0))
    return (F32(np.pi) * progress).astype(np.float32)


def dec_cos(x: float) -> Decimal:
    """cos(x) to ~60 significant digits by its Taylor series (|x| <= 3.15)."""
    with localcontext() as ctx:
        ctx.prec = 70
        x = Decimal(x)
        x2 = x * x
        term, total, k = Decimal(1), Decimal(1), 0
        while True:
            k += 1
            term = -term * x2 / ((2 * k - 1) * (2 * k))
            total += term
            if abs(term) < Decimal("1e-66"):
                return total


def round_exact_to_f32(v: Decimal) -> np.float32:
    """Round a decimal value to the nearest fp32 (ties to even) exactly."""
    f = Fraction(v)
    c = F32(float(f))
    best = None
    for cand in (np.nextafter(c, F32(-2)), c, np.nextafter(c, F32(2))):
        dist = abs(Fraction(float(cand)) - f)
        even = (int(cand.view(np.uint32)) & 1) == 0
        key = (dist, not even)
        if best is None or key < best[0]:
            best = (key, cand)
    return best[1]


def test_double_cos_is_within_one_ulp_on_a_sample():
    """The margin test below assumes libm's double cos errs by under 2 ulps;
    check it against the decimal cosine on every 400th argument."""
    xs = schedule_args()[::400]
    for x in xs:
        c = math.cos(float(x))
        exact = dec_cos(float(x))
        ulp = Decimal(math.ulp(c))
        assert abs(Decimal(c) - exact) <= ulp, (float(x), c)


def test_cos_f32_is_correctly_rounded_on_every_schedule_argument():
    xs = schedule_args()
    c64 = np.array([math.cos(float(x)) for x in xs], dtype=np.float64)
    lo = np.nextafter(np.nextafter(c64, -np.inf), -np.inf)
    hi = np.nextafter(np.nextafter(c64, np.inf), np.inf)
    cand = c64.astype(np.float32)
    safe = (lo.astype(np.float32) == cand) & (hi.astype(np.float32) == cand)
    for i in np.nonzero(~safe)[0]:  # near a rounding boundary: settle exactly
        cand[i] = round_exact_to_f32(dec_cos(float(xs[i])))
    got = np.array([cos_f32(x) for x in xs], dtype=np.float32)
    assert np.array_equal(got.view(np.uint32), cand.view(np.uint32))
    assert int((~safe).sum()) < 10  # the exact path is for rare cases only


def test_cos_f32_known_answers():
    """Closed forms independent of libm: fp32(pi) = pi + delta, so
    cos(fp32(pi) / 2) = -sin(delta / 2) = -delta / 2 to fp32 precision, and
    cos(fp32(pi)) = -cos(delta) rounds to -1."""
    with localcontext() as ctx:
        ctx.prec = 70
        delta = Decimal(float(F32(np.pi))) - Decimal(PI_DIGITS)
        minus_half_delta = -delta / 2
    half = F32(F32(np.pi) * F32(0.5))
    assert cos_f32(half) == round_exact_to_f32(minus_half_delta)
    assert cos_f32(F32(np.pi)) == F32(-1.0)
    assert cos_f32(F32(0.0)) == F32(1.0)


def reference_lr(cfg: AdamConfig, steps: np.ndarray, cos_of) -> np.ndarray:
    """optimizer.rs:80-92 vectorised in fp32, with the cosine supplied."""
    lr = F32(cfg.lr)
    s = steps.astype(np.int64)
    warm = s < cfg.warmup_steps
    out = np.empty(len(s), np.float32)
    out[warm] = lr * (s[warm].astype(np.float32) + F32(1.0)) / F32(cfg.warmup_steps)
    d = (s[~warm] - cfg.warmup_steps).astype(np.float32)
    progress = np.minimum(d / F32(TOTAL_DECAY), F32(1.0))
    cosine = F32(0.5) * (F32(1.0) + cos_of((F32(np.pi) * progress).astype(np.float32)))
    lr_min = lr * F32(0.1)
    out[~warm] = lr_min + (lr - lr_min) * cosine
    return out


@pytest.mark.parametrize("lr,warmup", [(3e-4, 100), (1e-3, 2000)])
def test_python_mirror_follows_the_schedule(lr, warmup):
    cfg = AdamConfig(lr=lr, warmup_steps=warmup)
    steps = np.unique(np.concatenate([
        np.arange(0, warmup + 3), np.arange(warmup, warmup + TOTAL_DECAY + 1, 7),
        warmup + TOTAL_DECAY + np.arange(-2, 5), [5_000_000]]))
    exact = np.vectorize(cos_f32, otypes=[np.float32])
    want = reference_lr(cfg, steps, exact)
    got = np.array([lr_now(cfg, int(s)) for s in steps], dtype=np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # known answers: the warmup is linear, the floor is exactly lr * 0.1
    assert lr_now(cfg, 0) == float(F32(lr) * F32(1.0) / F32(warmup))
    assert lr_now(cfg, warmup + TOTAL_DECAY) == float(F32(lr) * F32(0.1))
    assert lr_now(cfg, 10 * TOTAL_DECAY) == float(F32(lr) * F32(0.1))


@pytest.fixture(scope="module")
def lr_table():
    """The C++ mirror's table tool, built with hipcc when absent (host code only)."""
    if not os.path.exists(LR_TABLE):
        subprocess.run(["make", "-C", os.path.join(ROOT, "tests", "cpp"), "_build/lr_table"],
                       check=True, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
    return LR_TABLE


@pytest.mark.parametrize("lr,warmup", [(3e-4, 100), (1e-3, 2000)])
def test_cpp_mirror_equals_python_mirror_on_every_step(lr_table, lr, warmup):
    n = warmup + TOTAL_DECAY + 10
    r = subprocess.run([lr_table, repr(lr), str(warmup), str(n)], stdout=subprocess.PIPE,
                       timeout=120, check=True)
    cpp = np.frombuffer(r.stdout, dtype=np.float32)
    assert len(cpp) == n
    cfg = AdamConfig(lr=lr, warmup_steps=warmup)
    py = reference_lr(cfg, np.arange(n), np.vectorize(cos_f32, otypes=[np.float32]))
    assert np.array_equal(cpp.view(np.uint32), py.view(np.uint32))
