"""Pins of the oracle's AdamW element update and scalar prologue
(ark_asm_adam_step_f16, opti.s:192-360).

Independent checks, none of which reuses the oracle's C code:
  * a second restatement in Python: numpy float32 scalar operations (each an
    IEEE binary32 op), an exact-rational fused multiply-add rounded once to
    binary32 (the fmla of opti.s:287, :293), numpy's fp16 conversion;
  * closed forms (constant-gradient moments, bias corrections against f64
    pow, the t = 0 fix, zero gradients, wd = 0, the beta = 0 sign-SGD limit).
"""
from fractions import Fraction

import numpy as np
import pytest

import oracle

F32 = np.float32


def round_to_f32(x):
    """Exact rational -> nearest binary32, ties to even, subnormals kept."""
    if x == 0:
        return F32(0.0)
    sign = -1 if x < 0 else 1
    a = abs(x)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    e = max(e, -126)
    quantum = Fraction(2) ** (e - 23)
    q = a / quantum
    n = q.numerator // q.denominator
    r = q - n
    if r > Fraction(1, 2) or (r == Fraction(1, 2) and n % 2 == 1):
        n += 1
    val = n * quantum
    if val >= Fraction(2) ** 128:
        return F32(sign * np.inf)
    return F32(sign * float(val))


def fma32(a, b, c):
    """a*b + c rounded once; an exact zero keeps IEEE's sign rule."""
    a, b, c = F32(a), F32(b), F32(c)
    p = Fraction(float(a)) * Fraction(float(b))
    s = p + Fraction(float(c))
    if s == 0:
        p_neg = (np.signbit(a) != np.signbit(b)) if p == 0 else p < 0
        c_neg = bool(np.signbit(c)) if c == 0 else c < 0
        return F32(-0.0) if (p_neg and c_neg) else F32(0.0)
    return round_to_f32(s)


def py_prologue(lr, b1, b2, wd, t):
    lr, b1, b2, wd = F32(lr), F32(b1), F32(b2), F32(wd)
    if t == 0:
        t = 1

    def powb(b, k):
        r, base = F32(1.0), b
        while k:
            if k & 1:
                r = F32(r * base)
            base = F32(base * base)
            k >>= 1
        return r

    bc1 = F32(F32(1.0) - powb(b1, t))
    bc2 = F32(F32(1.0) - powb(b2, t))
    lr_eff = F32(F32(np.sqrt(bc2) / bc1) * lr)
    return dict(decay=F32(F32(1.0) - F32(lr * wd)), lr_eff=lr_eff,
                c1=F32(F32(1.0) - b1), c2=F32(F32(1.0) - b2))


def py_adam_elem(w16, g, m, v, s, b1, b2, eps):
    b1, b2, eps = F32(b1), F32(b2), F32(eps)
    w = np.array([w16], np.uint16).view(np.float16).astype(np.float32)[0]
    mm = fma32(s["c1"], g, F32(F32(m) * b1))
    vv = fma32(s["c2"], F32(F32(g) * F32(g)), F32(F32(v) * b2))
    d = F32(np.sqrt(vv) + eps)
    u = F32(F32(mm / d) * s["lr_eff"])
    wn = F32(F32(w * s["decay"]) - u)
    return int(np.array([wn], np.float32).astype(np.float16).view(np.uint16)[0]), mm, vv


def _random_inputs(n, seed):
    rng = np.random.default_rng(seed)
    w = rng.integers(0, 65536, n).astype(np.uint16)
    w[(w & 0x7C00) == 0x7C00] = 0x3C00
    kinds = rng.integers(0, 4, n)
    g = np.where(kinds == 0, rng.standard_normal(n) * 1e-3,
        np.where(kinds == 1, rng.standard_normal(n) * 1e-30,       # subnormal squares
        np.where(kinds == 2, rng.standard_normal(n) * 30.0, 0.0))).astype(np.float32)
    g[::37] = np.float32(1e-40)                                     # fp32 subnormal gradient
    m = (rng.standard_normal(n) * 1e-3).astype(np.float32)
    v = (rng.random(n) * 1e-6).astype(np.float32)
    v[::11] = 0.0
    return w, g, m, v


@pytest.mark.parametrize("t", [0, 1, 2, 7, 1000, 123457])
def test_second_restatement_bit_exact(t):
    lr, b1, b2, eps, wd = 3e-4, 0.9, 0.95, 1e-8, 0.1
    w, g, m, v = _random_inputs(1500, t)
    s = py_prologue(lr, b1, b2, wd, t)
    ow, om, ov = w.copy(), m.copy(), v.copy()
    oracle.adam_step_f16(ow, g, om, ov, lr, b1, b2, eps, wd, t)
    fused_differs = 0
    for i in range(w.size):
        pw, pm, pv = py_adam_elem(w[i], g[i], m[i], v[i], s, b1, b2, eps)
        assert ow[i] == pw, (i, hex(ow[i]), hex(pw))
        assert om[i].view(np.uint32) == F32(pm).view(np.uint32), i
        assert ov[i].view(np.uint32) == F32(pv).view(np.uint32), i
        unfused = F32(F32(s["c1"] * g[i]) + F32(m[i] * F32(b1)))
        fused_differs += int(unfused != pm)
    # the set exercises inputs where the fmla's single rounding matters
    assert fused_differs > 0


def test_prologue_matches_second_restatement():
    for t in [0, 1, 2, 3, 100, 2000, 65535, 800000, 2 ** 32 - 1]:
        for b1, b2 in [(0.9, 0.95), (0.9, 0.999), (0.5, 0.5)]:
            a = oracle.prologue(3e-4, b1, b2, 0.1, t)
            b = py_prologue(3e-4, b1, b2, 0.1, t)
            for k in ("decay", "lr_eff", "c1", "c2"):
                assert F32(a[k]) == b[k], (t, b1, b2, k)


def test_bias_corrections_vs_f64_pow():
    """beta^t by binary powering: relative error below 2 t u (u = 2^-24;
    each squaring doubles the error it inherits), exact for t = 1, 2."""
    u = 2.0 ** -24
    for b in (0.9, 0.95, 0.999):
        bf = float(F32(b))
        assert oracle.pow_binary(b, 1) == bf
        assert oracle.pow_binary(b, 2) == float(F32(F32(b) * F32(b)))
        for t in list(range(1, 64)) + [100, 999, 2000, 65535, 10 ** 5]:
            exact = bf ** t
            got = oracle.pow_binary(b, t)
            assert abs(got - exact) <= 2 * t * u * exact + 2.0 ** -149, (b, t)


def test_binary_exponentiation_is_not_the_sequential_product():
    """opti.s:223-253 replaced the O(t) product loop (CHANGELOG_ES.md:781-785);
    the two agree to ~1e-6 but not bit for bit, so the restatement must use
    the binary method."""
    b = F32(0.999)
    seq, differ = F32(1.0), 0
    for t in range(1, 3000):
        seq = F32(seq * b)
        differ += int(F32(oracle.pow_binary(0.999, t)) != seq)
        assert abs(float(seq) - oracle.pow_binary(0.999, t)) < 5e-6
    assert differ > 100


def test_lr_eff_closed_form_and_t0_fix():
    for t in (1, 2, 10, 1000):
        s = oracle.prologue(3e-4, 0.9, 0.95, 0.0, t)
        exact = 3e-4 * np.sqrt(1 - 0.95 ** t) / (1 - 0.9 ** t)
        assert abs(s["lr_eff"] - exact) < 2e-6 * exact
        assert s["decay"] == 1.0
    assert oracle.prologue(3e-4, 0.9, 0.95, 0.1, 0) == oracle.prologue(3e-4, 0.9, 0.95, 0.1, 1)


def test_zero_gradient_and_state_only_decays():
    w = oracle.synth_normal_f16(4099, 1, 0, 0, 0.02)
    z = np.zeros(w.size, np.float32)
    ww = w.copy()
    oracle.adam_step_f16(ww, z.copy(), z.copy(), z.copy(), 3e-4, 0.9, 0.95, 1e-8, 0.1, 5)
    decay = F32(F32(1.0) - F32(F32(3e-4) * F32(0.1)))
    expect = (w.view(np.float16).astype(np.float32) * decay).astype(np.float16).view(np.uint16)
    assert np.array_equal(ww, expect)
    ww = w.copy()
    oracle.adam_step_f16(ww, z.copy(), z.copy(), z.copy(), 3e-4, 0.9, 0.95, 1e-8, 0.0, 5)
    assert np.array_equal(ww, w)  # wd = 0: decay exactly 1


def test_constant_gradient_moments_closed_form():
    """m_T = g (1 - b1^T), v_T = g^2 (1 - b2^T) from zero state, so the
    bias-corrected update is lr * sign(g) (for |g| >> eps)."""
    n, T = 64, 40
    g = (np.linspace(-1, 1, n) * 1e-3).astype(np.float32)
    g[n // 2] = 1e-3
    w = np.zeros(n, np.uint16)
    m = np.zeros(n, np.float32)
    v = np.zeros(n, np.float32)
    for t in range(1, T + 1):
        w[:] = 0
        oracle.adam_step_f16(w, g, m, v, 1e-2, 0.9, 0.95, 1e-8, 0.0, t)
    g64 = g.astype(np.float64)
    assert np.allclose(m, g64 * (1 - 0.9 ** T), rtol=1e-5, atol=0)
    assert np.allclose(v, g64 ** 2 * (1 - 0.95 ** T), rtol=1e-5, atol=0)
    upd = -w.view(np.float16).astype(np.float64)  # one step from w = 0
    nz = np.abs(g64) > 1e-5
    assert np.allclose(upd[nz], 1e-2 * np.sign(g64[nz]), rtol=2e-3)


def test_zero_betas_reduce_to_sign_sgd():
    g = (np.random.default_rng(4).standard_normal(512) * 1e-2).astype(np.float32)
    w = oracle.synth_normal_f16(512, 2, 0, 0, 0.02)
    m = np.full(512, 5.0, np.float32)
    v = np.full(512, 7.0, np.float32)
    ww = w.copy()
    oracle.adam_step_f16(ww, g, m, v, 1e-3, 0.0, 0.0, 1e-8, 0.0, 9)
    assert np.array_equal(m, g) and np.array_equal(v, g * g)
    u = (g.astype(np.float64) / (np.abs(g.astype(np.float64)) + 1e-8)) * 1e-3
    expect = (w.view(np.float16).astype(np.float64) - u)
    got = ww.view(np.float16).astype(np.float64)
    ulp = np.spacing(np.abs(expect).astype(np.float16)).astype(np.float64)
    assert np.all(np.abs(got - expect) <= ulp)


# ---- the fp32-weight kernel (ark_asm_adam_step, opti.s:20-177) --------------

def py_adam_elem_f32(w, g, m, v, s, b1, b2, eps):
    """The fp32-weight element: py_adam_elem's operations on an fp32 weight,
    without the fp16 widening and narrowing (opti.s:114-130)."""
    b1, b2, eps = F32(b1), F32(b2), F32(eps)
    mm = fma32(s["c1"], g, F32(F32(m) * b1))
    vv = fma32(s["c2"], F32(F32(g) * F32(g)), F32(F32(v) * b2))
    d = F32(np.sqrt(vv) + eps)
    u = F32(F32(mm / d) * s["lr_eff"])
    return F32(F32(F32(w) * s["decay"]) - u), mm, vv


@pytest.mark.parametrize("t", [0, 1, 7, 123457])
def test_fp32_weight_step_second_restatement_bit_exact(t):
    """Weights the fp16 path never sees (fp32 values between fp16 ones,
    fp32 subnormals, beyond 65504) against the independent restatement."""
    lr, b1, b2, eps, wd = 3e-4, 0.9, 0.95, 1e-8, 0.1
    _, g, m, v = _random_inputs(1200, 1000 + t)
    rng = np.random.default_rng(t)
    w = (rng.standard_normal(g.size) * 10.0 ** rng.integers(-40, 6, g.size)).astype(np.float32)
    w[::13] = np.float32(1e-41)
    w[::17] = np.float32(1e6)
    s = py_prologue(lr, b1, b2, wd, t)
    ow, om, ov = w.copy(), m.copy(), v.copy()
    oracle.adam_step_f32(ow, g, om, ov, lr, b1, b2, eps, wd, t)
    for i in range(w.size):
        pw, pm, pv = py_adam_elem_f32(w[i], g[i], m[i], v[i], s, b1, b2, eps)
        assert ow[i].view(np.uint32) == F32(pw).view(np.uint32), (i, ow[i], pw)
        assert om[i].view(np.uint32) == F32(pm).view(np.uint32), i
        assert ov[i].view(np.uint32) == F32(pv).view(np.uint32), i


@pytest.mark.parametrize("t", [1, 50])
def test_fp32_weight_step_is_the_fp16_step_before_its_rounding(t):
    """On weights fp16 can hold, the fp16 kernel is the fp32 kernel followed
    by fcvtn: the same m and v bits, and the fp16 weight equal to the fp32
    weight rounded to nearest even (both restatements run in the oracle's C
    code, against each other)."""
    lr, b1, b2, eps, wd = 3e-4, 0.9, 0.95, 1e-8, 0.1
    w16, g, m, v = _random_inputs(4000, 77 + t)
    w32 = w16.view(np.float16).astype(np.float32)
    a_w, a_m, a_v = w16.copy(), m.copy(), v.copy()
    b_w, b_m, b_v = w32.copy(), m.copy(), v.copy()
    oracle.adam_step_f16(a_w, g, a_m, a_v, lr, b1, b2, eps, wd, t)
    oracle.adam_step_f32(b_w, g, b_m, b_v, lr, b1, b2, eps, wd, t)
    np.testing.assert_array_equal(a_m.view(np.uint32), b_m.view(np.uint32))
    np.testing.assert_array_equal(a_v.view(np.uint32), b_v.view(np.uint32))
    np.testing.assert_array_equal(a_w, oracle.f32_to_f16(b_w))
    # and the fp32 result is not merely the fp16 one widened
    assert (b_w != a_w.view(np.float16).astype(np.float32)).mean() > 0.5


def test_fp32_weight_step_closed_forms():
    """Zero gradient and state: w * decay exactly (lr 3e-4, wd 0.1); wd 0:
    decay exactly 1; first step from zero state: u = lr_eff * c1 g /
    (sqrt(c2 g^2) + eps)."""
    w = np.array([1.0, -3.5, 1e-30, 7e5], np.float32)
    z = np.zeros(4, np.float32)
    ow = w.copy()
    oracle.adam_step_f32(ow, z.copy(), z.copy(), z.copy(), 3e-4, 0.9, 0.95, 1e-8, 0.1, 1)
    decay = F32(F32(1.0) - F32(F32(3e-4) * F32(0.1)))
    np.testing.assert_array_equal(ow, (w * decay).astype(np.float32))
    g = np.array([1e-3, -2e-2, 5.0, 0.0], np.float32)
    ow, om, ov = w.copy(), z.copy(), z.copy()
    oracle.adam_step_f32(ow, g, om, ov, 3e-4, 0.9, 0.95, 1e-8, 0.0, 1)
    s = py_prologue(3e-4, 0.9, 0.95, 0.0, 1)
    for i in range(4):
        mm = fma32(s["c1"], g[i], F32(0.0))
        vv = fma32(s["c2"], F32(g[i] * g[i]), F32(0.0))
        u = F32(F32(mm / F32(np.sqrt(vv) + F32(1e-8))) * s["lr_eff"])
        assert ow[i] == F32(w[i] - u), i
