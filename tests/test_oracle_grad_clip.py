"""Pins of the oracle's per-tensor clip (ark_asm_grad_clip, opti.s:369-432):
the literal restatement against a second, independent one in Python with an
exactly rounded fma (four lane chains, the faddp pair sums, the scalar
tail, fsqrt); the build's form (canonical f64 tree) and the literal one
bit-identical wherever every partial sum is exact in fp32, so the compare,
division and multiply they share are checked against the reference's
sequence; the build's norm against an exact sum; and the special cases the
instruction sequence fixes (equality does not clip, unordered compares do
not clip, inf clips with coefficient 0, n = 0)."""
import math

import numpy as np
import pytest

import oracle
from test_oracle_adam import fma32

F32 = np.float32


def py_grad_clip_literal(g, thr):
    """opti.s:369-432 in Python, one exactly rounded operation at a time."""
    g = g.copy()
    n = g.size
    acc = [F32(0.0)] * 4
    i = 0
    while i + 4 <= n:                      # fmla v16.4s, v0.4s, v0.4s
        for lane in range(4):
            acc[lane] = fma32(g[i + lane], g[i + lane], acc[lane])
        i += 4
    s = F32(F32(acc[0] + acc[1]) + F32(acc[2] + acc[3]))  # faddp, faddp
    while i < n:                           # fmadd s16, s0, s0, s16
        s = fma32(g[i], g[i], s)
        i += 1
    norm = F32(np.sqrt(s))                 # fsqrt (correctly rounded)
    if norm > thr:                         # fcmp; b.le skips (also unordered)
        c = F32(F32(thr) / norm)           # fdiv
        g = (g * c).astype(F32)            # fmul
    return norm, g


def _bits(x):
    return np.asarray(x, F32).view(np.uint32)


@pytest.mark.parametrize("n", [0, 1, 3, 4, 5, 8, 13, 257, 1001])
def test_literal_matches_an_independent_restatement(n):
    rng = np.random.default_rng(n)
    g = (rng.standard_normal(n) * 10.0 ** rng.uniform(-3, 1, n)).astype(F32)
    for thr in (F32(0.5), F32(1e6)):
        want_norm, want = py_grad_clip_literal(g, thr)
        got = g.copy()
        norm = oracle.grad_clip_literal(got, thr)
        assert _bits(norm) == _bits(want_norm), (n, thr)
        assert np.array_equal(_bits(got), _bits(want)), (n, thr)


@pytest.mark.parametrize("n", [1, 3, 4, 5, 4095, 4096, 4097, 8193, 10001, 40000])
def test_tree_form_equals_the_literal_one_when_every_sum_is_exact(n):
    """Values k/16 with |k| <= 8: every square and every partial sum is a
    multiple of 2^-8 below 2^16, exact in fp32 and f64, so both sums are the
    exact sum and the two forms must agree on every bit, clipped or not."""
    rng = np.random.default_rng(100 + n)
    g = (rng.integers(-8, 9, n) / 16.0).astype(F32)
    exact = float(np.sum(g.astype(np.float64) ** 2))
    for thr in (F32(math.sqrt(exact) * 0.5), F32(math.sqrt(exact) * 2.0 + 1.0)):
        a, b = g.copy(), g.copy()
        na = oracle.grad_clip_literal(a, thr)
        nb = oracle.grad_clip(b, thr)
        assert _bits(na) == _bits(nb) == _bits(F32(np.sqrt(F32(exact)))), (n, thr)
        assert np.array_equal(_bits(a), _bits(b)), (n, thr)
        assert np.array_equal(a, g) == (not na > thr)


@pytest.mark.parametrize("n", [4096, 100_003, 1_572_864])
def test_tree_norm_is_the_exact_norm_rounded_twice(n):
    """The build's norm is fp32(sqrt(fp32(sum))) of the canonical f64 tree:
    within 1e-7 relative of the exact norm (the north star asks 1e-5); the
    literal form's four fp32 chains drift further at this size."""
    rng = np.random.default_rng(n)
    g = (rng.standard_normal(n) * 1e-3).astype(F32)
    exact = math.sqrt(math.fsum((g.astype(np.float64) ** 2).tolist()))
    got = g.copy()
    norm = oracle.grad_clip(got, F32(1e9))
    assert abs(norm - exact) / exact < 1e-7
    assert np.array_equal(got, g)  # not clipped
    lit = oracle.grad_clip_literal(g.copy(), F32(1e9))
    assert abs(lit - exact) / exact < 1e-3


def test_special_cases_follow_the_instruction_sequence():
    for clip in (oracle.grad_clip, oracle.grad_clip_literal):
        # norm exactly equal to the threshold: b.le skips
        g = np.array([0.5, -0.5, 0.5, 0.5], F32)
        assert clip(g, F32(1.0)) == 1.0 and np.array_equal(g, [0.5, -0.5, 0.5, 0.5])
        # one ulp below: clips with coefficient thr / norm
        g = np.array([0.5, -0.5, 0.5, 0.5], F32)
        thr = np.nextafter(F32(1.0), F32(0.0))
        assert clip(g, thr) == 1.0 and np.array_equal(g, np.array([0.5, -0.5, 0.5, 0.5], F32) * thr)
        # a NaN threshold: unordered, no clip
        g = np.array([3.0, 4.0], F32)
        assert clip(g, F32(np.nan)) == 5.0 and np.array_equal(g, [3.0, 4.0])
        # an inf value: norm inf, coefficient 0: finite values to signed zero, inf to NaN
        g = np.array([1.0, -2.0, np.inf, 3.0, -0.0], F32)
        assert clip(g, F32(1.0)) == np.inf
        assert np.isnan(g[2]) and _bits(g[[0, 3, 4]]).tolist() == [0, 0, 0x80000000]
        assert _bits(g[1]) == 0x80000000
        # a NaN value: norm NaN, unordered, untouched
        g = np.array([1.0, np.nan, np.inf], F32)
        assert np.isnan(clip(g, F32(1.0))) and g[0] == 1.0 and g[2] == np.inf
        # all zero under a negative threshold: 0 > thr clips, thr / 0 = -inf, 0 * -inf = NaN
        g = np.zeros(6, F32)
        assert clip(g, F32(-1.0)) == 0.0 and np.isnan(g).all()
    # n = 0: the Rust wrapper returns 0.0 (ffi.rs:208-210), the literal loops do nothing
    assert oracle.grad_clip(np.zeros(0, F32), F32(-1.0)) == 0.0
    assert oracle.grad_clip_literal(np.zeros(0, F32), F32(1.0)) == 0.0


# Inputs found by search where one rounding of the sequence decides the
# result (the bit patterns of the fp32 values).
_PAIRS_DECIDE = [1057502887, 3210889945, 1065743266, 1050315282]  # faddp grouping
_TAIL_DECIDES = [1051120621, 1041376160, 1056077718, 3177181853, 3208315759]  # fused tail
_ROUND_TWICE = [3197436739, 1089882025]  # fp32(sqrt(fp32(s))) != fp32(sqrt(s))


@pytest.mark.parametrize("bits", [_PAIRS_DECIDE, _TAIL_DECIDES])
def test_literal_on_inputs_where_one_rounding_decides(bits):
    """(a0 + a1) + (a2 + a3), not a left fold, and the tail's fmadd, not a
    multiply and an add: each input gives a different norm under the
    other choice; the literal form must equal the independent one."""
    g = np.array(bits, np.uint32).view(F32)
    want, _ = py_grad_clip_literal(g, F32(1e9))
    assert _bits(oracle.grad_clip_literal(g.copy(), F32(1e9))) == _bits(want)


def test_tree_norm_rounds_the_sum_to_fp32_before_the_root():
    """optimizer.rs:145 and opti.s:399 take the root of an fp32 sum; the
    build's form rounds the f64 sum to fp32 first, which differs here from
    rounding the f64 root."""
    g = np.array(_ROUND_TWICE, np.uint32).view(F32)
    s = float(g[0]) ** 2 + float(g[1]) ** 2  # the tree of two values, exact in f64
    want = F32(np.sqrt(F32(s)))
    assert want != F32(np.sqrt(s))
    assert _bits(oracle.grad_clip(g.copy(), F32(1e9))) == _bits(want)


def test_zero_norm_at_a_zero_threshold_does_not_clip():
    """norm == thr == 0: b.le skips; clipping would make 0 / 0 a NaN
    coefficient."""
    for clip in (oracle.grad_clip, oracle.grad_clip_literal):
        g = np.zeros(9, F32)
        assert clip(g, F32(0.0)) == 0.0 and not np.isnan(g).any()


def test_random_device_cases_reach_every_outcome():
    """The 30 seeded cases tests/test_gpu_grad_clip.py runs on the device,
    replayed through the oracle: among them calls that clip, calls that do
    not, an inf norm, a NaN norm, and norms far from 1 either way."""
    from test_gpu_grad_clip import random_case
    seen = set()
    for case in range(30):
        h, thr, _ = random_case(case)
        g = h.copy()
        norm = oracle.grad_clip(g, F32(thr))
        if np.isnan(norm):
            seen.add("nan")
        elif np.isinf(norm):
            seen.add("inf")
        else:
            seen.add("clipped" if norm > F32(thr) else "kept")
            seen.add("tiny" if norm < 1e-20 else "huge" if norm > 1e10 else "mid")
    assert {"nan", "inf", "clipped", "kept", "tiny", "huge", "mid"} <= seen, seen
