"""Pins of the oracle's fp16 <-> fp32 conversions (the fcvtl / fcvtn of
opti.s:279, :307, :318, :345 under the default FPCR: round to nearest even,
fp16 subnormals kept, overflow to infinity) against two independent
converters: x86 F16C hardware (exhaustive) and numpy's software conversion."""
import os

import numpy as np
import pytest

import oracle


def _f16c():
    r = oracle.lib().ark_ref_check_f16_to_f32_f16c()
    if r < 0:
        pytest.skip("no F16C on this host")
    return r


def test_f16_to_f32_exhaustive_vs_numpy():
    h = np.arange(65536, dtype=np.uint16)
    a = oracle.f16_to_f32(h)
    b = h.view(np.float16).astype(np.float32)
    nan = np.isnan(b)
    assert np.array_equal(np.isnan(a), nan)
    assert np.array_equal(a[~nan].view(np.uint32), b[~nan].view(np.uint32))


def test_f16_to_f32_exhaustive_vs_f16c():
    assert _f16c() == 0


def test_f32_to_f16_all_inputs_vs_f16c():
    """All 2^32 fp32 bit patterns against vcvtps2ph in RNE (a few seconds)."""
    _f16c()
    n = min(16, os.cpu_count() or 1)
    assert oracle.lib().ark_ref_check_f32_to_f16_f16c(0, 1 << 32, n) == 0


def test_f32_to_f16_sample_vs_numpy():
    rng = np.random.default_rng(7)
    x = rng.integers(0, 2 ** 32, 1 << 22, dtype=np.uint64).astype(np.uint32).view(np.float32)
    a = oracle.f32_to_f16(x)
    with np.errstate(over="ignore"):
        b = x.astype(np.float16).view(np.uint16)
    an, bn = (a & 0x7FFF) > 0x7C00, (b & 0x7FFF) > 0x7C00
    assert np.array_equal(an, bn)
    assert np.array_equal(a[~an], b[~an])


@pytest.mark.parametrize("x,bits", [
    (1.0, 0x3C00),
    (-0.0, 0x8000),
    (65504.0, 0x7BFF),            # largest finite
    (65519.99609375, 0x7BFF),     # just below the tie: rounds down
    (65520.0, 0x7C00),            # tie between 65504 (odd) and 2^16: to even -> inf
    (2.0 ** -14, 0x0400),         # smallest normal
    (2.0 ** -24, 0x0001),         # smallest subnormal
    (2.0 ** -25, 0x0000),         # tie between 0 and 2^-24: to even -> 0
    (3 * 2.0 ** -26, 0x0001),     # above the tie
    (1 + 2.0 ** -11, 0x3C00),     # tie between 1 and 1+2^-10: to even (down)
    (1 + 3 * 2.0 ** -11, 0x3C02), # tie between 0x3C01 and 0x3C02: to even (up)
    (float("inf"), 0x7C00),
    (-1e30, 0xFC00),
    (1e-45, 0x0000),              # fp32 subnormal
])
def test_f32_to_f16_known_answers(x, bits):
    assert int(oracle.f32_to_f16(np.array([x], np.float32))[0]) == bits


def test_nan_stays_nan_both_ways():
    assert np.isnan(oracle.f16_to_f32(np.array([0x7E00, 0xFC01], np.uint16))).all()
    h = oracle.f32_to_f16(np.array([np.nan, -np.nan], np.float32))
    assert np.all((h & 0x7FFF) > 0x7C00)


def test_splitmix64_known_answer():
    """The published SplitMix64 sequence from state 1234567 (Vigna's
    reference generator; also java.util.SplittableRandom's mixer)."""
    assert oracle.splitmix64_seq(1234567, 5) == [
        6457827717110365317, 3203168211198807973, 9817491932198370423,
        4593380528125082431, 16408922859458223821]


def test_generator_constant_and_moments():
    """z = d * K with K = fp32(sqrt(3)/131072): mean 0, variance 1 (Irwin-Hall
    of four 16-bit uniforms), support |z| <= sqrt(12); independent streams per
    (tensor, step)."""
    assert np.float32(np.sqrt(3.0) / 131072.0) == np.float32(float.fromhex("0x1.bb67aep-17"))
    z = oracle.synth_normal_f32(1 << 21, 42, 5, 9, 1.0).astype(np.float64)
    assert abs(z.mean()) < 3e-3 and abs(z.var() - 1.0) < 3e-3
    assert np.abs(z).max() <= np.sqrt(12.0)
    a = oracle.synth_normal_f32(1000, 42, 5, 10, 1.0)
    b = oracle.synth_normal_f32(1000, 42, 6, 9, 1.0)
    c = oracle.synth_normal_f32(1000, 42, 5, 9, 1.0)
    assert np.array_equal(c, z[:1000].astype(np.float32))
    assert not np.array_equal(a, c) and not np.array_equal(b, c)


def test_generator_f16_is_rounded_f32():
    """fp16 output = RNE of the fp32 value (one rounding after the fp32
    product, never a fused single rounding)."""
    f = oracle.synth_normal_f32(1 << 16, 1, 2, 3, 65.536)
    h = oracle.synth_normal_f16(1 << 16, 1, 2, 3, 65.536)
    assert np.array_equal(h, f.astype(np.float16).view(np.uint16))
