"""Pins of the oracle's global-norm clip (Optimizer::clip_all_grads,
optimizer.rs:126-168): the strict `norm > grad_clip` at the threshold (:148),
no clipping below it or for an all-zero gradient, the coefficient
grad_clip / norm, the closed form that the clipped gradient's norm equals
the threshold up to rounding, and the clipped step equal to an unclipped
step on the already-clipped gradients."""
import numpy as np
import pytest

import oracle
from ark_amd import _abi

SCALE = 1024.0  # a power of two: g16 * (1 / SCALE) is exact


def _hp(clip, scale=SCALE, grad_dtype=_abi.GRAD_F16):
    hp = oracle.default_hparams()
    hp.beta2 = 0.95
    hp.grad_clip = clip
    hp.loss_scale_init = scale
    hp.loss_scale_max = 2.0 ** 24
    hp.grad_dtype = grad_dtype
    return hp


def _step(true_grads, clip):
    """One step over one tensor whose unscaled gradient is `true_grads`
    (values exact in fp16 after scaling by SCALE)."""
    g = np.asarray(true_grads, np.float64) * SCALE
    g16 = g.astype(np.float16)
    assert np.array_equal(g16.astype(np.float64), g), "test values must be exact in fp16"
    n = g.size
    t = oracle.HostTensor(np.full(n, 0x3C00, np.uint16), g16.view(np.uint16).copy(),
                          np.zeros(n, np.float32), np.zeros(n, np.float32), 0.1)
    _, info = oracle.Optimizer([t], _hp(clip)).step(3e-4)
    assert info.applied == 1
    return info, t


def test_norm_equal_to_the_threshold_does_not_clip():
    # four halves: sum of squares exactly 1.0, norm exactly 1.0
    info, _ = _step([0.5, -0.5, 0.5, 0.5], clip=1.0)
    assert info.grad_norm == 1.0
    assert info.clipped == 0 and info.clip_coef == 1.0


def test_just_above_clips_with_coefficient_clip_over_norm():
    x = 1.0 + 2.0 ** -10
    info, _ = _step([x], clip=1.0)
    assert info.grad_norm == np.float32(x)
    assert info.clipped == 1
    assert info.clip_coef == np.float32(1.0) / np.float32(x)


def test_just_below_and_zero_do_not_clip():
    info, _ = _step([1.0 - 2.0 ** -11], clip=1.0)
    assert info.clipped == 0 and info.clip_coef == 1.0
    info, _ = _step([0.0] * 9, clip=1.0)  # norm 0: `norm > 0` fails too (:148)
    assert info.grad_norm == 0.0 and info.clipped == 0 and info.clip_coef == 1.0


@pytest.mark.parametrize("clip", [1.0, 0.25, 3.0])
def test_clipped_norm_equals_the_threshold(clip):
    """sqrt(sum((g * inv * coef)^2)) == clip within a few fp32 ulps."""
    rng = np.random.default_rng(int(clip * 100))
    g = (rng.standard_normal(20000) * 0.05 * SCALE).astype(np.float16)
    n = g.size
    t = oracle.HostTensor(np.zeros(n, np.uint16), g.view(np.uint16).copy(),
                          np.zeros(n, np.float32), np.zeros(n, np.float32), 0.0)
    _, info = oracle.Optimizer([t], _hp(clip)).step(3e-4)
    assert info.clipped == 1
    eff = (g.astype(np.float32) * np.float32(1.0 / SCALE)) * np.float32(info.clip_coef)
    norm = np.sqrt(np.sum(eff.astype(np.float64) ** 2))
    assert abs(norm - clip) <= 4 * np.spacing(np.float32(clip)), (norm, clip)


def test_clipped_step_equals_unclipped_step_on_clipped_gradients():
    """Stepping loss-scaled fp16 gradients that clip gives the same w/m/v
    bits as stepping, unscaled and with no clip, the fp32 gradients
    (g16 * inv) * coef: the clip is one multiply of the unscaled gradient
    by grad_clip / norm, ahead of AdamW (optimizer.rs:151-165, :216-226)."""
    rng = np.random.default_rng(9)
    n = 5000
    g = (rng.standard_normal(n) * 0.1 * SCALE).astype(np.float16)
    w = (rng.standard_normal(n) * 0.02).astype(np.float16).view(np.uint16)
    a = oracle.HostTensor(w.copy(), g.view(np.uint16).copy(), np.zeros(n, np.float32),
                          np.zeros(n, np.float32), 0.1)
    _, ia = oracle.Optimizer([a], _hp(1.0)).step(3e-4)
    assert ia.clipped == 1 and ia.clip_coef < 1.0
    eff = (g.astype(np.float32) * np.float32(1.0 / SCALE)) * np.float32(ia.clip_coef)
    b = oracle.HostTensor(w.copy(), eff.copy(), np.zeros(n, np.float32), np.zeros(n, np.float32),
                          0.1)
    _, ib = oracle.Optimizer([b], _hp(1e30, scale=1.0, grad_dtype=_abi.GRAD_F32)).step(3e-4)
    assert ib.clipped == 0
    assert np.array_equal(a.w, b.w)
    assert np.array_equal(a.m.view(np.uint32), b.m.view(np.uint32))
    assert np.array_equal(a.v.view(np.uint32), b.v.view(np.uint32))


def test_finalize_then_elementwise_update_is_the_step():
    """ark_ref_finalize (the step's scalars from a given sum of squares) and
    ark_ref_apply_given (the elementwise update from those scalars) together
    reproduce ark_ref_opt_step: 60 steps over three tensors with clipped,
    unclipped and non-finite steps, loss-scale growth, and an early stop.
    The full-size AMP stress test checks the device's scalars with this
    split, the sum taken once per distinct loss scale."""
    from oracle import harness as H
    rng = np.random.default_rng(41)
    sizes = [3000, 257, 64]
    hp = _hp(1.0, scale=2.0 ** 12)
    hp.scale_up_every = 7
    hp.max_consecutive_nonfinite = 3
    mk = lambda: [oracle.HostTensor((rng.standard_normal(n) * 0.02).astype(np.float16)
                                    .view(np.uint16), np.zeros(n, np.uint16),
                                    np.zeros(n, np.float32), np.zeros(n, np.float32),
                                    0.1 if k else 0.0) for k, n in enumerate(sizes)]
    a = mk()
    b = [t.copy() for t in a]
    ra = oracle.Optimizer(a, hp)
    st = _abi.State()
    oracle.lib().ark_ref_state_init(hp, st)
    bad_at = {5, 6, 20, 40, 41, 42, 43}  # 40-43: four in a row, past the limit of 3
    seen = set()
    for k in range(60):
        sig = float(10.0 ** rng.uniform(-4, -1)) * hp.loss_scale_init
        for ta, tb in zip(a, b):
            ta.g[:] = (rng.standard_normal(ta.n) * sig).astype(np.float16).view(np.uint16)
            if k in bad_at:
                ta.g[int(rng.integers(ta.n))] = 0x7E00
            tb.g[:] = ta.g
        sa, ia = ra.step(3e-4)
        inv = np.float32(1.0) / np.float32(st.loss_scale)
        sq, bad = oracle.sumsq(b, _abi.GRAD_F16, inv) if not st.early_stop else (0.0, False)
        sb, ib = oracle.finalize(hp, st, sq, bad, 3e-4)
        oracle.Optimizer(b, hp).apply_given(3e-4, st.t, ib)
        assert sa == sb and not H.info_matches(ia, ib), (k, H.info_matches(ia, ib))
        seen.add((ia.applied, ia.clipped, sa))
        for ta, tb in zip(a, b):
            assert np.array_equal(ta.w, tb.w) and np.array_equal(ta.m.view(np.uint32),
                                                                  tb.m.view(np.uint32))
            assert np.array_equal(ta.v.view(np.uint32), tb.v.view(np.uint32))
    assert ra.state.early_stop == 1 and ra.state.skipped_steps == 7
    # applied clipped and unclipped, skipped, and stopped steps all occurred
    assert {(1, 1, 0), (1, 0, 0), (0, 0, 0), (0, 0, _abi.EARLY_STOP)} <= seen, seen
