"""Host-side mirror of the reference's optimizer interface: the EKO
parameter-buffer set (tensor order, shapes, weight decay), the learning-rate
schedule and the device arena layout, all on the CPU."""
import numpy as np
import pytest

from ark_amd import _abi
from ark_amd.eko import EKO_1P3B, EKO_237M, EKO_LAYER, EkoConfig, config_tensors
from ark_amd.optimizer import AdamConfig, ParamSet, lr_now


def reference_param_count(cfg: EkoConfig):
    """Config::estimate_params (config.rs:184-194): embed v*d + d, per layer
    4 d^2 + 3 d h + 2 d."""
    d, h, v, l = cfg.d_model, cfg.hidden, cfg.vocab, cfg.n_layers
    return v * d + d + (d * d * 4 + d * h * 3 + d * 2) * l


def test_parameter_counts_match_reference_formula_and_baseline():
    assert EKO_237M.n_params() == reference_param_count(EKO_237M) == 236_959_488
    assert len(EKO_237M.tensors()) == 272
    assert EKO_1P3B.n_params() == reference_param_count(EKO_1P3B) == 1_279_887_360
    assert len(EKO_1P3B.tensors()) == 218
    c1 = config_tensors("c1")
    assert len(c1) == 9 and sum(t.n for t in c1) == 7_079_424
    assert sum(t.n for t in config_tensors("c0")) == 589_824
    # the trained model's vocabulary (CHANGELOG.md:648: 237.19603 M)
    assert reference_param_count(EkoConfig(30, 768, 2048, 32308)) == 237_196_032


def test_tensor_order_and_weight_decay_follow_step_all():
    """optimizer.rs:185-227: embed (wd), gamma_final (no wd), then per layer
    wq wk wv wo w1 w2 w3 (wd) and g1 g2 (no wd); shapes memory.rs:227-255."""
    ts = EKO_237M.tensors()
    assert [t.name for t in ts[:11]] == ["embed", "gamma_final", "l0.wq", "l0.wk", "l0.wv",
                                         "l0.wo", "l0.w1", "l0.w2", "l0.w3", "l0.g1", "l0.g2"]
    assert [t.decay for t in ts[:11]] == [True, False] + [True] * 7 + [False] * 2
    assert ts[6].shape == (768, 2048) and ts[7].shape == (2048, 768)
    assert all(t.gain == (not t.decay) for t in ts)


def test_lr_schedule_mirrors_lr_now():
    """optimizer.rs:80-92 with step already incremented (:172-173)."""
    cfg = AdamConfig(lr=3e-4, warmup_steps=100)
    f = np.float32
    assert lr_now(cfg, 1) == float(f(3e-4) * f(2.0) / f(100.0))
    assert lr_now(cfg, 99) == float(f(3e-4) * f(100.0) / f(100.0))
    assert lr_now(cfg, 100) == pytest.approx(3e-4, rel=1e-6)         # cosine at 0
    assert lr_now(cfg, 100 + 400_000) == pytest.approx(1.65e-4, rel=1e-5)  # half way
    assert lr_now(cfg, 100 + 800_000) == pytest.approx(3e-5, rel=1e-5)     # floor lr/10
    assert lr_now(cfg, 5_000_000) == pytest.approx(3e-5, rel=1e-5)


def test_param_arena_layout_on_cpu():
    ps = ParamSet(EKO_LAYER.tensors(with_embedding=False, with_gamma_final=False), 0.1,
                  device="cpu", no_unscale=("l0.g2",))
    tab = ps.table()
    assert len(tab) == 9
    base_w = ps.w_arena.data_ptr()
    for i, t in enumerate(tab):
        assert (t.w - base_w) % 256 == 0 and (t.m - ps.m_arena.data_ptr()) % 512 == 0
        assert t.n == ps.specs[i].n
        assert t.weight_decay == float(np.float32(0.1 if ps.specs[i].decay else 0.0))
    assert tab[8].flags == _abi.TENSOR_NO_UNSCALE and tab[7].flags == 0
    assert ps.n_params == 7_079_424
