"""GPU parity: the HIP path through the C ABI against the CPU oracle, bit for
bit (scalars of every step, every w/m/v element), at configurations c0 and
c1 and at edge cases of the reference kernel (opti.s:192-360) and the AMP
state machine (training.rs:289-326)."""
import ctypes as C

import numpy as np
import pytest

import oracle
from oracle import harness as H
from ark_amd import _abi
from ark_amd.eko import TensorSpec, config_tensors

pytestmark = pytest.mark.gpu

HP = dict(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1, grad_clip=1.0)


def _torch():
    import torch
    assert torch.cuda.is_available(), "GPU test run without a GPU"
    return torch


def _make(specs, seed, sig, scale, grad_dtype=_abi.GRAD_F16, no_unscale=(), **over):
    from ark_amd.optimizer import AdamConfig, AmpConfig, Optimizer
    hp = dict(HP)
    hp.update({k: v for k, v in over.items() if k in hp})
    amp_kw = {k: v for k, v in over.items() if k in AmpConfig.__dataclass_fields__}
    cfg = AdamConfig(**hp)
    amp = AmpConfig(**{"loss_scale_init": scale, "loss_scale_max": 2.0 ** 24, **amp_kw})
    ps = H.gpu_problem(specs, seed, cfg.weight_decay, sig, scale, grad_dtype=grad_dtype,
                       no_unscale=no_unscale)
    ts = H.host_problem(specs, seed, cfg.weight_decay, sig, scale, grad_dtype=grad_dtype,
                        no_unscale=no_unscale)
    opt = Optimizer(cfg, ps, amp)
    ref = oracle.Optimizer(ts, opt.hp, nthreads=8)
    return cfg, ps, ts, opt, ref


def _set_bits(t, pos, bits):
    """Write fp16 bit pattern `bits` at t[pos] (t: torch.float16 on the GPU)."""
    import torch
    t.view(torch.int16)[pos] = int(np.array(bits, np.uint16).view(np.int16))


def _run_steps(ps, ts, opt, ref, seed, sig, scale, steps, lr, check_every=1):
    last = None
    for k in range(steps):
        if k:
            H.gpu_regen_grads(ps, seed, sig, scale, k)
            H.host_regen_grads(ts, seed, sig, scale, k, grad_dtype=ps.grad_dtype)
        _, gi = opt.step_all(lr, info=True)
        _, ri = ref.step(lr)
        d = H.info_matches(gi, ri)
        assert not d, f"step {k}: scalars differ: {d}"
        if (k + 1) % check_every == 0 or k == steps - 1:
            c = H.compare(ps, ts)
            assert c["w"] == 0 and c["m"] == 0 and c["v"] == 0, f"step {k}: {c}"
        last = gi
    return last


def test_synth_generator_matches_oracle():
    torch = _torch()
    for n, tid, step, ss in [(1, 0, 0, 1.0), (4099, 3, 17, 0.02), (1 << 20, 271, 4999, 65.536)]:
        a = torch.empty(n, dtype=torch.float16, device="cuda")
        from ark_amd import synth
        synth.normal_f16(a, 1234, tid, step, ss)
        b = oracle.synth_normal_f16(n, 1234, tid, step, ss)
        assert np.array_equal(H.to_host(a), b)
        f = torch.empty(n, dtype=torch.float32, device="cuda")
        synth.normal_f32(f, 99, tid, step, ss)
        assert np.array_equal(H.to_host(f).view(np.uint32),
                              oracle.synth_normal_f32(n, 99, tid, step, ss).view(np.uint32))


def test_calibration_copy_kernel():
    torch = _torch()
    from ark_amd import synth
    src = torch.arange(1 << 20, dtype=torch.int32, device="cuda")
    dst = torch.zeros_like(src)
    synth.copy(dst, src)
    assert torch.equal(dst, src)


def test_config0_ten_steps_bit_exact():
    """Configuration c0: one 768x768 tensor, grads N(0,1e-3)*1024 fresh per step,
    10 steps; norm ~0.77 so no clipping."""
    specs = config_tensors("c0")
    sig = [1e-3]
    cfg, ps, ts, opt, ref = _make(specs, 11, sig, 1024.0)
    last = _run_steps(ps, ts, opt, ref, 11, sig, 1024.0, 10, cfg.lr)
    assert last.state.t == 10 and last.clipped == 0
    opt.close()


def test_config1_layer_hundred_steps_bit_exact():
    """Configuration c1: one EKO layer (9 tensors, g1/g2 = 1.0 without wd), 100
    steps; norm ~2.66 so every step clips."""
    specs = config_tensors("c1")
    sig = [1e-3] * len(specs)
    cfg, ps, ts, opt, ref = _make(specs, 5, sig, 1024.0)
    last = _run_steps(ps, ts, opt, ref, 5, sig, 1024.0, 100, cfg.lr, check_every=10)
    assert last.state.t == 100 and last.clipped == 1
    opt.close()


@pytest.mark.parametrize("grad_dtype", [_abi.GRAD_F16, _abi.GRAD_F32])
def test_norm_blocking_does_not_change_bits(grad_dtype, monkeypatch):
    """1, 2, 4 or 8 segments per norm block (with ragged and unaligned
    tensors, so fast and element-wise blocks mix), and any cap on the norm
    blocks a CU holds at once, give the same bits: the sum follows the
    canonical tree whatever the blocking and residency."""
    torch = _torch()
    specs = config_tensors("c1") + [TensorSpec("r", (4096 * 70 + 3,), True, False),
                                    TensorSpec("s", (5,), False, True)]
    sig = [1e-3] * len(specs)
    base = None
    for spb, cap in (("1", None), ("2", None), ("4", None), ("8", None),
                     ("2", "0"), ("2", "2"), ("8", "2"), ("2", "8")):
        monkeypatch.setenv("ARK_OPT_SUMSQ_SPB", spb)
        if cap is None:
            monkeypatch.delenv("ARK_OPT_SUMSQ_BLOCKS_PER_CU", raising=False)
        else:
            monkeypatch.setenv("ARK_OPT_SUMSQ_BLOCKS_PER_CU", cap)
        cfg, ps, ts, opt, ref = _make(specs, 21, sig, 4096.0, grad_dtype=grad_dtype)
        _, gi = opt.step_all(cfg.lr, info=True)
        _, ri = ref.step(cfg.lr)
        assert not H.info_matches(gi, ri), (spb, cap)
        base = base or gi.grad_sumsq
        assert gi.grad_sumsq == base
        opt.close()


@pytest.mark.parametrize("cap", ["0", "4", "16", "32"])
def test_adamw_residency_does_not_change_bits(cap, monkeypatch):
    """Any cap on the one-wave AdamW blocks a CU holds at once (none, the
    fewest allowed, the default, every wave slot) gives every w/m/v bit of
    the oracle's, on ragged and unaligned tensors too."""
    monkeypatch.setenv("ARK_OPT_ADAMW_BLOCKS_PER_CU", cap)
    specs = config_tensors("c1") + [TensorSpec("r", (4096 * 5 + 3,), True, False),
                                    TensorSpec("s", (5,), False, True)]
    sig = [1e-3] * len(specs)
    cfg, ps, ts, opt, ref = _make(specs, 31, sig, 2048.0)
    _run_steps(ps, ts, opt, ref, 31, sig, 2048.0, 2, cfg.lr)
    opt.close()


def test_ragged_and_tiny_tensors():
    specs = [TensorSpec("a", (1,), True, False), TensorSpec("b", (7,), False, True),
             TensorSpec("c", (4095,), True, False), TensorSpec("d", (4097,), True, False),
             TensorSpec("e", (8 * 4096 + 13,), True, False), TensorSpec("f", (2048 + 8,), False, False)]
    sig = [1e-3, 1e-2, 1e-3, 1e-4, 1e-3, 1e-3]
    cfg, ps, ts, opt, ref = _make(specs, 3, sig, 256.0)
    _run_steps(ps, ts, opt, ref, 3, sig, 256.0, 4, cfg.lr)
    opt.close()


def test_empty_tensors_in_the_table():
    """Zero-length tensors among others contribute nothing and are skipped;
    a table of only empty tensors still runs the AMP state machine (norm 0,
    the step counts as applied, as the reference's loop over empty slices)."""
    specs = [TensorSpec("z0", (0,), True, False), TensorSpec("a", (5,), True, False),
             TensorSpec("z1", (0,), False, True), TensorSpec("b", (4096,), True, False),
             TensorSpec("z2", (0,), True, False)]
    sig = [1e-3] * len(specs)
    cfg, ps, ts, opt, ref = _make(specs, 6, sig, 512.0)
    _run_steps(ps, ts, opt, ref, 6, sig, 512.0, 3, cfg.lr)
    opt.close()
    specs = [TensorSpec("z0", (0,), True, False), TensorSpec("z1", (0,), False, True)]
    cfg, ps, ts, opt, ref = _make(specs, 6, [1e-3, 1e-3], 512.0)
    last = _run_steps(ps, ts, opt, ref, 6, [1e-3, 1e-3], 512.0, 3, cfg.lr)
    assert last.applied == 1 and last.grad_norm == 0.0 and last.state.t == 3
    opt.close()


def test_fp32_gradients():
    specs = [TensorSpec("a", (3000,), True, False), TensorSpec("b", (768,), False, True)]
    sig = [1e-3, 1e-3]
    cfg, ps, ts, opt, ref = _make(specs, 8, sig, 1000.0, grad_dtype=_abi.GRAD_F32)
    _run_steps(ps, ts, opt, ref, 8, sig, 1000.0, 3, cfg.lr)
    opt.close()


def test_no_unscale_flag_reproduces_gamma_final_quirk():
    """training.rs:133-146 leaves gamma_final scaled; the flag reproduces it."""
    specs = [TensorSpec("embed", (64, 128), True, False),
             TensorSpec("gamma_final", (128,), False, True)]
    sig = [1e-3, 1e-3]
    cfg, ps, ts, opt, ref = _make(specs, 4, sig, 512.0, no_unscale=("gamma_final",))
    last = _run_steps(ps, ts, opt, ref, 4, sig, 512.0, 2, cfg.lr)
    assert last.clipped == 1  # the scaled gain dominates the norm
    opt.close()


def test_nonfinite_skip_and_recovery():
    """training.rs:293-305: inf/NaN -> halve the scale, no update, t kept."""
    torch = _torch()
    specs = [TensorSpec("a", (5000,), True, False), TensorSpec("b", (768,), False, True)]
    sig = [1e-3, 1e-3]
    cfg, ps, ts, opt, ref = _make(specs, 9, sig, 65536.0)
    w0 = H.to_host(ps.w(0)).copy()
    for bits, ti, pos in [(0x7C00, 0, 4999), (0xFC00, 1, 0), (0x7E01, 0, 1234)]:
        _set_bits(ps.g(ti), pos, bits)
        ts[ti].g[pos] = bits
        _, gi = opt.step_all(cfg.lr, info=True)
        _, ri = ref.step(cfg.lr)
        assert not H.info_matches(gi, ri)
        assert gi.applied == 0 and gi.nonfinite == 1 and gi.state.t == 0
        H.gpu_regen_grads(ps, 9, sig, 65536.0, 0)
        H.host_regen_grads(ts, 9, sig, 65536.0, 0)
    assert np.array_equal(H.to_host(ps.w(0)), w0)
    assert gi.state.loss_scale == 8192.0 and gi.state.skipped_steps == 3
    _, gi = opt.step_all(cfg.lr, info=True)
    _, ri = ref.step(cfg.lr)
    assert not H.info_matches(gi, ri) and gi.applied == 1 and gi.state.t == 1
    assert gi.state.consecutive_nonfinite == 0
    c = H.compare(ps, ts)
    assert c["w"] == c["m"] == c["v"] == 0
    opt.close()


def test_growth_cap_and_early_stop():
    """Growth every scale_up_every clean steps up to the cap with the counter
    reset even when capped (training.rs:319-326); early stop after more than
    max_consecutive_nonfinite skips, sticky (training.rs:298-301)."""
    torch = _torch()
    specs = [TensorSpec("a", (256,), True, False)]
    sig = [1e-3]
    cfg, ps, ts, opt, ref = _make(specs, 2, sig, 8.0, scale_up_every=3,
                                  max_consecutive_nonfinite=4, loss_scale_max=32.0)
    for k in range(12):
        _, gi = opt.step_all(cfg.lr, info=True)
        _, ri = ref.step(cfg.lr)
        assert not H.info_matches(gi, ri)
    assert gi.state.loss_scale == 32.0
    _set_bits(ps.g(0), 7, 0x7C00)
    ts[0].g[7] = 0x7C00
    codes = []
    for k in range(7):
        rc, gi = opt.step_all(cfg.lr, info=True)
        rrc, ri = ref.step(cfg.lr)
        assert rc == rrc and not H.info_matches(gi, ri)
        codes.append(rc)
    assert codes == [0, 0, 0, 0, 1, 1, 1]
    assert gi.state.early_stop == 1 and gi.state.skipped_steps == 5
    opt.close()


@pytest.mark.parametrize("scale", [1.0, 3.0])
def test_finite_flag_every_fp16_pattern(scale):
    """training.rs:291 on the device, exhaustively: each of the 2048 inf/NaN
    fp16 patterns, alone among zeros, makes the step skip -- placed in a
    tensor of eight full segments (one norm block of vector loads) or in a
    ragged one (mixed block, element-wise tail) at varying positions; and a
    tensor holding all 63,488 finite patterns applies, with every scalar and
    every w/m/v bit equal to the oracle's.  At a power-of-two loss scale
    (full blocks take the squares from the fp16 bits and find a non-finite
    gradient from their sum) and at one that is not (a per-element test);
    the minimum scale keeps the skips from halving it."""
    torch = _torch()
    from ark_amd.optimizer import AdamConfig, AmpConfig, Optimizer, ParamSet
    allp = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    nonfin = allp[(allp & 0x7C00) == 0x7C00]
    finite = allp[(allp & 0x7C00) != 0x7C00]
    assert nonfin.size == 2048 and finite.size == 63488
    cfg = AdamConfig(**HP)
    amp = AmpConfig(loss_scale_init=scale, loss_scale_min=scale,
                    max_consecutive_nonfinite=1 << 30)
    specs = [TensorSpec("full", (8 * 4096,), True, False), TensorSpec("ragged", (4133,), True, False)]
    ps = ParamSet(specs, cfg.weight_decay)
    opt = Optimizer(cfg, ps, amp)
    gi = None
    for i, p in enumerate(nonfin):
        t = i & 1
        pos = (i * 131) % specs[t].n if t == 0 else (i * 97) % specs[t].n
        g = ps.g(t).view(torch.int16)
        g[pos] = int(np.array(p, np.uint16).view(np.int16))
        _, gi = opt.step_all(cfg.lr, info=True)
        assert gi.applied == 0 and gi.nonfinite == 1, (hex(int(p)), t, pos)
        g[pos] = 0
    assert gi.state.skipped_steps == 2048 and gi.state.t == 0
    opt.close()

    n = finite.size
    specs = [TensorSpec("finite", (n,), True, False)]
    rng = np.random.default_rng(3)
    w = (rng.standard_normal(n) * 0.02).astype(np.float16).view(np.uint16)
    g = rng.permutation(finite)
    ps = ParamSet(specs, cfg.weight_decay)
    ps.w(0).copy_(torch.from_numpy(w.view(np.int16)).view(torch.float16))
    ps.g(0).copy_(torch.from_numpy(g.view(np.int16)).view(torch.float16))
    ts = [oracle.HostTensor(w.copy(), g.copy(), np.zeros(n, np.float32), np.zeros(n, np.float32),
                            cfg.weight_decay)]
    opt = Optimizer(cfg, ps, AmpConfig(loss_scale_init=scale, loss_scale_min=scale))
    ref = oracle.Optimizer(ts, opt.hp)
    _, gi = opt.step_all(cfg.lr, info=True)
    _, ri = ref.step(cfg.lr)
    assert gi.applied == 1 and gi.nonfinite == 0
    assert not H.info_matches(gi, ri)
    c = H.compare(ps, ts)
    assert c["w"] == c["m"] == c["v"] == 0, c
    opt.close()


# Powers of two inside and just outside 2^-100..2^100 (the norm pass takes
# the squares straight from the fp16 bits inside that range and unscales
# each element first outside it) and scales that are not powers of two.
NORM_SCALES = [1.0, 65536.0, 2.0 ** -20, 2.0 ** 100, 2.0 ** -100, 2.0 ** 101, 2.0 ** -101,
               3.0, 1000.0, 0.75, 65535.0]


@pytest.mark.parametrize("scale", NORM_SCALES)
def test_norm_bits_every_fp16_pattern_every_scale_kind(scale):
    """The step's scalars (the f64 sum of squares included) and every w/m/v
    bit against the oracle with all 63,488 finite fp16 gradient patterns:
    once in 16 full aligned segments (vector loads), once in a ragged tensor
    (element-wise tail) and once in a NO_UNSCALE tensor, at each loss scale
    (optimizer.rs:141-146, training.rs:244)."""
    torch = _torch()
    from ark_amd.optimizer import AdamConfig, AmpConfig, Optimizer, ParamSet
    allp = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    finite = allp[(allp & 0x7C00) != 0x7C00]
    rng = np.random.default_rng(int(np.float64(scale).view(np.uint64) % 1000))
    full = rng.permutation(np.concatenate([finite, np.zeros(2048, np.uint16)]))
    grads = [full, rng.permutation(finite)[:4096 * 3 + 17], rng.permutation(finite)[:4096]]
    specs = [TensorSpec("full", (full.size,), True, False),
             TensorSpec("ragged", (grads[1].size,), True, False),
             TensorSpec("gain", (4096,), False, True)]
    cfg = AdamConfig(**HP)
    amp = AmpConfig(loss_scale_init=scale, loss_scale_min=min(1.0, scale),
                    loss_scale_max=2.0 ** 120)
    ps = ParamSet(specs, cfg.weight_decay, no_unscale=("gain",))
    ts = []
    for i, (s, g) in enumerate(zip(specs, grads)):
        w = (rng.standard_normal(s.n) * 0.02).astype(np.float16).view(np.uint16)
        ps.w(i).copy_(torch.from_numpy(w.view(np.int16)).view(torch.float16))
        ps.g(i).copy_(torch.from_numpy(g.view(np.int16)).view(torch.float16))
        ts.append(oracle.HostTensor(w.copy(), g.copy(), np.zeros(s.n, np.float32),
                                    np.zeros(s.n, np.float32),
                                    cfg.weight_decay if s.decay else 0.0,
                                    _abi.TENSOR_NO_UNSCALE if s.name == "gain" else 0))
    opt = Optimizer(cfg, ps, amp)
    ref = oracle.Optimizer(ts, opt.hp)
    _, gi = opt.step_all(cfg.lr, info=True)
    _, ri = ref.step(cfg.lr)
    assert gi.applied == 1 and gi.nonfinite == 0, scale
    assert not H.info_matches(gi, ri), (scale, H.info_matches(gi, ri))
    c = H.compare(ps, ts)
    assert c["w"] == c["m"] == c["v"] == 0, (scale, c)
    opt.close()


@pytest.mark.parametrize("bits,skips", [(0x7F800000, 1), (0xFF800000, 1), (0x7FC00000, 1),
                                        (0x7F800001, 1), (0xFFFFFFFF, 1), (0x7F7FFFFF, 0),
                                        (0x00000001, 0)])
def test_fp32_gradient_special_values(bits, skips):
    """ARK_OPT_GRAD_F32 (the reference's own fp32 gradients): infinities
    and quiet, signalling and negative NaNs skip the step; the largest finite
    value (its square overflows fp32, not the f64 norm) and the smallest
    subnormal apply; placed in the vector rows and in the ragged tail; every
    scalar and w/m/v bit against the oracle."""
    torch = _torch()
    specs = [TensorSpec("a", (4096 * 3,), True, False), TensorSpec("b", (777,), True, False)]
    cfg, ps, ts, opt, ref = _make(specs, 4, [1e-3, 1e-3], 1.0, grad_dtype=_abi.GRAD_F32)
    for ti, pos in [(0, 5000), (1, 770)]:
        ps.g(ti).view(torch.int32)[pos] = int(np.array(bits, np.uint32).view(np.int32))
        ts[ti].g.view(np.uint32)[pos] = bits
    _, gi = opt.step_all(cfg.lr, info=True)
    _, ri = ref.step(cfg.lr)
    assert gi.applied == 1 - skips and gi.nonfinite == skips
    assert not H.info_matches(gi, ri)
    c = H.compare(ps, ts)
    assert c["w"] == c["m"] == c["v"] == 0, c
    opt.close()


def test_record_overflow_matches_oracle():
    specs = [TensorSpec("a", (512,), True, False)]
    sig = [1e-3]
    cfg, ps, ts, opt, ref = _make(specs, 1, sig, 1024.0, max_consecutive_nonfinite=2)
    for k in range(4):
        rc, gi = opt.record_overflow()
        rrc, ri = ref.record_overflow()
        assert rc == rrc and not H.info_matches(gi, ri)
    assert gi.state.early_stop == 1
    opt.close()


def test_single_tensor_dropin_matches_reference_kernel():
    """ark_hip_adam_step_f16 = one ark_asm_adam_step_f16 call (fp32 g, t=0
    treated as 1, any n, any element alignment)."""
    torch = _torch()
    from ark_amd._lib import check, lib
    rng = np.random.default_rng(0)
    for n, t, off in [(1, 0, 0), (8, 1, 0), (4096 * 3 + 5, 7, 0), (10000, 123456, 1),
                      (589824, 2, 0)]:
        w = oracle.synth_normal_f16(n + off, 3, 0, 0, 0.02)
        g = (rng.standard_normal(n + off) * 1e-3).astype(np.float32)
        m = (rng.standard_normal(n + off) * 1e-4).astype(np.float32)
        v = (rng.random(n + off) * 1e-6).astype(np.float32)
        dw = torch.from_numpy(w.view(np.int16)).cuda()
        dg, dm, dv = (torch.from_numpy(a).cuda() for a in (g, m, v))
        rc = lib().ark_hip_adam_step_f16(
            dw.data_ptr() + 2 * off, dg.data_ptr() + 4 * off, dm.data_ptr() + 4 * off,
            dv.data_ptr() + 4 * off, n, 3e-4, 0.9, 0.95, 1e-8, 0.1, t,
            C.c_void_p(torch.cuda.current_stream().cuda_stream))
        check(rc)
        torch.cuda.synchronize()
        ww, mm, vv = w[off:].copy(), m[off:].copy(), v[off:].copy()
        oracle.adam_step_f16(ww, g[off:].copy(), mm, vv, 3e-4, 0.9, 0.95, 1e-8, 0.1, t)
        assert not np.any(H.bits_differ16(dw.cpu().numpy().view(np.uint16)[off:], ww))
        assert not np.any(H.bits_differ32(dm.cpu().numpy()[off:], mm))
        assert not np.any(H.bits_differ32(dv.cpu().numpy()[off:], vv))


def _w32_step(torch, w, g, m, v, off, n, lr, b1, b2, eps, wd, t):
    from ark_amd._lib import check, lib
    check(lib().ark_hip_adam_step(
        w.data_ptr() + 4 * off, g.data_ptr() + 4 * off, m.data_ptr() + 4 * off,
        v.data_ptr() + 4 * off, n, lr, b1, b2, eps, wd, t,
        C.c_void_p(torch.cuda.current_stream().cuda_stream)))


@pytest.mark.parametrize("n,off", [(1, 0), (3, 1), (255, 0), (257, 2), (4096 * 3 + 5, 0),
                                   (10000, 3), (768 * 768, 0)])
def test_fp32_weight_dropin_matches_reference_kernel(n, off):
    """ark_hip_adam_step = successive ark_asm_adam_step calls (opti.s:20-177):
    ten steps from t = 0 (treated as 1) with a new gradient each, the c0
    tensor shape (768 x 768) among ragged sizes; offsets of 1-3 elements take
    the per-element path, aligned full rows the 16-byte one."""
    torch = _torch()
    rng = np.random.default_rng(n * 7 + off)
    w = (rng.standard_normal(n + off) * 0.02).astype(np.float32)
    m = np.zeros(n + off, np.float32)
    v = np.zeros(n + off, np.float32)
    dw, dm, dv = (torch.from_numpy(a.copy()).cuda() for a in (w, m, v))
    ww, mm, vv = w[off:].copy(), m[off:].copy(), v[off:].copy()
    for t in range(10):
        g = (rng.standard_normal(n + off) * 10.0 ** rng.uniform(-5, 0)).astype(np.float32)
        dg = torch.from_numpy(g).cuda()
        _w32_step(torch, dw, dg, dm, dv, off, n, 6e-4, 0.9, 0.95, 1e-8, 0.1, t)
        oracle.adam_step_f32(ww, g[off:].copy(), mm, vv, 6e-4, 0.9, 0.95, 1e-8, 0.1, t)
    torch.cuda.synchronize()
    for d, h in ((dw, ww), (dm, mm), (dv, vv)):
        got = d.cpu().numpy()
        assert not np.any(H.bits_differ32(got[off:], h)), n
    # the element before the span is untouched
    assert np.array_equal(dw.cpu().numpy()[:off], w[:off])


def test_python_wrappers_of_the_single_tensor_dropins():
    """ark_amd.optimizer.adam_step_zero_copy (optimizer.rs:27-40) and
    adam_step (ffi.rs:98-101) on torch's current stream, against the
    oracle; length and dtype mismatches raise before any device call."""
    torch = _torch()
    from ark_amd.optimizer import adam_step, adam_step_zero_copy
    rng = np.random.default_rng(11)
    n = 70001
    g = (rng.standard_normal(n) * 1e-3).astype(np.float32)
    m = (rng.standard_normal(n) * 1e-4).astype(np.float32)
    v = (rng.random(n) * 1e-6).astype(np.float32)
    w16 = oracle.synth_normal_f16(n, 5, 0, 0, 0.02)
    w32 = (rng.standard_normal(n) * 0.02).astype(np.float32)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        dw16 = torch.from_numpy(w16.view(np.int16)).cuda().view(torch.float16)
        dw32 = torch.from_numpy(w32).cuda()
        dg = torch.from_numpy(g).cuda()
        dm16, dv16, dm32, dv32 = (torch.from_numpy(a.copy()).cuda() for a in (m, v, m, v))
        adam_step_zero_copy(dw16, dg, dm16, dv16, 3e-4, 0.9, 0.95, 1e-8, 0.1, 4)
        adam_step(dw32, dg, dm32, dv32, 3e-4, 0.9, 0.95, 1e-8, 0.1, 4)
    s.synchronize()
    h = [a.copy() for a in (w16, m, v)]
    oracle.adam_step_f16(h[0], g.copy(), h[1], h[2], 3e-4, 0.9, 0.95, 1e-8, 0.1, 4)
    assert not np.any(H.bits_differ16(dw16.cpu().view(torch.int16).numpy().view(np.uint16), h[0]))
    assert not np.any(H.bits_differ32(dm16.cpu().numpy(), h[1]))
    assert not np.any(H.bits_differ32(dv16.cpu().numpy(), h[2]))
    h = [a.copy() for a in (w32, m, v)]
    oracle.adam_step_f32(h[0], g.copy(), h[1], h[2], 3e-4, 0.9, 0.95, 1e-8, 0.1, 4)
    for d, e in zip((dw32, dm32, dv32), h):
        assert not np.any(H.bits_differ32(d.cpu().numpy(), e))
    with pytest.raises(ValueError, match="lengths differ"):
        adam_step(dw32[1:], dg, dm32, dv32, 3e-4, 0.9, 0.95, 1e-8, 0.1, 4)
    with pytest.raises(ValueError, match="float32"):
        adam_step(dw16, dg, dm32, dv32, 3e-4, 0.9, 0.95, 1e-8, 0.1, 4)
    with pytest.raises(ValueError, match="float16"):
        adam_step_zero_copy(dw32, dg, dm32, dv32, 3e-4, 0.9, 0.95, 1e-8, 0.1, 4)


def test_fp32_weight_dropin_special_values():
    """Subnormal, huge, infinite and NaN gradients and weights, zero moments
    and eps = 0 (0/0 -> NaN), through both the 16-byte and the per-element
    paths: the same results as the reference kernel, NaN for NaN."""
    torch = _torch()
    vals = np.array([0.0, -0.0, 1e-45, -1e-40, 1e-20, 3e38, -3e38, np.inf, -np.inf, np.nan,
                     1.0, -1.0, 65504.0, 2.0 ** -126], np.float32)
    rng = np.random.default_rng(5)
    n = 1024 + 37
    for eps in (1e-8, 0.0):
        w = rng.choice(vals, n).astype(np.float32)
        g = rng.choice(vals, n).astype(np.float32)
        m = rng.choice(vals[:7], n).astype(np.float32)
        v = np.abs(rng.choice(vals[:7], n)).astype(np.float32)
        for off in (0, 1):
            dw, dg, dm, dv = (torch.from_numpy(a.copy()).cuda() for a in (w, g, m, v))
            k = n - off
            _w32_step(torch, dw, dg, dm, dv, off, k, 1e-3, 0.9, 0.999, eps, 0.01, 3)
            ww, mm, vv = w[off:].copy(), m[off:].copy(), v[off:].copy()
            oracle.adam_step_f32(ww, g[off:].copy(), mm, vv, 1e-3, 0.9, 0.999, eps, 0.01, 3)
            torch.cuda.synchronize()
            for d, h in ((dw, ww), (dm, mm), (dv, vv)):
                assert not np.any(H.bits_differ32(d.cpu().numpy()[off:], h)), (eps, off)


@pytest.mark.parametrize("true_grads,clipped", [
    ([0.5, -0.5, 0.5, 0.5], 0),          # norm exactly 1.0 = grad_clip: `>` is strict
    ([1.0 + 2.0 ** -10], 1),             # just above: coef = 1 / norm
    ([1.0 - 2.0 ** -11], 0),             # just below
    ([0.0] * 9, 0),                      # norm 0
])
def test_clip_boundary_matches_oracle(true_grads, clipped):
    """optimizer.rs:148-149 at the threshold (grad_clip 1.0, loss scale 1024),
    one tensor of these gradients among 4096 zeros; every scalar and every
    w/m/v bit against the oracle."""
    torch = _torch()
    from ark_amd.optimizer import AdamConfig, AmpConfig, Optimizer, ParamSet
    scale = 1024.0
    g = np.zeros(4096 + len(true_grads))
    g[-len(true_grads):] = np.asarray(true_grads) * scale
    g16 = g.astype(np.float16)
    assert np.array_equal(g16.astype(np.float64), g)
    n = g.size
    rng = np.random.default_rng(n)
    w = (rng.standard_normal(n) * 0.02).astype(np.float16).view(np.uint16)
    specs = [TensorSpec("a", (n,), True, False)]
    cfg = AdamConfig(**HP)
    ps = ParamSet(specs, cfg.weight_decay)
    ps.w(0).copy_(torch.from_numpy(w.view(np.int16)).view(torch.float16))
    ps.g(0).copy_(torch.from_numpy(g16))
    ts = [oracle.HostTensor(w.copy(), g16.view(np.uint16).copy(), np.zeros(n, np.float32),
                            np.zeros(n, np.float32), cfg.weight_decay)]
    opt = Optimizer(cfg, ps, AmpConfig(loss_scale_init=scale))
    ref = oracle.Optimizer(ts, opt.hp)
    _, gi = opt.step_all(cfg.lr, info=True)
    _, ri = ref.step(cfg.lr)
    assert not H.info_matches(gi, ri)
    assert gi.clipped == clipped and (clipped or gi.clip_coef == 1.0)
    c = H.compare(ps, ts)
    assert c["w"] == c["m"] == c["v"] == 0, c
    opt.close()


def test_element_math_over_an_edge_value_grid():
    """Every combination of edge values of w, g, m and v (signed zeros,
    subnormals, fp16 max, huge and tiny moments, infinite and NaN state,
    a negative v whose square root is NaN) in one tensor, one step without
    unscale or clip: each element against the oracle's opti.s:278-308
    sequence (NaNs compared as NaNs)."""
    torch = _torch()
    from ark_amd.optimizer import AdamConfig, AmpConfig, Optimizer, ParamSet
    f16 = lambda xs: np.array(xs, np.float16).view(np.uint16)
    ws = np.concatenate([f16([0.0, -0.0, 6e-8, 1e-3, 1.0, -1.0, 65504.0, -65504.0]),
                         np.array([0x7C00, 0x7E00], np.uint16)])
    gs = f16([0.0, -0.0, 6e-8, -6e-8, 1e-3, -1.0, 1.0, 100.0, -1000.0, 60000.0])
    ms = np.array([0.0, -0.0, 1e-30, -1e-3, 1.0, 1e30, np.inf, -np.inf, np.nan], np.float32)
    vs = np.array([0.0, 1e-45, 1e-30, 1e-8, 1.0, 1e30, 3e38, np.inf, np.nan, -1.0], np.float32)
    W, G, M, V = (a.ravel() for a in np.meshgrid(ws, gs, ms, vs, indexing="ij"))
    n = W.size
    cfg = AdamConfig(lr=1e-2, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1, grad_clip=1e30)
    ps = ParamSet([TensorSpec("grid", (n,), True, False)], cfg.weight_decay)
    ps.w(0).copy_(torch.from_numpy(W.view(np.int16)).view(torch.float16))
    ps.g(0).copy_(torch.from_numpy(G.view(np.int16)).view(torch.float16))
    ps.m(0).copy_(torch.from_numpy(M.copy()))
    ps.v(0).copy_(torch.from_numpy(V.copy()))
    ts = [oracle.HostTensor(W.copy(), G.copy(), M.copy(), V.copy(), cfg.weight_decay)]
    opt = Optimizer(cfg, ps, AmpConfig(loss_scale_init=1.0))
    ref = oracle.Optimizer(ts, opt.hp)
    _, gi = opt.step_all(cfg.lr, info=True)
    _, ri = ref.step(cfg.lr)
    assert gi.applied == 1 and not H.info_matches(gi, ri)
    c = H.compare(ps, ts)
    assert c["w"] == c["m"] == c["v"] == 0, c
    opt.close()


def test_edge_values_weights_near_overflow_and_subnormal_grads():
    """Weights near 65504 (overflow to inf on requantisation), fp16
    subnormal weights and gradients, zero gradients."""
    torch = _torch()
    from ark_amd.optimizer import AdamConfig, AmpConfig, Optimizer, ParamSet
    n = 4096 + 100
    specs = [TensorSpec("a", (n,), True, False)]
    rng = np.random.default_rng(5)
    w = rng.integers(0, 65536, n).astype(np.uint16)
    w[:64] = np.array([0x7BFF, 0xFBFF, 0x7BFE, 0x0001, 0x8001, 0x03FF, 0x0000, 0x8000] * 8, np.uint16)
    w[(w & 0x7C00) == 0x7C00] = 0x3C00  # keep weights finite
    g = rng.integers(0, 0x0400, n).astype(np.uint16) | (rng.integers(0, 2, n).astype(np.uint16) << 15)
    g[::7] = 0
    g[100:200] = 0x7BFF  # largest finite gradient
    # a negative decoupled decay (decay = 1 - lr*wd > 1) pushes weights near
    # 65504 over the fp16 range
    cfg = AdamConfig(lr=1e-2, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=-0.1, grad_clip=1e30)
    amp = AmpConfig(loss_scale_init=1.0)
    ps = ParamSet(specs, cfg.weight_decay)
    ps.w(0).copy_(torch.from_numpy(w.view(np.int16)).view(torch.float16))
    ps.g(0).copy_(torch.from_numpy(g.view(np.int16)).view(torch.float16))
    ts = [oracle.HostTensor(w.copy(), g.copy(), np.zeros(n, np.float32), np.zeros(n, np.float32),
                            -0.1)]
    opt = Optimizer(cfg, ps, amp)
    ref = oracle.Optimizer(ts, opt.hp)
    for k in range(3):
        _, gi = opt.step_all(cfg.lr, info=True)
        _, ri = ref.step(cfg.lr)
        assert not H.info_matches(gi, ri)
        c = H.compare(ps, ts)
        assert c["w"] == c["m"] == c["v"] == 0, c
    assert np.any((ts[0].w & 0x7FFF) == 0x7C00)  # some weight overflowed
    opt.close()
