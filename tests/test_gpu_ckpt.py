"""GPU parity of the checkpoint path (include/ark_ckpt.h) against the
checkpoint oracle (oracle/ckpt.py, the format of io.rs:432-671): files
written from device buffers equal the oracle's bytes, files the oracle
writes (V4, V3, V2) load into device buffers as the reference's chain of
conversions would, and the full EKO-237M image packs and unpacks bit for
bit."""
import numpy as np
import pytest

import oracle
from oracle import ckpt as K
from ark_amd import _abi, ckpt
from ark_amd._lib import ArkOptError
from ark_amd.eko import EKO_237M, EkoConfig

pytestmark = pytest.mark.gpu

ODD = EkoConfig(n_layers=2, d_model=33, hidden=47, vocab=101)  # odd sizes: unaligned records


def _torch():
    import torch
    assert torch.cuda.is_available(), "GPU test run without a GPU"
    return torch


def _bits(t):
    torch = _torch()
    it = {2: torch.int16, 4: torch.int32}[t.element_size()]
    u = {2: np.uint16, 4: np.uint32}[t.element_size()]
    return t.view(it).cpu().numpy().view(u)


def _fill_random(tensors, seed):
    """Every bit pattern equally likely: NaNs, infinities, subnormals."""
    torch = _torch()
    g = torch.Generator(device="cuda").manual_seed(seed)
    for t in tensors:
        if t.element_size() == 2:
            t.view(torch.int16).copy_(torch.randint(-32768, 32768, t.shape, device="cuda",
                                                    generator=g, dtype=torch.int32))
        else:
            t.view(torch.int32).copy_(torch.randint(-2 ** 31, 2 ** 31, t.shape, device="cuda",
                                                    generator=g, dtype=torch.int64))


def _quiet16(h):
    h = h.copy()
    snan = ((h & 0x7C00) == 0x7C00) & ((h & 0x03FF) != 0)
    h[snan] |= 0x0200
    return h


def _params(cfg, seed):
    from ark_amd.optimizer import ParamSet
    ps = ParamSet(cfg.tensors(), weight_decay=0.1)
    _fill_random(ckpt.param_tensors(ps), seed)
    return ps


def _oracle_bytes(ps, global_step, adam_step):
    t = [_bits(x) for x in ckpt.param_tensors(ps)]
    nl = (len(t) - 6) // 27
    lw = [t[3 + 27 * l: 12 + 27 * l] for l in range(nl)]
    lm = [t[12 + 27 * l: 21 + 27 * l] for l in range(nl)]
    lv = [t[21 + 27 * l: 30 + 27 * l] for l in range(nl)]
    return K.save_fp16(global_step, adam_step, t[0], t[1].view(np.float32), t[2].view(np.float32),
                       t[-3], t[-2].view(np.float32), t[-1].view(np.float32), lw,
                       [[a.view(np.float32) for a in l] for l in lm],
                       [[a.view(np.float32) for a in l] for l in lv])


def test_save_equals_oracle_bytes(tmp_path):
    torch = _torch()
    ps = _params(ODD, 1)
    st = _abi.State(t=37, loss_scale=4096.0, clean_steps=12, consecutive_nonfinite=0,
                    skipped_steps=5, early_stop=0, reserved=0)
    p = str(tmp_path / "a.bin")
    ckpt.save(p, ckpt.param_tensors(ps), 1234, 37, st)
    got = open(p, "rb").read()
    want = _oracle_bytes(ps, 1234, 37) + K.amp_trailer(bytes(st))
    assert len(got) == len(want)
    assert got == want
    # without the trailer: exactly the reference's file
    ckpt.save(p, ckpt.param_tensors(ps), 1234, 37)
    assert open(p, "rb").read() == want[:-40]
    torch.cuda.synchronize()


def test_round_trip_through_file(tmp_path):
    from ark_amd.optimizer import AdamConfig, AmpConfig, Optimizer, ParamSet
    ps = _params(ODD, 2)
    opt = Optimizer(AdamConfig(), ps, AmpConfig(loss_scale_init=1024.0))
    opt.set_state(t=99, loss_scale=2048.0, clean_steps=17, skipped_steps=3)
    p = str(tmp_path / "b.bin")
    ckpt.save_params(p, ps, opt, global_step=500)
    info, pairs = ckpt.probe(p)
    assert (info.version, info.global_step, info.adam_step, info.has_amp) == (4, 500, 99, True)
    assert info.n_tensors == 3 + 27 * 2 + 3 == len(pairs)
    qs = ParamSet(ODD.tensors(), weight_decay=0.1)
    opt2 = Optimizer(AdamConfig(), qs, AmpConfig(loss_scale_init=1024.0))
    ckpt.load_params(p, qs, opt2)
    for a, b in zip(ckpt.param_tensors(ps), ckpt.param_tensors(qs)):
        want = _bits(a)
        if a.element_size() == 2:
            want = _quiet16(want)  # half::to_f32 then fcvtn quiets signalling NaNs
        np.testing.assert_array_equal(_bits(b), want)
    s1, s2 = opt.get_state(), opt2.get_state()
    for k in ("t", "loss_scale", "clean_steps", "consecutive_nonfinite", "skipped_steps"):
        assert getattr(s1, k) == getattr(s2, k), k
    opt.close(), opt2.close()


def test_load_oracle_v4_into_f32(tmp_path):
    """CheckpointV3::load's pesos are fp32: F16 records widen exactly."""
    torch = _torch()
    rng = np.random.default_rng(4)
    tens = [rng.integers(0, 65536, n, dtype=np.uint32).astype(np.uint16) for n in (1, 5, 4096, 4099)]
    tens += [rng.integers(0, 2 ** 32, n, dtype=np.uint64).astype(np.uint32).view(np.float32)
             for n in (3, 8191)]
    p = str(tmp_path / "c.bin")
    open(p, "wb").write(K.write_v4(7, 8, tens))
    outs = [torch.empty(t.size, dtype=torch.float32, device="cuda") for t in tens]
    info, amp = ckpt.load(p, outs)
    assert amp is None and info.adam_step == 8
    for t, o in zip(tens, outs):
        want = oracle.f16_to_f32(t).view(np.uint32) if t.dtype == np.uint16 else t.view(np.uint32)
        np.testing.assert_array_equal(_bits(o), want)


@pytest.mark.parametrize("version", [3, 2])
def test_load_oracle_v3_v2_into_fp16_weights(tmp_path, version):
    """V3 / V2 weights are fp32: into fp16 buffers they round to nearest
    even (sync_weights_to_gpu's ark_quant_f32_to_f16, memory.rs:347-377)."""
    torch = _torch()
    rng = np.random.default_rng(version)
    ns = [7, 4096, 12345, 33]
    tens = [rng.integers(0, 2 ** 32, n, dtype=np.uint64).astype(np.uint32).view(np.float32)
            for n in ns]
    data = K.write_v3(5, 6, tens) if version == 3 else K.write_v2(5, tens)
    p = str(tmp_path / "d.bin")
    open(p, "wb").write(data)
    info, pairs = ckpt.probe(p)
    assert info.version == version and [n for n, _ in pairs] == ns
    assert all(t == _abi.CKPT_F32 for _, t in pairs)
    outs = [torch.empty(n, dtype=torch.float16 if i % 2 == 0 else torch.float32, device="cuda")
            for i, n in enumerate(ns)]
    info, _ = ckpt.load(p, outs)
    assert info.has_moments == (version == 3) and info.adam_step == (6 if version == 3 else 0)
    for t, o in zip(tens, outs):
        want = oracle.f32_to_f16(t) if o.element_size() == 2 else t.view(np.uint32)
        np.testing.assert_array_equal(_bits(o), want)


def test_full_eko237m_image():
    """Pack the 816-record EKO-237M checkpoint (2.37 GB) on the device: the
    image equals the oracle's file bytes; unpacking it restores every
    buffer."""
    torch = _torch()
    from ark_amd.optimizer import ParamSet
    ps = _params(EKO_237M, 3)
    tens = ckpt.param_tensors(ps)
    nb = ckpt.image_bytes(tens)
    img = torch.empty(nb, dtype=torch.uint8, device="cuda")
    ckpt.pack(tens, img, 4000, 3999)
    got = img.cpu().numpy()
    want = np.frombuffer(_oracle_bytes(ps, 4000, 3999), np.uint8)
    assert got.size == want.size
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, f"{bad.size} bytes differ, first at {bad[0]}"
    del got, want
    qs = ParamSet(EKO_237M.tensors(), weight_decay=0.1)
    ckpt.unpack(img, ckpt.param_tensors(qs))
    for a, b in zip(tens, ckpt.param_tensors(qs)):
        if a.element_size() == 4:
            assert torch.equal(a.view(torch.int32), b.view(torch.int32))
        else:
            np.testing.assert_array_equal(_bits(b), _quiet16(_bits(a)))


@pytest.mark.parametrize("per_launch", ["1", "7", "1000"])
def test_pack_and_unpack_split_over_launches(per_launch, monkeypatch):
    """Pack and unpack launch at most 2^32 work-items at a time, so an image
    past 64 GiB (pack) or 128 GiB (unpack) takes several launches, each from
    a block offset.  ARK_CKPT_LAUNCH_BLOCKS caps the blocks per launch so that
    a small image takes that path too: the image is byte-identical to the
    one-launch image, and unpacking it restores every buffer."""
    torch = _torch()
    from ark_amd.optimizer import ParamSet
    ps = _params(ODD, 4)
    tens = ckpt.param_tensors(ps)
    nb = ckpt.image_bytes(tens)
    one = torch.empty(nb, dtype=torch.uint8, device="cuda")
    ckpt.pack(tens, one, 77, 66)
    monkeypatch.setenv("ARK_CKPT_LAUNCH_BLOCKS", per_launch)
    split = torch.zeros(nb, dtype=torch.uint8, device="cuda")
    ckpt.pack(tens, split, 77, 66)
    assert torch.equal(one, split)
    qs = ParamSet(ODD.tensors(), weight_decay=0.1)
    ckpt.unpack(split, ckpt.param_tensors(qs))
    for a, b in zip(tens, ckpt.param_tensors(qs)):
        if a.element_size() == 4:
            assert torch.equal(a.view(torch.int32), b.view(torch.int32))
        else:
            np.testing.assert_array_equal(_bits(b), _quiet16(_bits(a)))


def test_resume_is_bit_continuous(tmp_path):
    """Train, save (V4 with the AMP trailer), load into fresh buffers and a
    fresh optimizer, continue: the weights, moments and scaler state equal an
    uninterrupted run's bit for bit.  A non-finite step before the save and a
    growth period of 3 make the skipped/clean counters and the scale part of
    what must carry over (the reference restarts its scaler at init on every
    resume, training.rs:120-124)."""
    torch = _torch()
    from ark_amd import synth
    from ark_amd.optimizer import AdamConfig, AmpConfig, Optimizer
    specs = EkoConfig(n_layers=2, d_model=64, hidden=96, vocab=500).tensors()
    seed, scale = 5, 1024.0
    sig = synth.log_uniform_sigmas(len(specs), seed)
    cfg = AdamConfig(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1, grad_clip=1.0)
    amp = AmpConfig(loss_scale_init=scale, loss_scale_max=2.0 ** 24, scale_up_every=3)
    N, M, bad = 6, 5, 2

    def run(ps, opt, steps):
        for k in steps:
            synth.regen_grads(ps, seed, sig, scale, k)
            if k == bad:
                ps.g(0).view(torch.int16)[3] = 0x7C00
            opt.step_all(cfg.lr)

    pa = synth.problem(specs, seed, cfg.weight_decay, sig, scale)
    oa = Optimizer(cfg, pa, amp)
    run(pa, oa, range(N + M))

    pb = synth.problem(specs, seed, cfg.weight_decay, sig, scale)
    ob = Optimizer(cfg, pb, amp)
    run(pb, ob, range(N))
    path = str(tmp_path / "resume.ark")
    ckpt.save_params(path, pb, ob, global_step=N)
    ob.close()

    pc = synth.problem(specs, seed + 1, cfg.weight_decay, sig, scale)  # other contents
    oc = Optimizer(cfg, pc, amp)
    info, st = ckpt.load_params(path, pc, oc)
    assert info.has_amp and st.skipped_steps == 1 and info.adam_step == N - 1
    run(pc, oc, range(N, N + M))
    torch.cuda.synchronize()
    sa, sc = oa.get_state(), oc.get_state()
    for f in ("t", "loss_scale", "clean_steps", "consecutive_nonfinite", "skipped_steps"):
        assert getattr(sa, f) == getattr(sc, f), f
    assert sa.loss_scale != scale  # the scale moved: the trailer carried it
    for i in range(len(specs)):
        for a, c in ((pa.w(i), pc.w(i)), (pa.m(i), pc.m(i)), (pa.v(i), pc.v(i))):
            it = torch.int16 if a.element_size() == 2 else torch.int32
            assert torch.equal(a.view(it), c.view(it)), specs[i].name
    oa.close(), oc.close()


def test_pack_unpack_empty_and_tiny_records():
    """Empty records (they start where the next one does), runs of one- and
    few-element records, and records of hundreds of blocks, so that one
    256-block range of the kernels' record search spans many records and
    others lie inside one record: image bytes against the oracle writer, then
    unpacked back."""
    torch = _torch()
    sizes = [0, 1, 3000, 0, 0, 7, 600001, 0, 1, 1, 2, 150000, 0, 5, 0] + [3] * 300 + [0, 777777, 1]
    tens = []
    for i, n in enumerate(sizes):
        dt = torch.float16 if i % 3 == 0 else torch.float32
        tens.append(torch.empty(n, dtype=dt, device="cuda"))
    _fill_random(tens, 12)
    nb = ckpt.image_bytes(tens)
    img = torch.empty(nb, dtype=torch.uint8, device="cuda")
    ckpt.pack(tens, img, 77, 66)
    torch.cuda.synchronize()
    want = K.write_v4(77, 66, [_bits(t) if t.numel() else
                               np.zeros(0, np.uint16 if t.element_size() == 2 else np.float32)
                               for t in tens])
    got = img.cpu().numpy()
    assert got.tobytes() == want
    back = [torch.empty_like(t) for t in tens]
    ckpt.unpack(img, back)
    torch.cuda.synchronize()
    for a, b in zip(tens, back):
        x, y = _bits(a), _bits(b)
        if a.element_size() == 2:
            x = _quiet16(x)  # fp16 -> fp16 passes through f32: a signalling NaN comes back quiet
        np.testing.assert_array_equal(x, y)


def test_thousands_of_tiny_records():
    """3000 records of 0-40 elements (fp16 and fp32, so every later record is
    misaligned one way or another) followed by a large one: hundreds of
    records inside one 256-block range of the kernels' tensor lookup; image
    bytes against the oracle writer, and unpacked back."""
    torch = _torch()
    rng = np.random.default_rng(23)
    sizes = [int(x) for x in rng.integers(0, 41, 3000)] + [300000]
    tens = [torch.empty(n, dtype=torch.float16 if rng.random() < 0.5 else torch.float32,
                        device="cuda") for n in sizes]
    _fill_random(tens, 24)
    img = torch.empty(ckpt.image_bytes(tens), dtype=torch.uint8, device="cuda")
    ckpt.pack(tens, img, 5, 4)
    torch.cuda.synchronize()
    want = K.write_v4(5, 4, [_bits(t) if t.numel() else
                             np.zeros(0, np.uint16 if t.element_size() == 2 else np.float32)
                             for t in tens])
    assert img.cpu().numpy().tobytes() == want
    back = [torch.empty_like(t) for t in tens]
    ckpt.unpack(img, back)
    torch.cuda.synchronize()
    for a, b in zip(tens, back):
        x, y = _bits(a), _bits(b)
        if a.element_size() == 2:
            x = _quiet16(x)
        np.testing.assert_array_equal(x, y)


@pytest.mark.parametrize("case", range(12))
def test_random_tables_at_random_buffer_alignments(case):
    """Seeded random record tables whose buffers start at random element
    offsets inside larger allocations, so every source and destination
    alignment modulo 16 bytes (fp16: 0-14 in steps of 2; fp32: 0-12 in steps
    of 4) meets every image offset: 1-60 records of mixed fp16/fp32 with
    sizes from empty through a few elements, around 4096 and up to ~70k.
    Image bytes against the oracle writer, then unpacked into buffers at
    other random offsets and compared bit for bit (an fp16 signalling NaN
    comes back quiet)."""
    torch = _torch()
    rng = np.random.default_rng(9000 + case)
    nrec = int(rng.integers(1, 61))
    sizes = []
    for _ in range(nrec):
        r = rng.random()
        sizes.append(0 if r < 0.1 else int(rng.integers(1, 9)) if r < 0.35 else
                     int(rng.integers(4090, 4103)) if r < 0.55 else int(rng.integers(9, 70000)))
    f16 = [bool(rng.random() < 0.5) for _ in range(nrec)]

    def views(offsets):
        out = []
        for n, h, off in zip(sizes, f16, offsets):
            base = torch.empty(n + 8, dtype=torch.float16 if h else torch.float32, device="cuda")
            out.append(base[off:off + n])
        return out

    src = views([int(x) for x in rng.integers(0, 8, nrec)])
    _fill_random(src, 100 + case)
    nb = ckpt.image_bytes(src)
    img = torch.empty(nb + 64, dtype=torch.uint8, device="cuda")[16 * int(rng.integers(0, 4)):][:nb]
    ckpt.pack(src, img, case, 2 * case)
    torch.cuda.synchronize()
    want = K.write_v4(case, 2 * case,
                      [_bits(t) if t.numel() else
                       np.zeros(0, np.uint16 if t.element_size() == 2 else np.float32)
                       for t in src])
    assert img.cpu().numpy().tobytes() == want, (case, nrec)
    dst = views([int(x) for x in rng.integers(0, 8, nrec)])
    ckpt.unpack(img, dst)
    torch.cuda.synchronize()
    for i, (a, b) in enumerate(zip(src, dst)):
        x, y = _bits(a), _bits(b)
        if a.element_size() == 2:
            x = _quiet16(x)
        np.testing.assert_array_equal(x, y, err_msg=f"case {case} record {i}")


def _state(t, scale, skipped):
    return _abi.State(t=t, loss_scale=scale, clean_steps=t % 7, consecutive_nonfinite=t % 3,
                      skipped_steps=skipped, early_stop=0)


@pytest.mark.parametrize("case", range(6))
def test_pack_plan_runs_write_the_oracle_bytes(case):
    """A pack plan over a seeded random table (buffers at random element
    offsets, as above) run several times with new steps, new AMP states and
    new buffer contents in between: after each run the image equals the
    oracle writer's bytes for that save (with the 40-byte trailer when the
    plan carries one), and ark_ckpt_v4_pack's image of the same save."""
    torch = _torch()
    rng = np.random.default_rng(7000 + case)
    nrec = int(rng.integers(1, 40))
    with_amp = case % 2 == 1
    src = []
    for _ in range(nrec):
        r = rng.random()
        n = 0 if r < 0.1 else int(rng.integers(1, 9)) if r < 0.35 else int(rng.integers(9, 30000))
        dt = torch.float16 if rng.random() < 0.5 else torch.float32
        off = int(rng.integers(0, 8))
        src.append(torch.empty(n + 8, dtype=dt, device="cuda")[off:off + n])
    nb = ckpt.image_bytes(src, with_amp)
    img = torch.empty(nb + 64, dtype=torch.uint8, device="cuda")[16 * int(rng.integers(0, 4)):][:nb]
    ref = torch.empty(nb, dtype=torch.uint8, device="cuda")
    plan = ckpt.PackPlan(src, img, with_amp=with_amp)
    try:
        for k in range(3):
            _fill_random(src, 300 + 10 * case + k)
            amp = _state(5 * k + case, 2.0 ** (k + 3), 11 * k) if with_amp else None
            gs, ad = 1000 * case + k, 999 * case + 2 * k
            img.fill_(0xAB)
            plan.run(gs, ad, amp)
            torch.cuda.synchronize()
            want = K.write_v4(gs, ad, [_bits(t) if t.numel() else
                                       np.zeros(0, np.uint16 if t.element_size() == 2
                                                else np.float32) for t in src])
            if with_amp:
                want += K.amp_trailer(bytes(amp))
            assert img.cpu().numpy().tobytes() == want, (case, k)
            ckpt.pack(src, ref, gs, ad, amp)
            assert torch.equal(img, ref), (case, k)
    finally:
        plan.close()


def test_pack_plan_full_eko237m_and_split_launches(monkeypatch):
    """The plan over the 816-record EKO-237M table writes the image the
    one-call pack writes (2.37 GB, the oracle's bytes in test_full_eko237m_image),
    with its data split over many launches too (ARK_CKPT_LAUNCH_BLOCKS is read
    at each run)."""
    torch = _torch()
    ps = _params(EKO_237M, 5)
    tens = ckpt.param_tensors(ps)
    nb = ckpt.image_bytes(tens, True)
    ref = torch.empty(nb, dtype=torch.uint8, device="cuda")
    img = torch.empty(nb, dtype=torch.uint8, device="cuda")
    amp = _state(4000, 65536.0, 3)
    ckpt.pack(tens, ref, 4001, 4000, amp)
    plan = ckpt.PackPlan(tens, img, with_amp=True)
    try:
        img.zero_()
        plan.run(4001, 4000, amp)
        torch.cuda.synchronize()
        assert torch.equal(img, ref)
        monkeypatch.setenv("ARK_CKPT_LAUNCH_BLOCKS", "4099")
        img.zero_()
        plan.run(4001, 4000, amp)
        torch.cuda.synchronize()
        assert torch.equal(img, ref)
    finally:
        plan.close()


def test_pack_plan_in_a_hip_graph():
    """A plan run captured in a HIP graph (header and data kernels, no
    memset node) and replayed several times, with the buffers changed and
    the image cleared eagerly between replays: every replay writes the bytes
    of an eager pack of the buffers at that moment (the steps and state are
    the captured ones)."""
    torch = _torch()
    ps = _params(ODD, 6)
    tens = ckpt.param_tensors(ps)
    nb = ckpt.image_bytes(tens, True)
    img = torch.empty(nb, dtype=torch.uint8, device="cuda")
    ref = torch.empty(nb, dtype=torch.uint8, device="cuda")
    amp = _state(12, 1024.0, 1)
    stream = torch.cuda.Stream()
    plan = ckpt.PackPlan(tens, img, with_amp=True, stream=stream)
    try:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            plan.run(13, 12, amp)
        for k in range(4):
            _fill_random(tens, 60 + k)
            img.fill_(k)
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            ckpt.pack(tens, ref, 13, 12, amp)
            assert torch.equal(img, ref), k
        del graph
    finally:
        plan.close()


@pytest.mark.parametrize("with_amp", [False, True])
def test_pack_plan_of_an_empty_table(with_amp):
    """No records: a run writes the file header (and the trailer) only."""
    torch = _torch()
    nb = ckpt.image_bytes([], with_amp)
    assert nb == 28 + (40 if with_amp else 0)
    img = torch.full((nb,), 0xAB, dtype=torch.uint8, device="cuda")
    plan = ckpt.PackPlan([], img, with_amp=with_amp)
    try:
        amp = _state(3, 8.0, 2) if with_amp else None
        plan.run(21, 20, amp)
        torch.cuda.synchronize()
        want = K.write_v4(21, 20, []) + (K.amp_trailer(bytes(amp)) if with_amp else b"")
        assert img.cpu().numpy().tobytes() == want
    finally:
        plan.close()


def test_pack_plan_refuses_a_state_that_does_not_match():
    torch = _torch()
    ps = _params(ODD, 7)
    tens = ckpt.param_tensors(ps)
    img = torch.empty(ckpt.image_bytes(tens, True), dtype=torch.uint8, device="cuda")
    with_t = ckpt.PackPlan(tens, img, with_amp=True)
    without = ckpt.PackPlan(tens, img[:ckpt.image_bytes(tens)], with_amp=False)
    try:
        with pytest.raises(ArkOptError, match="amp is NULL"):
            with_t.run(1, 1)
        with pytest.raises(ArkOptError, match="amp must be NULL"):
            without.run(1, 1, _state(1, 1.0, 0))
    finally:
        with_t.close()
        without.close()
    with pytest.raises(ArkOptError, match="the checkpoint needs"):
        ckpt.PackPlan(tens, img[:ckpt.image_bytes(tens)], with_amp=True)


def test_rejects_bad_files(tmp_path):
    torch = _torch()
    x = [torch.zeros(5, dtype=torch.float16, device="cuda"),
         torch.zeros(3, dtype=torch.float32, device="cuda")]
    p = str(tmp_path / "e.bin")
    open(p, "wb").write(b"\x12\x34\x56\x78" + b"\0" * 60)
    with pytest.raises(ArkOptError, match="bad magic"):
        ckpt.load(p, x)
    good = K.write_v4(1, 1, [np.zeros(5, np.uint16), np.zeros(3, np.float32)])
    open(p, "wb").write(good[:-1])
    with pytest.raises(ArkOptError, match="truncated"):
        ckpt.load(p, x)
    open(p, "wb").write(good)
    with pytest.raises(ArkOptError, match="2 tensors, 1 records"):
        ckpt.load(p, x[:1])
    with pytest.raises(ArkOptError, match="n=5"):
        ckpt.load(p, [x[0][:4], x[1]])
    ckpt.load(p, x)  # and the good file loads
    with pytest.raises(ArkOptError):
        ckpt.load(str(tmp_path / "missing.bin"), x)


def test_unpack_checks_headers():
    torch = _torch()
    x = [torch.arange(9, dtype=torch.float16, device="cuda"),
         torch.arange(4, dtype=torch.float32, device="cuda")]
    img = torch.empty(ckpt.image_bytes(x), dtype=torch.uint8, device="cuda")
    ckpt.pack(x, img, 1, 2)
    y = [torch.empty_like(t) for t in x]
    ckpt.unpack(img, y)
    assert all(torch.equal(a, b) for a, b in zip(x, y))
    img[28 + 16 + 18] ^= 1  # second record's n
    with pytest.raises(ArkOptError, match="tensor 1 header"):
        ckpt.unpack(img, y)
    img[28 + 16 + 18] ^= 1
    img[0] ^= 1
    with pytest.raises(ArkOptError, match="file header"):
        ckpt.unpack(img, y)


def test_entry_points_reject_host_or_short_buffers(tmp_path):
    """Save, pack and unpack check every record and the image on the host
    before any launch or file: a record in host memory, a record past its
    allocation and an image shorter than the layout are refused with EINVAL
    and a message, and no file is created."""
    import ctypes as C
    import os
    import torch
    from ark_amd._lib import lib
    L = lib()
    msg = lambda: L.ark_opt_last_error().decode()
    w = torch.zeros(1000, dtype=torch.float16, device="cuda")
    m = torch.zeros(1000, device="cuda")
    host = np.zeros(1000, np.float32)
    recs = (_abi.CkptRecord * 2)()
    recs[0] = _abi.CkptRecord(w.data_ptr(), 1000, _abi.CKPT_F16, 0)
    recs[1] = _abi.CkptRecord(host.ctypes.data, 1000, _abi.CKPT_F32, 0)
    path = str(tmp_path / "x.ark")
    assert L.ark_ckpt_save_v4(os.fsencode(path), 1, 1, recs, 2, None, None) == _abi.EINVAL
    assert "buffer 1" in msg() and not os.path.exists(path), msg()
    image = torch.zeros(1 << 14, dtype=torch.uint8, device="cuda")
    recs[1] = _abi.CkptRecord(m.data_ptr(), 1 << 28, _abi.CKPT_F32, 0)  # 1 GiB from m
    assert L.ark_ckpt_save_v4(os.fsencode(path), 1, 1, recs, 2, None, None) == _abi.EINVAL
    assert "exceeds its allocation" in msg() and not os.path.exists(path), msg()
    # pack and unpack refuse it too: as past its allocation, or, where the
    # image lies inside that gigabyte, as overlapping the image
    refused = lambda: "exceeds its allocation" in msg() or "overlaps the image" in msg()
    rc = L.ark_ckpt_v4_pack(recs, 2, 1, 1, None, image.data_ptr(), image.numel(), None)
    assert rc == _abi.EINVAL and refused(), msg()
    types = (C.c_uint32 * 2)(_abi.CKPT_F16, _abi.CKPT_F32)
    rc = L.ark_ckpt_v4_unpack(image.data_ptr(), image.numel(), recs, 2, types, None)
    assert rc == _abi.EINVAL and refused(), msg()
    recs[1] = _abi.CkptRecord(m.data_ptr(), 1000, _abi.CKPT_F32, 0)
    need = C.c_uint64()
    assert L.ark_ckpt_v4_image_bytes(recs, 2, 0, C.byref(need)) == 0
    rc = L.ark_ckpt_v4_pack(recs, 2, 1, 1, None, image.data_ptr(), need.value - 1, None)
    assert rc == _abi.EINVAL and "image holds" in msg(), msg()
    # unpack reads the image size the caller states: 1 GiB is past the allocation
    rc = L.ark_ckpt_v4_unpack(image.data_ptr(), 1 << 30, recs, 2, types, None)
    assert rc == _abi.EINVAL and "image" in msg() and "exceeds its allocation" in msg(), msg()
    torch.cuda.synchronize()
    assert torch.count_nonzero(image).item() == 0


def test_save_replaces_the_file_whole(tmp_path):
    """A save goes through a temporary file and a rename: afterwards only the
    finished file is there (and a user's own ckpt.ark.tmp, untouched), and it
    replaces an earlier one completely."""
    import os
    import torch
    path = tmp_path / "ckpt.ark"
    path.write_bytes(b"an earlier, longer file " * 1000)
    (tmp_path / "ckpt.ark.tmp").write_bytes(b"the user's own file")
    w = torch.arange(777, dtype=torch.float32, device="cuda").half()
    m = torch.full((777,), 0.5, device="cuda")
    ckpt.save(str(path), [w, m], 12, 34)
    torch.cuda.synchronize()
    assert sorted(os.listdir(tmp_path)) == ["ckpt.ark", "ckpt.ark.tmp"]
    assert (tmp_path / "ckpt.ark.tmp").read_bytes() == b"the user's own file"
    want = K.write_v4(12, 34, [w.cpu().numpy().view(np.uint16), m.cpu().numpy()])
    assert path.read_bytes() == want


def test_failed_save_keeps_the_earlier_state(tmp_path):
    """Host-side failures after the data is written: when the rename fails
    (the path is a non-empty directory) the call returns ARK_OPT_EIO, the
    directory is as it was and no temporary file is left; when the directory
    cannot be written the temporary file cannot be created (EIO, nothing
    left either).  A symbolic link at the path is followed: the link stays
    and its target holds the new checkpoint."""
    import os
    import stat
    import torch
    from ark_amd._lib import lib
    L = lib()
    w = torch.arange(300, dtype=torch.float32, device="cuda").half()
    recs = (_abi.CkptRecord * 1)()
    recs[0] = _abi.CkptRecord(w.data_ptr(), 300, _abi.CKPT_F16, 0)
    want = K.write_v4(5, 6, [w.cpu().numpy().view(np.uint16)])
    # rename over a non-empty directory fails after the whole file was written
    d = tmp_path / "ckpt.ark"
    d.mkdir()
    (d / "inside").write_bytes(b"keep me")
    rc = L.ark_ckpt_save_v4(os.fsencode(str(d)), 5, 6, recs, 1, None, None)
    assert rc == _abi.EIO and "rename" in L.ark_opt_last_error().decode()
    assert sorted(os.listdir(tmp_path)) == ["ckpt.ark"]
    assert sorted(os.listdir(d)) == ["inside"] and (d / "inside").read_bytes() == b"keep me"
    # a directory that cannot be written: no temporary file, the old file kept
    ro = tmp_path / "ro"
    ro.mkdir()
    old = ro / "c.ark"
    old.write_bytes(b"earlier checkpoint")
    ro.chmod(stat.S_IRUSR | stat.S_IXUSR)
    try:
        if not os.access(ro, os.W_OK):  # root can write anyway
            rc = L.ark_ckpt_save_v4(os.fsencode(str(old)), 5, 6, recs, 1, None, None)
            assert rc == _abi.EIO and "create" in L.ark_opt_last_error().decode()
            assert sorted(os.listdir(ro)) == ["c.ark"] and old.read_bytes() == b"earlier checkpoint"
    finally:
        ro.chmod(stat.S_IRWXU)
    # a symbolic link at the path: the link stays, its target is replaced
    real = tmp_path / "real.ark"
    real.write_bytes(b"old")
    link = tmp_path / "latest.ark"
    link.symlink_to(real)
    assert L.ark_ckpt_save_v4(os.fsencode(str(link)), 5, 6, recs, 1, None, None) == 0
    assert link.is_symlink() and os.readlink(link) == str(real)
    assert real.read_bytes() == want
    assert sorted(os.listdir(tmp_path)) == ["ckpt.ark", "latest.ark", "real.ark", "ro"]


def test_save_keeps_modes_and_follows_links_as_file_create(tmp_path):
    """File::create (io.rs:450) semantics the save keeps although it writes a
    temporary file and renames it: a new file gets mode 0666 less the umask;
    a replaced file's mode carries over; a chain of symbolic links with
    relative targets is followed to the file it names, which becomes the
    checkpoint while the links stay; a dangling link is followed too, and
    the file it names is created."""
    import os
    import stat
    import torch
    from ark_amd._lib import lib
    L = lib()
    w = torch.arange(300, dtype=torch.float32, device="cuda").half()
    recs = (_abi.CkptRecord * 1)()
    recs[0] = _abi.CkptRecord(w.data_ptr(), 300, _abi.CKPT_F16, 0)
    want = K.write_v4(5, 6, [w.cpu().numpy().view(np.uint16)])

    def save(p):
        rc = L.ark_ckpt_save_v4(os.fsencode(str(p)), 5, 6, recs, 1, None, None)
        assert rc == 0, L.ark_opt_last_error().decode()

    umask = os.umask(0o022)
    os.umask(umask)
    new = tmp_path / "new.ark"
    save(new)
    assert stat.S_IMODE(new.stat().st_mode) == 0o666 & ~umask and new.read_bytes() == want
    for mode in (0o600, 0o640, 0o604):
        old = tmp_path / f"old{mode:o}.ark"
        old.write_bytes(b"earlier")
        old.chmod(mode)
        save(old)
        assert stat.S_IMODE(old.stat().st_mode) == mode and old.read_bytes() == want
    # link -> link2 -> d/real.ark, targets relative to each link's directory
    (tmp_path / "d").mkdir()
    real = tmp_path / "d" / "real.ark"
    real.write_bytes(b"old")
    real.chmod(0o640)
    (tmp_path / "link2").symlink_to("d/real.ark")
    (tmp_path / "link").symlink_to("link2")
    save(tmp_path / "link")
    assert os.readlink(tmp_path / "link") == "link2"
    assert os.readlink(tmp_path / "link2") == "d/real.ark"
    assert real.read_bytes() == want and stat.S_IMODE(real.stat().st_mode) == 0o640
    # a dangling link: the link stays and the file it names is created
    (tmp_path / "dangling").symlink_to("d/created.ark")
    save(tmp_path / "dangling")
    assert (tmp_path / "dangling").is_symlink()
    assert (tmp_path / "d" / "created.ark").read_bytes() == want
    assert sorted(os.listdir(tmp_path / "d")) == ["created.ark", "real.ark"]


@pytest.mark.parametrize("kind", ["v4_without_gamma_final", "v2_weights_only"])
def test_load_params_follows_the_file(tmp_path, kind):
    """load_params on the files the reference also resumes from: a V4 file
    without gamma_final fills everything else (gamma_final stays as it was)
    and sets t; a V2 file fills the weights, zeroes the moments and sets t
    to 0 (training.rs:488-509)."""
    torch = _torch()
    from ark_amd.optimizer import AdamConfig, AmpConfig, Optimizer
    cfg = EkoConfig(n_layers=2, d_model=16, hidden=24, vocab=40)
    ps = _params(cfg, 4)
    opt = Optimizer(AdamConfig(), ps, AmpConfig())
    opt.set_state(t=99)
    g = [sp.name for sp in ps.specs].index("gamma_final")
    before = {f: getattr(ps, f)(g).clone() for f in "wmv"}
    rng = np.random.default_rng(8)
    path = tmp_path / "f.ark"
    if kind == "v4_without_gamma_final":
        tens = ckpt.file_tensors(ps, 4, 3 + 27 * 2)
        host = [rng.integers(0, 0x7C00, t.numel(), dtype=np.uint32).astype(np.uint16)
                if t.element_size() == 2 else rng.standard_normal(t.numel()).astype(np.float32)
                for t in tens]
        path.write_bytes(K.write_v4(7, 31, host))
    else:
        tens = ckpt.file_tensors(ps, 2, 1 + 9 * 2)
        host = [rng.standard_normal(t.numel()).astype(np.float32) for t in tens]
        path.write_bytes(K.write_v2(7, host))
    info, amp = ckpt.load_params(str(path), ps, opt)
    torch.cuda.synchronize()
    assert amp is None and info.global_step == 7
    for t, h in zip(tens, host):
        got = _bits(t)
        want = h.view(np.uint16) if t.element_size() == 2 else h.view(np.uint32)
        if t.element_size() == 2 and h.dtype == np.float32:  # V2 fp32 into fp16 weights
            want = oracle.f32_to_f16(h).view(np.uint16)
        np.testing.assert_array_equal(got, want)
    if kind == "v4_without_gamma_final":
        assert opt.get_state().t == 31
        for f in "wmv":
            assert torch.equal(getattr(ps, f)(g), before[f])
    else:
        assert opt.get_state().t == 0
        assert torch.count_nonzero(ps.m_arena).item() == 0
        assert torch.count_nonzero(ps.v_arena).item() == 0
        assert torch.equal(ps.w(g), before["w"])
    opt.close()
