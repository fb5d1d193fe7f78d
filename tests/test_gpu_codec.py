"""GPU parity of the fp16 <-> fp32 weight codec (include/ark_codec.h) against
the oracle's conversions (the fcvtl / fcvtn rule of asm/kern.s:826-913):
every fp16 pattern, every fp32 pattern, NaN payloads included, through the
drop-in entry points and the one-launch plan over EKO-237M's tensors."""
import numpy as np
import pytest

import oracle
from ark_amd import codec
from ark_amd.eko import EKO_237M

pytestmark = pytest.mark.gpu


def _torch():
    import torch
    assert torch.cuda.is_available(), "GPU test run without a GPU"
    return torch


def _bits16(t):
    torch = _torch()
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def _bits32(t):
    torch = _torch()
    return t.view(torch.int32).cpu().numpy().view(np.uint32)


def test_dequant_every_f16_pattern():
    torch = _torch()
    allh = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = oracle.f16_to_f32(allh).view(np.uint32)
    src = torch.from_numpy(allh.view(np.int16)).cuda()
    dst = torch.empty(65536, dtype=torch.float32, device="cuda")
    codec.dequant_f16_to_f32(src, dst)
    torch.cuda.synchronize()
    got = _bits32(dst)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, f"{bad.size} patterns differ, first {allh[bad[0]]:#06x}"


def test_quant_every_f32_pattern():
    """All 2^32 inputs in 16 chunks of 2^28, each checked by the oracle."""
    torch = _torch()
    chunk = 1 << 28
    out = torch.empty(chunk, dtype=torch.int16, device="cuda")
    for lo in range(0, 1 << 32, chunk):
        x = torch.arange(lo, lo + chunk, dtype=torch.int64, device="cuda").to(torch.int32)
        codec.quant_f32_to_f16(x.view(torch.float32), out)
        got = out.cpu().numpy().view(np.uint16)
        del x
        bad, first = oracle.compare_f32_to_f16_range(lo, got, nthreads=16)
        assert bad == 0, f"chunk {lo:#x}: {bad} patterns differ, first {first:#010x}"


@pytest.mark.parametrize("n,off", [(1, 0), (7, 0), (8, 0), (4099, 0), (4099, 1), (1000, 3),
                                   (12345, 5)])
def test_ragged_and_unaligned(n, off):
    """Tails and pointers off the 16-byte grid take the per-element path."""
    torch = _torch()
    rng = np.random.default_rng(n * 31 + off)
    h = rng.integers(0, 65536, size=n + off, dtype=np.uint32).astype(np.uint16)
    src = torch.from_numpy(h.view(np.int16)).cuda()
    dst = torch.full((n + off,), -7.0, dtype=torch.float32, device="cuda")
    codec.dequant_f16_to_f32(src[off:], dst[off:])
    q = torch.full((n + off,), 0x1234, dtype=torch.int16, device="cuda")
    codec.quant_f32_to_f16(dst[off:], q[off:])
    torch.cuda.synchronize()
    got = _bits32(dst)
    assert (got[:off] == np.float32(-7.0).view(np.uint32)).all()
    assert (got[off:] == oracle.f16_to_f32(h[off:]).view(np.uint32)).all()
    gq = _bits16(q)
    assert (gq[:off] == 0x1234).all()
    assert (gq[off:] == oracle.f32_to_f16(got[off:].view(np.float32))).all()


def test_plan_eko237m_round_trip():
    """Dequantise all 272 EKO-237M weight tensors in one launch, quantise back:
    every fp16 pattern returns unchanged except signalling NaNs, which come
    back quiet (the bits compared against the oracle on a sample)."""
    torch = _torch()
    specs = EKO_237M.tensors()
    g = torch.Generator(device="cuda").manual_seed(5)
    w = [torch.randint(-32768, 32768, (s.n,), dtype=torch.int32, device="cuda",
                       generator=g).to(torch.int16) for s in specs]
    f = [torch.empty(s.n, dtype=torch.float32, device="cuda") for s in specs]
    back = [torch.empty(s.n, dtype=torch.int16, device="cuda") for s in specs]
    dq = codec.CodecPlan(list(zip(w, f)), "f16_to_f32")
    qt = codec.CodecPlan(list(zip(f, back)), "f32_to_f16")
    for _ in range(2):
        dq.run()
        qt.run()
    torch.cuda.synchronize()
    for i, (a, b, c) in enumerate(zip(w, f, back)):
        a16 = _bits16(a)
        want = a16.copy()
        snan = ((a16 & 0x7C00) == 0x7C00) & ((a16 & 0x03FF) != 0) & ((a16 & 0x0200) == 0)
        want[snan] |= 0x0200
        assert (_bits16(c) == want).all(), f"tensor {i} ({specs[i].name})"
        if i < 4 or specs[i].n <= 4096:
            assert (_bits32(b) == oracle.f16_to_f32(a16).view(np.uint32)).all(), i
    dq.close()
    qt.close()


def test_plan_matches_single_calls():
    torch = _torch()
    sizes = [1, 4096, 4097, 8191, 100000, 768]
    src = [torch.randn(n, device="cuda", dtype=torch.float32) * 1e3 for n in sizes]
    a = [torch.empty(n, dtype=torch.float16, device="cuda") for n in sizes]
    b = [torch.empty(n, dtype=torch.float16, device="cuda") for n in sizes]
    p = codec.CodecPlan(list(zip(src, a)), "f32_to_f16")
    p.run()
    for s, t in zip(src, b):
        codec.quant_f32_to_f16(s, t)
    torch.cuda.synchronize()
    for x, y in zip(a, b):
        assert torch.equal(x.view(torch.int16), y.view(torch.int16))
    p.close()


def test_rejects_bad_buffers():
    torch = _torch()
    from ark_amd._lib import ArkOptError, check, lib
    x = torch.zeros(16, dtype=torch.float32, device="cuda")
    y = torch.zeros(16, dtype=torch.int16, device="cuda")
    with pytest.raises(ArkOptError, match="exceeds its allocation"):
        check(lib().ark_hip_quant_f32_to_f16(x.data_ptr(), y.data_ptr(), 1 << 30, None))
    h = np.zeros(16, np.float32)
    with pytest.raises(ArkOptError, match="host memory|not memory known"):
        check(lib().ark_hip_quant_f32_to_f16(h.ctypes.data, y.data_ptr(), 16, None))
    with pytest.raises(ArkOptError, match="overlap"):
        check(lib().ark_hip_dequant_f16_to_f32(x.data_ptr(), x.data_ptr() + 4, 4, None))


@pytest.mark.parametrize("case", range(6))
def test_plan_spans_at_random_alignments(case):
    """Seeded codec plans of 1-40 spans, from empty through a few elements,
    around one 4096-element segment and up to ~70k, each source and
    destination at its own element offset inside its own allocation (so most
    spans miss the 16-byte grid and take the element path), one source shared
    by two spans; dequantise every fp16 pattern class, then quantise the
    results back: both directions against the oracle's conversions bit for
    bit."""
    torch = _torch()
    rng = np.random.default_rng(700 + case)
    spans = []
    for _ in range(int(rng.integers(1, 41))):
        r = rng.random()
        n = (0 if r < 0.1 else int(rng.integers(1, 9)) if r < 0.3 else
             int(rng.integers(4090, 4103)) if r < 0.5 else int(rng.integers(9, 70000)))
        spans.append((n, int(rng.integers(0, 8)), int(rng.integers(0, 4)), int(rng.integers(0, 8))))
    bits, src, mid, back = [], [], [], []
    shared = None
    for n, os_, om, ob in spans:
        if shared is not None and shared[0].size == n and rng.random() < 0.5:
            h, s16 = shared
        else:
            h = rng.integers(0, 65536, n, dtype=np.uint32).astype(np.uint16)
            base = torch.empty(n + 8, dtype=torch.int16, device="cuda")
            base[os_:os_ + n] = torch.from_numpy(h.view(np.int16)).cuda()
            s16 = base[os_:os_ + n].view(torch.float16)
            shared = (h, s16)
        bits.append(h)
        src.append(s16)
        mid.append(torch.empty(n + 4, dtype=torch.float32, device="cuda")[om:om + n])
        back.append(torch.empty(n + 8, dtype=torch.float16, device="cuda")[ob:ob + n])
    up = codec.CodecPlan(list(zip(src, mid)), "f16_to_f32")
    up.run()
    torch.cuda.synchronize()
    for i, (h, d) in enumerate(zip(bits, mid)):
        want = oracle.f16_to_f32(h) if h.size else np.zeros(0, np.float32)
        assert np.array_equal(d.cpu().numpy().view(np.uint32), want.view(np.uint32)), (case, i)
    up.close()
    down = codec.CodecPlan(list(zip(mid, back)), "f32_to_f16")
    down.run()
    torch.cuda.synchronize()
    for i, (d, b) in enumerate(zip(mid, back)):
        f = d.cpu().numpy()
        want = oracle.f32_to_f16(f) if f.size else np.zeros(0, np.uint16)
        got = b.view(torch.int16).cpu().numpy().view(np.uint16)
        assert np.array_equal(got, want), (case, i)
    down.close()


def test_plans_over_thousands_of_tiny_spans():
    """2000 spans of 0-300 elements (empty ones skipped) in one codec plan
    and one accumulation plan, against the oracle's conversion and an fp32
    add: every segment ragged, a 2000-entry descriptor table."""
    torch = _torch()
    from ark_amd import grad
    rng = np.random.default_rng(21)
    sizes = [int(x) for x in rng.integers(0, 301, 2000)]
    h16 = [rng.integers(0, 65536, n, dtype=np.uint32).astype(np.uint16) for n in sizes]
    src = [torch.from_numpy(h.view(np.int16)).cuda().view(torch.float16) for h in h16]
    dst = [torch.empty(n, dtype=torch.float32, device="cuda") for n in sizes]
    plan = codec.CodecPlan(list(zip(src, dst)), "f16_to_f32")
    plan.run()
    torch.cuda.synchronize()
    for h, d in zip(h16, dst):
        want = oracle.f16_to_f32(h) if h.size else np.zeros(0, np.float32)
        assert np.array_equal(d.cpu().numpy().view(np.uint32), want.view(np.uint32))
    plan.close()
    a = [torch.randn(n, device="cuda") for n in sizes]
    b = [torch.randn(n, device="cuda") for n in sizes]
    want = [x + y for x, y in zip(a, b)]
    gp = grad.GradPlan(list(zip(a, b)))
    gp.run()
    torch.cuda.synchronize()
    assert all(torch.equal(x.view(torch.int32), w.view(torch.int32)) for x, w in zip(a, want))
    gp.close()
