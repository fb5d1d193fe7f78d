"""GPU parity of the gradient hand-off (include/ark_grad.h) against the
oracle's literal restatement of the CPU loops of objc/bridge.m:902-948:
fp32 accumulation of every gradient buffer, the LM-head and gamma_final
adds, and the token scatter-add into the embedding gradient with the loop's
summation order; then the produced fp32 gradients through ark_opt_step
against the oracle's optimizer."""
import numpy as np
import pytest

import oracle
from ark_amd import grad
from ark_amd.eko import EKO_237M

pytestmark = pytest.mark.gpu


def _torch():
    import torch
    assert torch.cuda.is_available(), "GPU test run without a GPU"
    return torch


def _bits(t):
    torch = _torch()
    return t.view(torch.int32).cpu().numpy().view(np.uint32)


def _zipf_tokens(rng, n, vocab, extra=0):
    t = (rng.zipf(1.2, n) - 1) % (vocab + extra)
    return t.astype(np.uint32)


@pytest.mark.parametrize("vocab,d,n,extra", [(32000, 768, 4096, 0), (32000, 768, 4096, 50),
                                             (1000, 33, 777, 10), (5, 64, 2000, 2),
                                             (32000, 768, 1, 0), (32768, 768, 4096, 0),
                                             (32000, 768, 4097, 0), (32000, 768, 4146, 0),
                                             (32000, 256, 9000, 5), (32000, 64, 8192, 0),
                                             (256, 16, 12289, 3), (1, 8, 5000, 4),
                                             (70000, 8, 20000, 100), (100000, 4, 70001, 0)])
def test_scatter_matches_oracle(vocab, d, n, extra):
    """Up to 4096 tokens the positions are sorted by one block in LDS, past
    that by one hist/scan/scatter launch triple per 8-bit digit over
    4096-token tiles: two tiles exactly (8192), a one-token last tile
    (4097, 12289), one pass (vocab 256 and 1), two, and three (vocab 70000
    and 100000 take 17 key bits); vocab 32768 puts the largest real key on
    the block sort's padding key."""
    torch = _torch()
    rng = np.random.default_rng(vocab + d + n)
    tokens = _zipf_tokens(rng, n, vocab, extra)
    dx0 = (rng.standard_normal((n, d)) * 10.0 ** rng.integers(-6, 3, (n, 1))).astype(np.float32)
    g = rng.standard_normal((vocab, d)).astype(np.float32)
    want = g.copy()
    oracle.embed_scatter(want, tokens, dx0)
    gg = torch.from_numpy(g).cuda()
    grad.embed_scatter(gg, torch.from_numpy(tokens.view(np.int32)).cuda(),
                       torch.from_numpy(dx0).cuda())
    got = _bits(gg).reshape(vocab, d)
    bad = np.argwhere(got != want.view(np.uint32))
    assert bad.size == 0, f"{len(bad)} elements differ, first {bad[0].tolist()}"


def test_scatter_largest_key_ties_with_the_block_sort_padding():
    """vocab 32768 sorts over 15 bits, where the padding past n (all-ones key)
    equals the largest real key 32767: the real rows of that token must still
    come first, in order, and only they are added."""
    torch = _torch()
    vocab, d, n = 32768, 64, 1000
    rng = np.random.default_rng(13)
    tokens = rng.integers(0, vocab, n).astype(np.uint32)
    tokens[::7] = vocab - 1
    tokens[3] = vocab + 5  # out of range: row 0
    dx0 = rng.standard_normal((n, d)).astype(np.float32)
    g = rng.standard_normal((vocab, d)).astype(np.float32)
    want = g.copy()
    oracle.embed_scatter(want, tokens, dx0)
    gg = torch.from_numpy(g).cuda()
    grad.embed_scatter(gg, torch.from_numpy(tokens.view(np.int32)).cuda(),
                       torch.from_numpy(dx0).cuda())
    np.testing.assert_array_equal(_bits(gg).reshape(vocab, d), want.view(np.uint32))


@pytest.mark.parametrize("n", [4097, 8191, 8193])
def test_scatter_largest_key_ties_with_the_last_tile_padding(n):
    """Past one tile the last tile's positions beyond n carry the all-ones
    key too; the real rows of token 32767 (the largest key over 15 bits)
    spread over every tile must keep their order and land before it."""
    torch = _torch()
    vocab, d = 32768, 16
    rng = np.random.default_rng(n)
    tokens = rng.integers(0, vocab, n).astype(np.uint32)
    tokens[::5] = vocab - 1
    tokens[-3:] = vocab - 1
    tokens[7] = vocab + 9  # out of range: row 0
    dx0 = (rng.standard_normal((n, d)) * 10.0 ** rng.integers(-4, 4, (n, 1))).astype(np.float32)
    g = rng.standard_normal((vocab, d)).astype(np.float32)
    want = g.copy()
    oracle.embed_scatter(want, tokens, dx0)
    gg = torch.from_numpy(g).cuda()
    grad.embed_scatter(gg, torch.from_numpy(tokens.view(np.int32)).cuda(),
                       torch.from_numpy(dx0).cuda())
    np.testing.assert_array_equal(_bits(gg).reshape(vocab, d), want.view(np.uint32))


def test_scatter_one_long_run_across_tiles():
    """One token at all 10000 positions: a single run that the multi-tile
    sort must keep in position order across three tiles, added with the
    order-revealing values (1e8, 1, -1e8, 1) at the tile seams."""
    torch = _torch()
    vocab, d, n = 50, 64, 10000
    rng = np.random.default_rng(17)
    dx0 = rng.standard_normal((n, d)).astype(np.float32)
    for seam in (4094, 8190):
        dx0[seam:seam + 4, :] = np.array([1e8, 1.0, -1e8, 1.0], np.float32)[:, None]
    tokens = np.full(n, 31, np.uint32)
    want = np.zeros((vocab, d), np.float32)
    oracle.embed_scatter(want, tokens, dx0)
    gg = torch.zeros(vocab, d, device="cuda")
    grad.embed_scatter(gg, torch.from_numpy(tokens.view(np.int32)).cuda(),
                       torch.from_numpy(dx0).cuda())
    np.testing.assert_array_equal(_bits(gg).reshape(vocab, d), want.view(np.uint32))


def test_scatter_one_long_run_and_order():
    """Every position the same token: one run of 4096 rows added in order;
    plus the order-revealing values (1e8, 1, -1e8, 1)."""
    torch = _torch()
    vocab, d, n = 100, 256, 4096
    rng = np.random.default_rng(7)
    dx0 = rng.standard_normal((n, d)).astype(np.float32)
    dx0[:4, :] = np.array([1e8, 1.0, -1e8, 1.0], np.float32)[:, None]
    tokens = np.full(n, 42, np.uint32)
    want = np.zeros((vocab, d), np.float32)
    oracle.embed_scatter(want, tokens, dx0)
    gg = torch.zeros(vocab, d, device="cuda")
    grad.embed_scatter(gg, torch.from_numpy(tokens.view(np.int32)).cuda(),
                       torch.from_numpy(dx0).cuda())
    np.testing.assert_array_equal(_bits(gg).reshape(vocab, d), want.view(np.uint32))


@pytest.mark.parametrize("d", [768, 770, 5])
def test_scatter_run_lengths_at_the_path_boundaries(d):
    """Runs of 1, 7 and 8 rows (the short and long paths meet at 8) and of
    59, 60, 61, 120, 121 and 500 rows (the long path adds 60 rows per round,
    then a tail), positions shuffled, against the oracle."""
    torch = _torch()
    rng = np.random.default_rng(d)
    lengths = [1, 7, 8, 59, 60, 61, 120, 121, 500]
    vocab = 1000
    ids = rng.choice(vocab, len(lengths), replace=False)
    tokens = np.concatenate([np.full(k, t, np.uint32) for k, t in zip(lengths, ids)])
    tokens = tokens[rng.permutation(len(tokens))]
    n = len(tokens)
    dx0 = (rng.standard_normal((n, d)) * 10.0 ** rng.integers(-4, 4, (n, 1))).astype(np.float32)
    g = rng.standard_normal((vocab, d)).astype(np.float32)
    want = g.copy()
    oracle.embed_scatter(want, tokens, dx0)
    gg = torch.from_numpy(g).cuda()
    grad.embed_scatter(gg, torch.from_numpy(tokens.view(np.int32)).cuda(),
                       torch.from_numpy(dx0).cuda())
    np.testing.assert_array_equal(_bits(gg).reshape(vocab, d), want.view(np.uint32))


@pytest.mark.parametrize("d,g_off", [(768, 0), (4, 0), (68, 0), (100, 0), (1028, 0), (768, 1)])
def test_scatter_long_runs_at_odd_widths(d, g_off):
    """Runs of 127 to 1500 rows (many 60-row rounds, then a tail) at widths
    that leave a partial column tile (4, 68, 100, 1028), and with an
    embedding gradient that is only 4-byte aligned (g_off = 1); the
    order-revealing values (1e8, 1, -1e8, 1) straddle rows 510-513 of the
    1500-row run."""
    torch = _torch()
    rng = np.random.default_rng(100 + d + g_off)
    lengths = [127, 128, 129, 255, 256, 257, 511, 512, 513, 1024, 1025, 1500, 3]
    vocab = 2000
    ids = rng.choice(vocab, len(lengths), replace=False)
    tokens = np.concatenate([np.full(k, t, np.uint32) for k, t in zip(lengths, ids)])
    tokens = tokens[rng.permutation(len(tokens))]
    n = len(tokens)
    dx0 = (rng.standard_normal((n, d)) * 10.0 ** rng.integers(-4, 4, (n, 1))).astype(np.float32)
    rows = np.flatnonzero(tokens == ids[lengths.index(1500)])
    dx0[rows[510:514], :] = np.array([1e8, 1.0, -1e8, 1.0], np.float32)[:, None]
    g = rng.standard_normal((vocab, d)).astype(np.float32)
    want = g.copy()
    oracle.embed_scatter(want, tokens, dx0)
    base = torch.zeros(vocab * d + g_off, device="cuda")
    gg = base[g_off:].view(vocab, d)
    gg.copy_(torch.from_numpy(g))
    grad.embed_scatter(gg, torch.from_numpy(tokens.view(np.int32)).cuda(),
                       torch.from_numpy(dx0).cuda())
    np.testing.assert_array_equal(_bits(gg).reshape(vocab, d), want.view(np.uint32))


def test_scatter_unaligned_rows_take_the_scalar_path():
    torch = _torch()
    vocab, d, n = 300, 64, 500
    rng = np.random.default_rng(8)
    tokens = _zipf_tokens(rng, n, vocab)
    base = torch.from_numpy(rng.standard_normal(n * d + 1).astype(np.float32)).cuda()
    dx0 = base[1:].view(n, d)  # 4-byte, not 16-byte, aligned
    want = np.zeros((vocab, d), np.float32)
    oracle.embed_scatter(want, tokens, dx0.cpu().numpy())
    gg = torch.zeros(vocab, d, device="cuda")
    grad.embed_scatter(gg, torch.from_numpy(tokens.view(np.int32)).cuda(), dx0)
    np.testing.assert_array_equal(_bits(gg).reshape(vocab, d), want.view(np.uint32))


def test_accumulate_and_plan_eko237m():
    """All 272 EKO-237M fp32 gradient buffers += their backward outputs in
    one launch, against torch's fp32 add (an independent reference of an
    elementwise IEEE add) and the oracle on the small tensors."""
    torch = _torch()
    specs = EKO_237M.tensors()
    g = torch.Generator(device="cuda").manual_seed(3)
    dst = [torch.randn(s.n, device="cuda", generator=g) for s in specs]
    src = [torch.randn(s.n, device="cuda", generator=g) * 1e-3 for s in specs]
    want = [a + b for a, b in zip(dst, src)]
    small = [(i, dst[i].cpu().numpy().copy(), src[i].cpu().numpy()) for i, s in enumerate(specs)
             if s.n <= 768 * 2048][:12]
    plan = grad.GradPlan(list(zip(dst, src)))
    plan.run()
    torch.cuda.synchronize()
    for a, w in zip(dst, want):
        assert torch.equal(a.view(torch.int32), w.view(torch.int32))
    for i, a, b in small:
        oracle.grad_accumulate(a, b)
        np.testing.assert_array_equal(_bits(dst[i]), a.view(np.uint32))
    plan.close()
    x = torch.randn(4099, device="cuda")
    y = torch.randn(4100, device="cuda")[1:]  # unaligned source
    w = x + y
    grad.accumulate(x, y)
    torch.cuda.synchronize()
    assert torch.equal(x, w)


@pytest.mark.parametrize("case", range(8))
def test_plan_spans_at_random_alignments(case):
    """Seeded plans of 1-40 spans, from empty through a few elements,
    around one 4096-element segment and up to ~70k, each dst and src at its
    own element offset (0-3, so 4-byte but mostly not 16-byte aligned: the
    element path) in its own allocation, one source shared by two spans:
    every result bit equal to torch's fp32 add, and a plain accumulation of
    one such span too."""
    torch = _torch()
    rng = np.random.default_rng(500 + case)
    g = torch.Generator(device="cuda").manual_seed(case)
    pairs, want = [], []
    shared = None
    for _ in range(int(rng.integers(1, 41))):
        r = rng.random()
        n = (0 if r < 0.1 else int(rng.integers(1, 9)) if r < 0.3 else
             int(rng.integers(4090, 4103)) if r < 0.5 else int(rng.integers(9, 70000)))
        od, os_ = (int(x) for x in rng.integers(0, 4, 2))
        d = torch.randn(n + 4, device="cuda", generator=g)[od:od + n]
        if shared is not None and shared.numel() == n and rng.random() < 0.5:
            src = shared
        else:
            src = torch.randn(n + 4, device="cuda", generator=g)[os_:os_ + n] * 1e-2
            shared = src
        want.append(d + src)
        pairs.append((d, src))
    plan = grad.GradPlan(pairs)
    plan.run()
    torch.cuda.synchronize()
    for i, ((d, _), w) in enumerate(zip(pairs, want)):
        assert torch.equal(d.view(torch.int32), w.view(torch.int32)), (case, i, d.numel())
    plan.close()
    d, src = pairs[-1]
    w = d + src
    grad.accumulate(d, src)
    torch.cuda.synchronize()
    assert torch.equal(d.view(torch.int32), w.view(torch.int32))


@pytest.mark.parametrize("d_model,fused", [(64, False), (256, True), (64, True)])
def test_handoff_into_optimizer_step(d_model, fused):
    """The backward tail on the device feeding ark_opt_step (fp32 grads):
    every gradient buffer += its backward output (the LM-head add is the
    embedding's), then the token scatter, then one AMP + clip + AdamW step;
    gradients, step scalars and w/m/v against the oracle's loops and
    optimizer, bit for bit.  fused: the accumulation and the scatter write
    the norm's units and the step reads them instead of the gradients."""
    torch = _torch()
    from ark_amd import _abi
    from ark_amd.eko import EkoConfig
    from ark_amd.optimizer import AdamConfig, AmpConfig, Optimizer, ParamSet
    from oracle import harness as H

    cfg = EkoConfig(n_layers=2, d_model=d_model, hidden=96, vocab=500)
    specs = cfg.tensors()
    rng = np.random.default_rng(11)
    scale = 1024.0
    ps = ParamSet(specs, weight_decay=0.1, grad_dtype=_abi.GRAD_F32)
    w0 = [(rng.standard_normal(s.n) * 0.02).astype(np.float16) for s in specs]
    for i in range(len(specs)):
        ps.w(i).copy_(torch.from_numpy(w0[i]))
    outs = [(rng.standard_normal(s.n) * 1e-3 * scale).astype(np.float32) for s in specs]
    n_tok = 300
    tokens = _zipf_tokens(rng, n_tok, cfg.vocab, 3)
    dx0 = (rng.standard_normal((n_tok, cfg.d_model)) * 1e-3 * scale).astype(np.float32)
    e = [s.name for s in specs].index("embed")
    # device: grads start at zero (training.rs:248), += outputs, then the scatter
    dev_out = [torch.from_numpy(o).cuda() for o in outs]
    plan = grad.GradPlan([(ps.g(i), dev_out[i]) for i in range(len(specs))])
    acfg = AdamConfig(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1, grad_clip=1.0)
    opt = Optimizer(acfg, ps, AmpConfig(loss_scale_init=scale))
    plan.run(final_for=opt if fused else None)
    grad.embed_scatter(ps.g(e).view(cfg.vocab, cfg.d_model),
                       torch.from_numpy(tokens.view(np.int32)).cuda(), torch.from_numpy(dx0).cuda(),
                       final_for=opt if fused else None)
    _, gi = opt.step_all(3e-4, info=True)
    # host: the same loops, then the oracle optimizer on the same inputs
    host_g = [np.zeros(s.n, np.float32) for s in specs]
    for h, o in zip(host_g, outs):
        oracle.grad_accumulate(h, o)
    oracle.embed_scatter(host_g[e].reshape(cfg.vocab, cfg.d_model), tokens, dx0)
    for i in range(len(specs)):
        np.testing.assert_array_equal(_bits(ps.g(i)), host_g[i].view(np.uint32))
    ts = [oracle.HostTensor(w0[i].view(np.uint16).copy(), host_g[i], np.zeros(s.n, np.float32),
                            np.zeros(s.n, np.float32), 0.1 if s.decay else 0.0)
          for i, s in enumerate(specs)]
    ref = oracle.Optimizer(ts, opt.hp)
    _, ri = ref.step(3e-4)
    d = H.info_matches(gi, ri)
    assert not d, d
    assert gi.applied == 1
    c = H.compare(ps, ts)
    assert c["w"] == 0 and c["m"] == 0 and c["v"] == 0, c
    opt.close()
    plan.close()


def test_entry_points_reject_host_or_short_buffers():
    """The accumulation, a gradient plan and the scatter check every buffer
    on the host before any launch: host memory and a span longer than its
    allocation are refused with EINVAL and a message naming the buffer."""
    import ctypes as C
    from ark_amd import _abi
    from ark_amd._lib import lib
    torch = _torch()
    L = lib()
    msg = lambda: L.ark_opt_last_error().decode()
    dst = torch.zeros(1000, device="cuda")
    src = torch.zeros(1000, device="cuda")
    host = np.zeros(1000, np.float32)
    assert L.ark_grad_accumulate(dst.data_ptr(), host.ctypes.data, 1000, None) == _abi.EINVAL
    assert "host memory" in msg() or "not memory known" in msg(), msg()
    assert L.ark_grad_accumulate(dst.data_ptr(), src.data_ptr(), 1 << 28, None) == _abi.EINVAL
    assert "exceeds its allocation" in msg(), msg()
    dst2 = torch.zeros(1000, device="cuda")
    spans = (_abi.GradSpan * 2)()
    spans[0] = _abi.GradSpan(dst.data_ptr(), src.data_ptr(), 1000)
    spans[1] = _abi.GradSpan(dst2.data_ptr(), host.ctypes.data, 1000)
    h = C.c_void_p()
    assert L.ark_grad_plan_create(spans, 2, None, C.byref(h)) == _abi.EINVAL
    assert "buffer 1" in msg() and not h.value, msg()
    g = torch.zeros(100, 64, device="cuda")
    dx0 = torch.zeros(10, 64, device="cuda")
    tokens = np.zeros(10, np.uint32)
    rc = L.ark_grad_embed_scatter(g.data_ptr(), 100, 64, tokens.ctypes.data, dx0.data_ptr(), 10,
                                  None)
    assert rc == _abi.EINVAL and "tokens" in msg(), msg()
    tok_dev = torch.zeros(1 << 22, dtype=torch.int32, device="cuda")  # 4M tokens, dx0 holds 10 rows
    rc = L.ark_grad_embed_scatter(g.data_ptr(), 100, 64, tok_dev.data_ptr(), dx0.data_ptr(),
                                  1 << 22, None)
    assert rc == _abi.EINVAL and "dx0" in msg() and "exceeds its allocation" in msg(), msg()
    torch.cuda.synchronize()
    assert torch.count_nonzero(g).item() == 0 and torch.count_nonzero(dst).item() == 0


def test_plans_refuse_more_segments_than_one_launch_covers():
    """A gradient plan launches 16 one-wave blocks per 4096-element segment
    and a codec plan 512 work-items per segment, all in one launch, whose
    work-items must stay below 2^32: 4,194,303 and 8,388,607 segments are
    the most they take, one more is refused with ARK_OPT_EINVAL.  Spans here
    all share one small dst, so a table of exactly the limit passes the
    segment count and is then refused for the shared dst (the overlap check
    follows the count; a table of disjoint spans that large would need tens
    of GB)."""
    import ctypes as C
    torch = _torch()
    from ark_amd import _abi
    from ark_amd._lib import lib
    L = lib()
    dst = torch.zeros(4096, device="cuda")
    src = torch.zeros(4096, device="cuda")
    half = torch.zeros(4096, dtype=torch.float16, device="cuda")
    stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    for limit, make, fields in (
            (4194303, L.ark_grad_plan_create, (dst, src)),
            (8388607, L.ark_codec_plan_create, (half, dst))):
        arr = np.zeros(limit + 1, dtype=[("a", "<u8"), ("b", "<u8"), ("n", "<u8")])
        arr["a"], arr["b"], arr["n"] = fields[0].data_ptr(), fields[1].data_ptr(), 4096
        h = C.c_void_p()
        if make is L.ark_grad_plan_create:
            spans = arr.ctypes.data_as(C.POINTER(_abi.GradSpan))
            call = lambda k: make(spans, k, stream, C.byref(h))
        else:
            spans = arr.ctypes.data_as(C.POINTER(_abi.CodecSpan))
            call = lambda k: make(spans, k, _abi.CODEC_F16_TO_F32, stream, C.byref(h))
        assert call(limit + 1) == _abi.EINVAL
        assert "too many elements" in L.ark_opt_last_error().decode()
        assert call(limit) == _abi.EINVAL and not h.value
        m = L.ark_opt_last_error().decode()
        assert "overlaps" in m and "too many" not in m, m


@pytest.mark.parametrize("case", range(40))
def test_random_scatters_match_the_loop(case):
    """Seeded random token scatters against the loop of bridge.m:922-928:
    vocabularies up to 2^17 (three sort passes past one tile), widths that
    are and are not multiples of 4 and 256, batches on both sides of the
    one-block sort's 4096-token tile, uniform, Zipf, single-token, sorted,
    reversed and out-of-range token draws, and embedding rows at an element
    offset; the allocating and the no-allocation forms, bit for bit."""
    torch = _torch()
    from ark_amd._lib import ArkOptError
    rng = np.random.default_rng(7000 + case)
    vocab = int(rng.choice([1, 2, 7, 256, 1000, 32000, 70000, 1 << 17]))
    d = int(rng.choice([1, 3, 4, 5, 64, 255, 256, 257, 768, 1024]))
    batch = int(rng.choice([0, 1, 2, 4095, 4096, 4097, 8192, 12289, int(rng.integers(1, 20000))]))
    d = max(1, min(d, 8_000_000 // max(batch, 1), 16_000_000 // vocab))
    dist = str(rng.choice(["uniform", "zipf", "same", "oob", "sorted", "reversed"]))
    if dist == "uniform":
        t = rng.integers(0, vocab, batch)
    elif dist == "zipf":
        t = np.minimum(rng.zipf(1.2, batch) - 1, vocab - 1)
    elif dist == "same":
        t = np.full(batch, rng.integers(0, vocab))
    elif dist == "oob":
        t = rng.integers(0, vocab * 2 + 5, batch)
    else:
        t = np.sort(rng.integers(0, vocab, batch))
        if dist == "reversed":
            t = t[::-1]
    t = np.ascontiguousarray(t, dtype=np.uint32)
    dx0 = (rng.standard_normal((batch, d)) * 10.0 ** rng.uniform(-3, 3)).astype(np.float32)
    base = rng.standard_normal((vocab, d)).astype(np.float32)
    off = int(rng.choice([0, 0, 1, 3]))
    want = base.copy()
    oracle.embed_scatter(want, t, dx0)
    case_info = dict(vocab=vocab, d=d, batch=batch, dist=dist, off=off)
    for noalloc in (False, True):
        buf = torch.zeros(vocab * d + off, device="cuda")
        eg = buf[off:off + vocab * d].view(vocab, d)
        eg.copy_(torch.from_numpy(base))
        tt = torch.from_numpy(t.view(np.int32)).cuda()
        xx = torch.from_numpy(dx0).cuda()
        try:
            grad.embed_scatter(eg, tt, xx, noalloc=noalloc)
        except ArkOptError as e:
            assert noalloc and "static scratch" in str(e), (case_info, str(e))
            continue
        got = eg.cpu().numpy()
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (case_info, noalloc)
