"""The norm's sharding across GPUs (designed, not built: one GPU here).

aligned: each rank owns an aligned power-of-two block of the global
4096-element segment list, so its partial sum of squares is one subtree of
the canonical tree; one all-gather of one double per rank, then the same
pairwise finish on every rank.

balanced: each rank owns a contiguous run of the segment list of equal
length to within one segment (any number of ranks), which splits into at
most 2 log2(P) aligned dyadic blocks, each a subtree; the ranks all-gather
their (start, size, sum) entries and every rank rebuilds the tree from them,
taking a node's value from an entry where one covers it exactly and zero
for nodes past the last segment.

Either way every rank gets the single-device sum bit for bit, and a
non-finite gradient on any rank turns every rank's sum into NaN.  Checked
here with the CPU oracle standing in for each rank's norm pass, on gloo
ranks (one process each, 127.0.0.1)."""
import socket

import numpy as np
import pytest

SEG = 4096
SIZES = [5000, 3 * SEG, 17, 9000, SEG, 123, 2 * SEG + 1]  # 10 segments, padded to 16


def _tensors(nan_at=None):
    rng = np.random.default_rng(17)
    gs = [(rng.standard_normal(n) * 1e3).astype(np.float16).view(np.uint16) for n in SIZES]
    if nan_at is not None:
        gs[nan_at[0]][nan_at[1]] = 0x7E00
    return gs


def _host(gs):
    import oracle
    return [oracle.HostTensor(np.zeros(g.size, np.uint16), g, np.zeros(g.size, np.float32),
                              np.zeros(g.size, np.float32), 0.0) for g in gs]


def _segments(gs):
    return [(t, k) for t, g in enumerate(gs) for k in range((g.size + SEG - 1) // SEG)]


def _padded(n):
    p = 1
    while p < n:
        p *= 2
    return p


def _rank_pieces(gs, rank, world):
    """The gradient pieces of rank's aligned block of segments."""
    segs = _segments(gs)
    per = _padded(max(len(segs), world)) // world
    return _pieces(gs, segs[rank * per:(rank + 1) * per])


def _pieces(gs, mine):
    """Whole segments (t, k) of each tensor as slices, cut only at segment
    boundaries."""
    pieces = []
    for t, k in mine:
        lo, hi = k * SEG, min((k + 1) * SEG, gs[t].size)
        if pieces and pieces[-1][0] == t and pieces[-1][2] == lo:
            pieces[-1][2] = hi
        else:
            pieces.append([t, lo, hi])
    return [np.ascontiguousarray(gs[t][lo:hi]) for t, lo, hi in pieces]


def _dyadic(a, b):
    """[a, b) as aligned power-of-two blocks (start, size), largest first."""
    out = []
    while a < b:
        size = 1
        while a % (2 * size) == 0 and a + 2 * size <= b:
            size *= 2
        out.append((a, size))
        a += size
    return out


def _assemble(entries, nseg):
    """The canonical root from (start, size) -> subtree sums covering the
    segments [0, nseg) exactly."""
    def node(start, size):
        if (start, size) in entries:
            return entries[(start, size)]
        if start >= nseg:
            return 0.0
        assert size > 1, ("segment not covered", start)
        h = size // 2
        return node(start, h) + node(start + h, h)
    return node(0, _padded(nseg))


def _finish(parts):
    """The pairwise tree over the ranks' partials (len a power of two)."""
    parts = list(parts)
    while len(parts) > 1:
        parts = [parts[i] + parts[i + 1] for i in range(0, len(parts), 2)]
    return parts[0]


def _worker(rank, world, port, nan_at, out, scheme="aligned"):
    import torch
    import torch.distributed as dist
    import oracle
    from ark_amd import _abi
    dist.init_process_group("gloo", init_method=f"tcp://127.0.0.1:{port}", rank=rank,
                            world_size=world)
    sumsq = lambda pieces: oracle.sumsq(_host(pieces), _abi.GRAD_F16, 1.0 / 1024)[0]
    try:
        gs = _tensors(nan_at)
        if scheme == "aligned":
            pieces = _rank_pieces(gs, rank, world)
            part = sumsq(pieces) if pieces else 0.0
            got = [torch.zeros(1, dtype=torch.float64) for _ in range(world)]
            dist.all_gather(got, torch.tensor([part], dtype=torch.float64))
            total = _finish(float(x.item()) for x in got)
        else:
            segs = _segments(gs)
            S = len(segs)
            a, b = rank * S // world, (rank + 1) * S // world
            # a fixed-size record per rank: up to 2 log2(P) + 2 entries of
            # (start, size, sum); size 0 marks an unused entry
            cap = 2 * _padded(S).bit_length() + 2
            rec = torch.zeros(cap, 3, dtype=torch.float64)
            for i, (st, sz) in enumerate(_dyadic(a, b)):
                rec[i] = torch.tensor([st, sz, sumsq(_pieces(gs, segs[st:st + sz]))],
                                      dtype=torch.float64)
            got = [torch.zeros(cap, 3, dtype=torch.float64) for _ in range(world)]
            dist.all_gather(got, rec)
            entries = {(int(r[0]), int(r[1])): float(r[2]) for g in got for r in g if r[1] > 0}
            total = _assemble(entries, S)
        with open(f"{out}.{rank}", "w") as f:
            f.write(np.float64(total).tobytes().hex())
    finally:
        dist.destroy_process_group()


def _free_port():
    with socket.socket() as s:
        s.bind(("127.0.0.1", 0))
        return s.getsockname()[1]


@pytest.mark.parametrize("scheme,world", [("aligned", 2), ("aligned", 4), ("balanced", 3),
                                          ("balanced", 8)])
@pytest.mark.parametrize("nan_at", [None, (5, 100)])
def test_sharded_norm_equals_single_device_sum(tmp_path, scheme, world, nan_at):
    import multiprocessing as mp
    import oracle
    from ark_amd import _abi
    gs = _tensors(nan_at)
    want = oracle.sumsq(_host(gs), _abi.GRAD_F16, 1.0 / 1024)[0]
    out = str(tmp_path / "sum")
    ctx = mp.get_context("spawn")
    port = _free_port()
    procs = [ctx.Process(target=_worker, args=(r, world, port, nan_at, out, scheme))
             for r in range(world)]
    for p in procs:
        p.start()
    for p in procs:
        p.join(120)
    assert all(p.exitcode == 0 for p in procs), [p.exitcode for p in procs]
    for r in range(world):
        got = np.frombuffer(bytes.fromhex(open(f"{out}.{r}").read()), np.float64)[0]
        if nan_at is None:
            assert np.float64(got).tobytes() == np.float64(want).tobytes(), (r, got, want)
        else:
            assert np.isnan(got) and np.isnan(want)


def test_dyadic_blocks_tile_a_range_and_rebuild_any_tree():
    """_dyadic covers [a, b) exactly with aligned blocks, at most 2 log2 per
    range; _assemble over any split's blocks gives the pairwise tree of the
    leaves (exact small integers, so every association is checked by value
    as well as by structure through the leaf order)."""
    import random
    rnd = random.Random(3)
    for S in (1, 2, 3, 10, 57, 64, 100):
        leaves = [float(rnd.randrange(1, 1 << 20)) * 2.0 ** rnd.randrange(-30, 30)
                  for _ in range(S)]
        want = _finish(leaves + [0.0] * (_padded(S) - S))
        for world in (1, 2, 3, 5, 8):
            entries = {}
            for r in range(world):
                a, b = r * S // world, (r + 1) * S // world
                blocks = _dyadic(a, b)
                assert sum(sz for _, sz in blocks) == b - a
                assert all(st % sz == 0 for st, sz in blocks)
                assert len(blocks) <= 2 * max(1, (b - a).bit_length())
                for st, sz in blocks:
                    entries[(st, sz)] = _finish(leaves[st:st + sz])
            got = _assemble(entries, S)
            assert np.float64(got).tobytes() == np.float64(want).tobytes(), (S, world)


def test_balanced_shares_of_the_benchmark_sets():
    """ark_amd.eko.shard_tensors: the 8 shares of c2 and c4 cover every
    element once, in table order, cut only at segment boundaries, each within
    one segment of an eighth of the segment list."""
    from ark_amd.eko import SEGMENT, config_tensors, shard_tensors
    for name in ("c2", "c4"):
        full = config_tensors(name)
        segs = sum((s.n + SEGMENT - 1) // SEGMENT for s in full)
        flat, counts = [], []
        for r in range(8):
            share = shard_tensors(full, r, 8)
            counts.append(sum((s.n + SEGMENT - 1) // SEGMENT for s in share))
            for s in share:
                base, _, rng = s.name.partition("[")
                lo, hi = (map(int, rng[:-1].split(":")) if rng else
                          (0, next(f.n for f in full if f.name == base)))
                assert lo % SEGMENT == 0 and hi - lo == s.n
                flat.append((base, lo, hi))
        merged = []
        for base, lo, hi in flat:
            if merged and merged[-1][0] == base and merged[-1][2] == lo:
                merged[-1][2] = hi
            else:
                merged.append([base, lo, hi])
        assert [(b, lo, hi) for b, lo, hi in merged] == [(f.name, 0, f.n) for f in full]
        assert sum(counts) == segs and max(counts) - min(counts) <= 1
    assert [s.name for s in config_tensors("c2s8")][-1] == "l0.w2[0:1130496]"
