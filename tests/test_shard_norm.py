"""The norm's sharding across GPUs (designed, not built: one GPU here).
Giving each rank an aligned power-of-two block of the global 4096-element
segment list makes its partial sum of squares a subtree of the canonical
tree.  One all-gather of one double per rank, then the same pairwise finish
on every rank, reproduces the single-device sum bit for bit, and a
non-finite gradient on any rank turns every rank's sum into NaN.  Checked
here with the CPU oracle standing in for each rank's norm pass, on 2 and 4
gloo ranks (one process each, 127.0.0.1)."""
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


def _rank_pieces(gs, rank, world):
    """The gradient pieces of rank's aligned block of segments: whole
    segments of each tensor, cut only at segment boundaries."""
    segs = [(t, k) for t, g in enumerate(gs) for k in range((g.size + SEG - 1) // SEG)]
    padded = 1
    while padded < max(len(segs), world):
        padded *= 2
    per = padded // world
    mine = segs[rank * per:(rank + 1) * per]
    pieces = []
    for t, k in mine:
        lo, hi = k * SEG, min((k + 1) * SEG, gs[t].size)
        if pieces and pieces[-1][0] == t and pieces[-1][2] == lo:
            pieces[-1][2] = hi
        else:
            pieces.append([t, lo, hi])
    return [np.ascontiguousarray(gs[t][lo:hi]) for t, lo, hi in pieces]


def _finish(parts):
    """The pairwise tree over the ranks' partials (len a power of two)."""
    parts = list(parts)
    while len(parts) > 1:
        parts = [parts[i] + parts[i + 1] for i in range(0, len(parts), 2)]
    return parts[0]


def _worker(rank, world, port, nan_at, out):
    import torch
    import torch.distributed as dist
    import oracle
    from ark_amd import _abi
    dist.init_process_group("gloo", init_method=f"tcp://127.0.0.1:{port}", rank=rank,
                            world_size=world)
    try:
        gs = _tensors(nan_at)
        pieces = _rank_pieces(gs, rank, world)
        part = oracle.sumsq(_host(pieces), _abi.GRAD_F16, 1.0 / 1024)[0] if pieces else 0.0
        got = [torch.zeros(1, dtype=torch.float64) for _ in range(world)]
        dist.all_gather(got, torch.tensor([part], dtype=torch.float64))
        total = _finish(float(x.item()) for x in got)
        with open(f"{out}.{rank}", "w") as f:
            f.write(np.float64(total).tobytes().hex())
    finally:
        dist.destroy_process_group()


def _free_port():
    with socket.socket() as s:
        s.bind(("127.0.0.1", 0))
        return s.getsockname()[1]


@pytest.mark.parametrize("world", [2, 4])
@pytest.mark.parametrize("nan_at", [None, (5, 100)])
def test_sharded_norm_equals_single_device_sum(tmp_path, world, nan_at):
    import multiprocessing as mp
    import oracle
    from ark_amd import _abi
    gs = _tensors(nan_at)
    want = oracle.sumsq(_host(gs), _abi.GRAD_F16, 1.0 / 1024)[0]
    out = str(tmp_path / "sum")
    ctx = mp.get_context("spawn")
    port = _free_port()
    procs = [ctx.Process(target=_worker, args=(r, world, port, nan_at, out)) for r in range(world)]
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
