"""ark_grad_embed_scatter_noalloc (include/ark_grad.h) through the C ABI:
the scatter whose workspace is the library's static device array must give
exactly the bits of ark_grad_embed_scatter, the entry point that allocates,
on consecutive calls that share the array (the second smaller than the
first, so stale workspace from the first call would show), on calls queued
back to back on two streams and from two host threads (the library orders
them on the array), and in a HIP graph whose capture holds the first call
of a fresh process; it must refuse a batch whose workspace exceeds the
array, and a first use under capture before the device is set up, before
queueing anything."""
import ctypes as C
import os
import subprocess
import sys
import threading

import numpy as np
import pytest

from ark_amd import _abi
from ark_amd._lib import lib

pytestmark = pytest.mark.gpu


def _torch():
    import torch
    assert torch.cuda.is_available(), "GPU test run without a GPU"
    return torch


def _case(torch, rng, vocab, d, n):
    tokens = ((rng.zipf(1.2, n) - 1) % (vocab + 7)).astype(np.uint32)
    dx0 = (rng.standard_normal((n, d)) * 10.0 ** rng.integers(-5, 3, (n, 1))).astype(np.float32)
    g0 = rng.standard_normal((vocab, d)).astype(np.float32)
    return (torch.from_numpy(tokens.view(np.int32)).cuda(), torch.from_numpy(dx0).cuda(),
            torch.from_numpy(g0).cuda())


def _call(fn, g, tokens, dx0, stream):
    vocab, d = g.shape
    return fn(g.data_ptr(), vocab, d, tokens.data_ptr(), dx0.data_ptr(), tokens.numel(),
              C.c_void_p(stream))


@pytest.mark.parametrize("sizes", [[(32000, 768, 4096), (32000, 768, 1000)],
                                   [(32000, 512, 20000), (5000, 64, 4097)],
                                   [(32000, 2048, 4096), (300, 96, 700)]])
def test_noalloc_scatter_matches_the_allocating_one(sizes):
    torch = _torch()
    L = lib()
    rng = np.random.default_rng(sum(v * 7 + d * 3 + n for v, d, n in sizes))
    stream = torch.cuda.current_stream().cuda_stream
    for vocab, d, n in sizes:
        tokens, dx0, g0 = _case(torch, rng, vocab, d, n)
        want = g0.clone()
        got = g0.clone()
        assert _call(L.ark_grad_embed_scatter, want, tokens, dx0, stream) == 0
        rc = _call(L.ark_grad_embed_scatter_noalloc, got, tokens, dx0, stream)
        assert rc == 0, L.ark_opt_last_error().decode()
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int32), want.view(torch.int32)), (vocab, d, n)
        assert not torch.equal(got, g0)


def test_noalloc_scatter_rejects_a_batch_beyond_the_scratch():
    torch = _torch()
    L = lib()
    vocab, d, n = 100, 4096, 4096  # 64 MiB of row copies > 48 MiB
    g = torch.zeros(vocab, d, device="cuda")
    dx0 = torch.ones(n, d, device="cuda")
    tokens = torch.zeros(n, dtype=torch.int32, device="cuda")
    rc = _call(L.ark_grad_embed_scatter_noalloc, g, tokens, dx0,
               torch.cuda.current_stream().cuda_stream)
    assert rc == _abi.EINVAL
    assert "static scratch" in L.ark_opt_last_error().decode()
    torch.cuda.synchronize()
    assert torch.count_nonzero(g).item() == 0


def _pairs(torch, rng, shapes):
    """Inputs and the allocating scatter's result for each (vocab, d, n)."""
    L = lib()
    out = []
    stream = torch.cuda.current_stream().cuda_stream
    for vocab, d, n in shapes:
        tokens, dx0, g0 = _case(torch, rng, vocab, d, n)
        want = g0.clone()
        assert _call(L.ark_grad_embed_scatter, want, tokens, dx0, stream) == 0
        out.append((tokens, dx0, g0, want))
    torch.cuda.synchronize()
    return out


# two batches past 4096 tokens (the multi-launch radix sort) whose workspaces
# fit the 48 MiB array
_SHAPES = [(32000, 768, 12000), (32000, 512, 16384)]


def test_calls_on_two_streams_take_the_array_in_turn():
    """Two different batches queued back to back on two streams, with no
    host wait between them, three times over: each result is the allocating
    call's, bit for bit."""
    torch = _torch()
    L = lib()
    rng = np.random.default_rng(71)
    cases = _pairs(torch, rng, _SHAPES)
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for rep in range(3):
        gots = [g0.clone() for _, _, g0, _ in cases]
        torch.cuda.synchronize()
        for (tokens, dx0, _, _), got, st in zip(cases, gots, streams):
            rc = _call(L.ark_grad_embed_scatter_noalloc, got, tokens, dx0, st.cuda_stream)
            assert rc == 0, L.ark_opt_last_error().decode()
        torch.cuda.synchronize()
        for k, ((_, _, _, want), got) in enumerate(zip(cases, gots)):
            assert torch.equal(got.view(torch.int32), want.view(torch.int32)), (rep, k)


def test_calls_from_two_host_threads_take_the_array_in_turn():
    """Two host threads, each with its own stream, each queueing four calls
    into buffers of its own: every result is the allocating call's."""
    torch = _torch()
    L = lib()
    rng = np.random.default_rng(72)
    cases = _pairs(torch, rng, _SHAPES)
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    gots = [[g0.clone() for _ in range(4)] for _, _, g0, _ in cases]
    torch.cuda.synchronize()
    codes = [[], []]

    def run(k):
        tokens, dx0, _, _ = cases[k]
        for got in gots[k]:
            codes[k].append(_call(L.ark_grad_embed_scatter_noalloc, got, tokens, dx0,
                                  streams[k].cuda_stream))

    threads = [threading.Thread(target=run, args=(k,)) for k in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    torch.cuda.synchronize()
    assert codes == [[0] * 4, [0] * 4], codes
    for k, (_, _, _, want) in enumerate(cases):
        for j, got in enumerate(gots[k]):
            assert torch.equal(got.view(torch.int32), want.view(torch.int32)), (k, j)


_CHILD = r"""
import ctypes as C, sys
import numpy as np
import torch
sys.path.insert(0, sys.argv[1])
from ark_amd import _abi, grad
from ark_amd._lib import lib
L = lib()
mode = sys.argv[2]
torch.cuda.set_device(0)
vocab, d, n = 32000, 768, 4096
rng = np.random.default_rng(5)
tokens = torch.zeros(n, dtype=torch.int32, device="cuda")
dx0 = torch.zeros(n, d, device="cuda")
g = torch.zeros(vocab, d, device="cuda")
def refill():
    tokens.copy_(torch.from_numpy(((rng.zipf(1.2, n) - 1) % vocab).astype(np.int32)))
    dx0.copy_(torch.from_numpy(rng.standard_normal((n, d)).astype(np.float32)))
    g.copy_(torch.from_numpy(rng.standard_normal((vocab, d)).astype(np.float32)))
def call(fn, out, stream):
    return fn(out.data_ptr(), vocab, d, tokens.data_ptr(), dx0.data_ptr(), n, C.c_void_p(stream))
s = torch.cuda.Stream()
refill()
torch.cuda.synchronize()
if mode == "set_up_first":
    # a gradient plan is one of the library's set-up calls for this device
    keep = torch.zeros(8, device="cuda")
    plan = grad.GradPlan([(keep, torch.ones(8, device="cuda"))])
graph = torch.cuda.CUDAGraph()
rc = []
with torch.cuda.graph(graph, stream=s):
    rc.append(call(L.ark_grad_embed_scatter_noalloc, g, s.cuda_stream))
    g.mul_(1.0)
msg = L.ark_opt_last_error().decode()
torch.cuda.synchronize()
if mode == "fresh":
    # refused before anything was queued; the capture itself completed
    assert rc == [_abi.EINVAL], rc
    assert "not set up yet" in msg, msg
    print("refused ok", flush=True)
    sys.exit(0)
assert rc == [0], (rc, msg)
for k in range(4):
    with torch.cuda.stream(s):
        refill()
        want = g.clone()
        # eager work between replays: the allocating scatter, and an eager
        # no-allocation call on another buffer, on the replay's stream
        assert call(L.ark_grad_embed_scatter, want, s.cuda_stream) == 0
        other = g.clone()
        assert call(L.ark_grad_embed_scatter_noalloc, other, s.cuda_stream) == 0
        graph.replay()
    s.synchronize()
    assert torch.equal(g.view(torch.int32), want.view(torch.int32)), k
    assert torch.equal(other.view(torch.int32), want.view(torch.int32)), k
print("replays ok", flush=True)
"""


@pytest.mark.parametrize("mode", ["fresh", "set_up_first"])
def test_first_call_of_a_process_under_graph_capture(mode):
    """In a fresh process: a first no-allocation call under capture on a
    device the library has not set up is refused (ARK_OPT_EINVAL, nothing
    queued, the capture still completes); after a set-up call (a gradient
    plan) the first call may be captured, and four replays, each after new
    inputs and eager work on the same stream, equal the allocating scatter
    bit for bit."""
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", _CHILD, root, mode], cwd=root,
                       stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=300)
    assert r.returncode == 0, r.stdout[-3000:]
    assert ("refused ok" if mode == "fresh" else "replays ok") in r.stdout
