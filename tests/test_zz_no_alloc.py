"""ark_grad_embed_scatter_noalloc (include/ark_grad.h) through the C ABI:
the scatter whose workspace is the library's static device array must give
exactly the bits of ark_grad_embed_scatter, the entry point that allocates,
on consecutive calls that share the array (the second smaller than the
first, so stale workspace from the first call would show), and refuse a
batch whose workspace exceeds the array before queueing anything."""
import ctypes as C

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
