"""The gradient hand-off (include/ark_grad.h) for torch tensors: the device
form of the CPU loops at the end of ark_mps_backward
(proyecto_ark/ark01/objc/bridge.m:902-948).

``accumulate(dst, src)`` is one ``dst += src`` loop; ``GradPlan`` runs all of a
model's in one launch; ``embed_scatter`` is the token scatter-add of
bridge.m:922-928 with the loop's exact summation order.
"""
import ctypes as C

from . import _abi
from ._lib import check, lib, current_stream as _stream


def _f32(t):
    import torch
    assert t.is_cuda and t.is_contiguous() and t.dtype == torch.float32, (t.dtype, t.shape)
    return t


def accumulate(dst, src):
    """dst += src (float32 GPU tensors of equal size)."""
    _f32(dst), _f32(src)
    assert dst.numel() == src.numel()
    check(lib().ark_grad_accumulate(dst.data_ptr(), src.data_ptr(), dst.numel(), _stream()))


class GradPlan:
    """One launch doing dst += src for every (dst, src) pair.  No dst may
    share memory with another pair's dst or src (the library refuses such
    pairs); sources may be shared.  The tensors must outlive the plan."""

    def __init__(self, pairs, stream=None):
        import torch
        spans = (_abi.GradSpan * max(1, len(pairs)))()
        for i, (d, s) in enumerate(pairs):
            _f32(d), _f32(s)
            assert d.numel() == s.numel()
            spans[i] = _abi.GradSpan(d.data_ptr(), s.data_ptr(), d.numel())
        self._keep = list(pairs)
        stream = stream or torch.cuda.current_stream()
        h = C.c_void_p()
        check(lib().ark_grad_plan_create(spans, len(pairs), C.c_void_p(stream.cuda_stream),
                                         C.byref(h)))
        self._h = h

    def run(self, final_for=None):
        """dst += src for every pair.  final_for: an Optimizer (fp32
        gradients) whose next step this is the last accumulation for; the
        launch also writes that step's norm units, so the step does not
        read the gradients again."""
        if final_for is None:
            check(lib().ark_grad_plan_run(self._h))
        else:
            check(lib().ark_grad_plan_run_final(self._h, final_for.handle))

    def close(self):
        if self._h:
            check(lib().ark_grad_plan_destroy(self._h))
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def embed_scatter(embed_grad, tokens, dx0, noalloc=False, final_for=None):
    """embed_grad (vocab x d float32) += rows of dx0 (batch x d float32) at
    the rows of tokens (int32/uint32, batch); tokens >= vocab go to row 0.
    noalloc: use the entry point whose workspace is the library's static
    device array instead of the stream-ordered pool.  final_for: the
    Optimizer whose GradPlan.run(final_for=...) came just before; the scatter
    runs on its stream and keeps its norm units current."""
    _f32(embed_grad), _f32(dx0)
    assert tokens.is_cuda and tokens.is_contiguous() and tokens.element_size() == 4
    vocab, d = embed_grad.shape
    assert dx0.shape == (tokens.numel(), d)
    args = (embed_grad.data_ptr(), vocab, d, tokens.data_ptr(), dx0.data_ptr(), tokens.numel())
    if final_for is not None:
        assert not noalloc
        check(lib().ark_grad_embed_scatter_final(*args, final_for.handle))
        return
    fn = lib().ark_grad_embed_scatter_noalloc if noalloc else lib().ark_grad_embed_scatter
    check(fn(*args, _stream()))
