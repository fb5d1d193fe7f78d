"""fp16 <-> fp32 weight codec (include/ark_codec.h) for torch tensors.

The host mirror of the reference's conversion calls: ``dequant_f16_to_f32``
and ``quant_f32_to_f16`` take the arguments of ark_dequant_f16_to_f32 /
ark_quant_f32_to_f16 (proyecto_ark/ark01/src/ffi.rs:87-92) as tensors, and
``CodecPlan`` is the one-launch form of their per-tensor loops
(src/training.rs:162-186, src/memory.rs:347-377).
"""
import ctypes as C

from . import _abi
from ._lib import check, lib, current_stream as _stream


def _flat(t, size):
    assert t.is_cuda and t.is_contiguous() and t.element_size() == size, (t.dtype, t.shape)
    return t


def dequant_f16_to_f32(src, dst):
    """dst (float32) <- src (float16 or int16/uint16 bits), element for element."""
    _flat(src, 2), _flat(dst, 4)
    assert src.numel() == dst.numel()
    check(lib().ark_hip_dequant_f16_to_f32(src.data_ptr(), dst.data_ptr(), src.numel(),
                                           _stream(src)))


def quant_f32_to_f16(src, dst):
    """dst (float16 or 16-bit bits) <- src (float32), round to nearest even."""
    _flat(src, 4), _flat(dst, 2)
    assert src.numel() == dst.numel()
    check(lib().ark_hip_quant_f32_to_f16(src.data_ptr(), dst.data_ptr(), src.numel(),
                                         _stream(src)))


class CodecPlan:
    """One launch converting every (src, dst) pair; direction is
    ``"f16_to_f32"`` or ``"f32_to_f16"``.  No dst may share memory with
    another pair's dst or src (the library refuses such pairs); sources may
    be shared.  The tensors must outlive the plan."""

    def __init__(self, pairs, direction, stream=None):
        import torch
        d = {"f16_to_f32": _abi.CODEC_F16_TO_F32, "f32_to_f16": _abi.CODEC_F32_TO_F16}[direction]
        ss, ds = (2, 4) if d == _abi.CODEC_F16_TO_F32 else (4, 2)
        spans = (_abi.CodecSpan * max(1, len(pairs)))()
        for i, (s, t) in enumerate(pairs):
            _flat(s, ss), _flat(t, ds)
            assert s.numel() == t.numel()
            spans[i] = _abi.CodecSpan(s.data_ptr(), t.data_ptr(), s.numel())
        self._keep = list(pairs)
        if stream is None:
            stream = torch.cuda.current_stream()
        self._stream = stream
        h = C.c_void_p()
        check(lib().ark_codec_plan_create(spans, len(pairs), d, C.c_void_p(stream.cuda_stream),
                                          C.byref(h)))
        self._h = h

    def run(self):
        check(lib().ark_codec_plan_run(self._h))

    def close(self):
        if self._h:
            check(lib().ark_codec_plan_destroy(self._h))
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
