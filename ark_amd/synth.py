"""Seeded synthetic inputs on the device (include/ark_synth.h) for torch
tensors: fp16 weights and loss-scaled fp16 gradients of the EKO shapes."""
import ctypes as C

from ._lib import check, lib


def _stream(t):
    import torch
    return C.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def normal_f16(t, seed, tensor_id, step, sigma_scale):
    """t (torch.float16, contiguous, on the GPU) <- fp16(z * sigma_scale)."""
    assert t.is_cuda and t.is_contiguous() and t.element_size() == 2
    check(lib().ark_synth_normal_f16(t.data_ptr(), t.numel(), seed, tensor_id, step,
                                     sigma_scale, _stream(t)))


def normal_f32(t, seed, tensor_id, step, sigma_scale):
    assert t.is_cuda and t.is_contiguous() and t.element_size() == 4
    check(lib().ark_synth_normal_f32(t.data_ptr(), t.numel(), seed, tensor_id, step,
                                     sigma_scale, _stream(t)))


def copy(dst, src):
    """dst <- src bytes with the library's plain streaming copy kernel."""
    nbytes = src.numel() * src.element_size()
    assert dst.is_cuda and src.is_cuda and dst.numel() * dst.element_size() == nbytes
    check(lib().ark_synth_copy(dst.data_ptr(), src.data_ptr(), nbytes, _stream(src)))


def fill_u16(t, bits):
    assert t.is_cuda and t.is_contiguous() and t.element_size() == 2
    check(lib().ark_synth_fill_u16(t.data_ptr(), t.numel(), bits, _stream(t)))
