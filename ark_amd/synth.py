"""Seeded synthetic inputs on the device (include/ark_synth.h) for torch
tensors: fp16 weights and loss-scaled fp16 gradients of the EKO shapes, and
the parameter sets built from them (the benchmark configurations' workloads).

Streams of the generator: weights use (tensor_id = i, step = WEIGHT_STEP);
gradients of step k use (tensor_id = i, step = k).  The CPU oracle builds the
same inputs from the same counter-based generator, so both sides start from
identical bits.
"""

import numpy as np

from . import _abi
from ._lib import check, lib, current_stream as _stream

WEIGHT_STEP = 0xFFFFFFFF
W_SIGMA = 0.02   # weights ~ N(0, 0.02)
F16_ONE = 0x3C00  # RMSNorm gains start at 1.0


def grad_sigma_scale(sigma, loss_scale):
    """sigma * loss_scale rounded to fp32 (the generator's scale)."""
    return float(np.float32(np.float32(sigma) * np.float32(loss_scale)))


def log_uniform_sigmas(n, seed, lo=-5.0, hi=-2.0):
    """Per-tensor sigma = 10^U(lo, hi), drawn on the host (configuration c2)."""
    rng = np.random.default_rng(seed)
    return [float(np.float32(10.0 ** rng.uniform(lo, hi))) for _ in range(n)]


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


def stream_mix(w, g, m, v, spacing, blocks_per_cu=0):
    """The AdamW pass's accesses without its arithmetic (ark_synth_stream_mix):
    w, g 16-bit and m, v fp32 tensors of n elements (n a multiple of 256);
    w, m and v are written back unchanged.  blocks_per_cu: resident blocks
    per CU (0: every wave slot)."""
    n = w.numel()
    assert all(t.is_cuda and t.is_contiguous() and t.numel() == n for t in (w, g, m, v))
    assert w.element_size() == g.element_size() == 2 and m.element_size() == v.element_size() == 4
    check(lib().ark_synth_stream_mix(w.data_ptr(), g.data_ptr(), m.data_ptr(), v.data_ptr(), n,
                                     spacing, blocks_per_cu, _stream(w)))


def fill_u16(t, bits):
    assert t.is_cuda and t.is_contiguous() and t.element_size() == 2
    check(lib().ark_synth_fill_u16(t.data_ptr(), t.numel(), bits, _stream(t)))


def problem(specs, seed, weight_decay, sigmas, loss_scale, step=0, grad_dtype=_abi.GRAD_F16,
            no_unscale=(), device="cuda"):
    """A ParamSet of `specs` on the device: fp16 weights N(0, W_SIGMA) (gains
    1.0), gradients N(0, sigma_i) * loss_scale of step `step`, m = v = 0."""
    from .optimizer import ParamSet
    ps = ParamSet(specs, weight_decay, device=device, grad_dtype=grad_dtype,
                  no_unscale=no_unscale)
    for i, s in enumerate(specs):
        if s.gain:
            fill_u16(ps.w(i), F16_ONE)
        else:
            normal_f16(ps.w(i), seed, i, WEIGHT_STEP, W_SIGMA)
    regen_grads(ps, seed, sigmas, loss_scale, step)
    return ps


def regen_grads(ps, seed, sigmas, loss_scale, step):
    """The gradients of step `step` into every tensor of the ParamSet."""
    for i in range(len(ps)):
        ss = grad_sigma_scale(sigmas[i], loss_scale)
        if ps.grad_dtype == _abi.GRAD_F16:
            normal_f16(ps.g(i), seed, i, step, ss)
        else:
            normal_f32(ps.g(i), seed, i, step, ss)
