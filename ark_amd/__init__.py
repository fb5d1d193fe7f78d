"""ark_amd: the MI355X (gfx950) optimizer step of the ARK/EKO trainer --
AMP unscale with inf/NaN skip, global L2 gradient norm, global-norm clipping
and fused fp16-weight / fp32-moment AdamW -- as HIP kernels behind the C ABI
of include/ark_opt.h, with the paths on either side of it: the fp16/fp32
weight codec (codec.py, include/ark_codec.h), the checkpoint V4 state
(ckpt.py, include/ark_ckpt.h) and the gradient hand-off with the embedding
scatter (grad.py, include/ark_grad.h).  This package holds the HIP sources
(csrc/), the built library (lib/), the host-side mirror of the reference's
optimizer interface (optimizer.py, host/ark_host.hpp for C++) and the seeded
synthetic workloads (synth.py)."""
from . import _abi  # noqa: F401
from .eko import EKO_1P3B, EKO_237M, EKO_LAYER, EkoConfig, TensorSpec, config_tensors  # noqa: F401

__all__ = ["_abi", "EkoConfig", "TensorSpec", "config_tensors", "EKO_237M", "EKO_LAYER",
           "EKO_1P3B"]
