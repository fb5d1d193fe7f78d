"""ark_amd: the MI355X (gfx950) optimizer step of the ARK/EKO trainer --
AMP unscale with inf/NaN skip, global L2 gradient norm, global-norm clipping
and fused fp16-weight / fp32-moment AdamW -- as HIP kernels behind the C ABI
of include/ark_opt.h.  This package holds the HIP sources (csrc/), the built
library (lib/) and the host-side mirror of the reference's optimizer
interface (optimizer.py)."""
from . import _abi  # noqa: F401
from .eko import EKO_1P3B, EKO_237M, EKO_LAYER, EkoConfig, TensorSpec, config_tensors  # noqa: F401

__all__ = ["_abi", "EkoConfig", "TensorSpec", "config_tensors", "EKO_237M", "EKO_LAYER",
           "EKO_1P3B"]
