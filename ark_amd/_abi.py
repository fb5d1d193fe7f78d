"""ctypes mirror of the C ABI structs and constants in include/ark_opt.h.

Layouts are checked against the library's own sizeof values
(`ark_opt_struct_sizes`) when the library is loaded.
"""
import ctypes as C

ABI_VERSION = 1

OK = 0
EARLY_STOP = 1
EINVAL = -1
EHIP = -2
ENOMEM = -3
EIO = -4

NORM_SEGMENT = 4096

GRAD_F16 = 0
GRAD_F32 = 1

TENSOR_NO_UNSCALE = 1


class Tensor(C.Structure):
    _fields_ = [
        ("w", C.c_void_p),
        ("g", C.c_void_p),
        ("m", C.c_void_p),
        ("v", C.c_void_p),
        ("n", C.c_uint64),
        ("weight_decay", C.c_float),
        ("flags", C.c_uint32),
    ]


class HParams(C.Structure):
    _fields_ = [
        ("beta1", C.c_float),
        ("beta2", C.c_float),
        ("eps", C.c_float),
        ("grad_clip", C.c_float),
        ("loss_scale_init", C.c_float),
        ("loss_scale_min", C.c_float),
        ("loss_scale_max", C.c_float),
        ("scale_up_every", C.c_uint32),
        ("max_consecutive_nonfinite", C.c_uint32),
        ("grad_dtype", C.c_uint32),
    ]


class State(C.Structure):
    _fields_ = [
        ("t", C.c_uint32),
        ("loss_scale", C.c_float),
        ("clean_steps", C.c_uint32),
        ("consecutive_nonfinite", C.c_uint32),
        ("skipped_steps", C.c_uint64),
        ("early_stop", C.c_uint32),
        ("reserved", C.c_uint32),
    ]

    def as_dict(self):
        return {k: getattr(self, k) for k, _ in self._fields_ if k != "reserved"}


class StepInfo(C.Structure):
    _fields_ = [
        ("applied", C.c_int32),
        ("nonfinite", C.c_int32),
        ("clipped", C.c_int32),
        ("status", C.c_int32),
        ("grad_sumsq", C.c_double),
        ("grad_norm", C.c_float),
        ("clip_coef", C.c_float),
        ("inv_scale", C.c_float),
        ("lr", C.c_float),
        ("lr_eff", C.c_float),
        ("reserved", C.c_float),
        ("state", State),
    ]

    def as_dict(self):
        d = {k: getattr(self, k) for k, _ in self._fields_ if k not in ("reserved", "state")}
        d["state"] = self.state.as_dict()
        return d


class Timing(C.Structure):
    _fields_ = [
        ("steps", C.c_uint64),
        ("ms_norm", C.c_double),
        ("ms_finalize", C.c_double),
        ("ms_adamw", C.c_double),
        ("ms_step", C.c_double),
    ]


STRUCTS = (Tensor, HParams, State, StepInfo, Timing)


# include/ark_codec.h
CODEC_F16_TO_F32 = 0
CODEC_F32_TO_F16 = 1


class CodecSpan(C.Structure):
    _fields_ = [("src", C.c_void_p), ("dst", C.c_void_p), ("n", C.c_uint64)]


# include/ark_ckpt.h
CKPT_F16 = 0
CKPT_F32 = 1
CKPT_MAGIC_V2 = 0x4B325241
CKPT_MAGIC_V3 = 0x4B335241
CKPT_MAGIC_V4 = 0x4B345241
CKPT_MAGIC_AMP = 0x53504D41


class CkptRecord(C.Structure):
    _fields_ = [("data", C.c_void_p), ("n", C.c_uint64), ("dtype", C.c_uint32),
                ("reserved", C.c_uint32)]


class CkptInfo(C.Structure):
    _fields_ = [("version", C.c_uint32), ("has_moments", C.c_uint32),
                ("global_step", C.c_uint64), ("adam_step", C.c_uint64),
                ("n_tensors", C.c_uint64), ("file_bytes", C.c_uint64),
                ("has_amp", C.c_uint32), ("reserved", C.c_uint32)]


# include/ark_grad.h
class GradSpan(C.Structure):
    _fields_ = [("dst", C.c_void_p), ("src", C.c_void_p), ("n", C.c_uint64)]


# every struct whose size ark_opt_struct_sizes reports, in its order
ALL_STRUCTS = STRUCTS + (CodecSpan, CkptRecord, CkptInfo, GradSpan)
