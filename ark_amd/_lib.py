"""Loader of the gfx950 library ark_amd/lib/libark_opt.so (the C ABI declared
in include/*.h).

There is no fallback: if the library is missing or fails to load, every
caller gets an ImportError-like failure with the reason.
"""
import ctypes as C
import os

from . import _abi

_HERE = os.path.dirname(os.path.abspath(__file__))
# ARK_OPT_LIB names another build of the same library (the sanitizer build
# the CPU tests load); by default the in-tree one.
LIB_PATH = os.environ.get("ARK_OPT_LIB") or os.path.join(_HERE, "lib", "libark_opt.so")
CSRC = os.path.join(_HERE, "csrc")
INCLUDE = os.path.join(os.path.dirname(_HERE), "include")

_lib = None


class ArkOptError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"ark_opt error {code}: {msg}")
        self.code = code


def _declare(L):
    P = C.c_void_p
    u64, u32, i32, f32 = C.c_uint64, C.c_uint32, C.c_int32, C.c_float
    H = C.c_void_p  # opaque handle
    sig = {
        "ark_opt_abi_version": ([], C.c_int),
        "ark_opt_last_error": ([], C.c_char_p),
        "ark_opt_struct_sizes": ([C.POINTER(C.c_size_t), C.c_int], C.c_int),
        "ark_opt_default_hparams": ([C.POINTER(_abi.HParams)], C.c_int),
        "ark_opt_create": ([C.POINTER(_abi.Tensor), i32, C.POINTER(_abi.HParams), P,
                            C.POINTER(H)], C.c_int),
        "ark_opt_destroy": ([H], C.c_int),
        "ark_opt_step": ([H, f32, C.POINTER(_abi.StepInfo)], C.c_int),
        "ark_opt_step_lr_dev": ([H, P, C.POINTER(_abi.StepInfo)], C.c_int),
        "ark_opt_record_overflow": ([H, C.POINTER(_abi.StepInfo)], C.c_int),
        "ark_opt_get_state": ([H, C.POINTER(_abi.State)], C.c_int),
        "ark_opt_set_state": ([H, C.POINTER(_abi.State)], C.c_int),
        "ark_opt_set_timing": ([H, C.c_int], C.c_int),
        "ark_opt_get_timing": ([H, C.POINTER(_abi.Timing)], C.c_int),
        "ark_hip_adam_step_f16": ([P, P, P, P, u64, f32, f32, f32, f32, f32, u32, P], C.c_int),
        "ark_hip_adam_step": ([P, P, P, P, u64, f32, f32, f32, f32, f32, u32, P], C.c_int),
        "ark_hip_grad_clip": ([P, u64, f32, C.POINTER(f32), P], C.c_int),
        "ark_synth_normal_f16": ([P, u64, u64, u32, u32, f32, P], C.c_int),
        "ark_synth_normal_f32": ([P, u64, u64, u32, u32, f32, P], C.c_int),
        "ark_synth_fill_u16": ([P, u64, C.c_uint16, P], C.c_int),
        "ark_synth_copy": ([P, P, u64, P], C.c_int),
        "ark_synth_stream_mix": ([P, P, P, P, u64, u32, u32, P], C.c_int),
        "ark_hip_dequant_f16_to_f32": ([P, P, u64, P], C.c_int),
        "ark_hip_quant_f32_to_f16": ([P, P, u64, P], C.c_int),
        "ark_codec_plan_create": ([C.POINTER(_abi.CodecSpan), i32, u32, P, C.POINTER(H)],
                                  C.c_int),
        "ark_codec_plan_run": ([H], C.c_int),
        "ark_codec_plan_destroy": ([H], C.c_int),
        "ark_ckpt_save_v4": ([C.c_char_p, u64, u64, C.POINTER(_abi.CkptRecord), i32,
                              C.POINTER(_abi.State), P], C.c_int),
        "ark_ckpt_probe": ([C.c_char_p, C.POINTER(_abi.CkptInfo), C.POINTER(u64),
                            C.POINTER(u32), i32], C.c_int),
        "ark_ckpt_load": ([C.c_char_p, C.POINTER(_abi.CkptRecord), i32,
                           C.POINTER(_abi.CkptInfo), C.POINTER(_abi.State), P], C.c_int),
        "ark_ckpt_v4_image_bytes": ([C.POINTER(_abi.CkptRecord), i32, C.c_int, C.POINTER(u64)],
                                    C.c_int),
        "ark_ckpt_v4_pack": ([C.POINTER(_abi.CkptRecord), i32, u64, u64, C.POINTER(_abi.State),
                              P, u64, P], C.c_int),
        "ark_ckpt_v4_unpack": ([P, u64, C.POINTER(_abi.CkptRecord), i32, C.POINTER(u32), P],
                               C.c_int),
        "ark_ckpt_v4_pack_plan_create": ([C.POINTER(_abi.CkptRecord), i32, C.c_int, P, u64, P,
                                          C.POINTER(H)], C.c_int),
        "ark_ckpt_v4_pack_plan_run": ([H, u64, u64, C.POINTER(_abi.State)], C.c_int),
        "ark_ckpt_plan_destroy": ([H], C.c_int),
        "ark_grad_accumulate": ([P, P, u64, P], C.c_int),
        "ark_grad_plan_create": ([C.POINTER(_abi.GradSpan), i32, P, C.POINTER(H)], C.c_int),
        "ark_grad_plan_run": ([H], C.c_int),
        "ark_grad_plan_destroy": ([H], C.c_int),
        "ark_grad_embed_scatter": ([P, u32, u32, P, P, u32, P], C.c_int),
        "ark_grad_embed_scatter_noalloc": ([P, u32, u32, P, P, u32, P], C.c_int),
        "ark_grad_plan_run_final": ([H, H], C.c_int),
        "ark_grad_embed_scatter_final": ([P, u32, u32, P, P, u32, H], C.c_int),
    }
    for name, (args, res) in sig.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = res
    return sig


def lib():
    """The loaded library (raises if it is not built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is not built; run __graft_entry__.build() (hipcc, gfx950)")
    # torch's wheel carries its own HIP runtime (soname libamdhip64.so.7).  Loading
    # it first makes this library's libamdhip64.so.7 dependency bind to that same
    # runtime, so torch's device pointers and streams are valid here; the other
    # order would put two HIP runtimes in the process.
    import torch  # noqa: F401
    L = C.CDLL(LIB_PATH)
    _declare(L)
    if L.ark_opt_abi_version() != _abi.ABI_VERSION:
        raise ImportError("libark_opt ABI version mismatch")
    k = len(_abi.ALL_STRUCTS)
    sizes = (C.c_size_t * k)()
    if L.ark_opt_struct_sizes(sizes, k) != k:
        raise ImportError("libark_opt reports fewer struct sizes than the bindings know")
    for s, st in zip(sizes, _abi.ALL_STRUCTS):
        if s != C.sizeof(st):
            raise ImportError(f"struct {st.__name__}: C size {s} != ctypes size {C.sizeof(st)}")
    _lib = L
    return L


def check(rc):
    """Raise ArkOptError for a negative status; return the status otherwise."""
    if rc < 0:
        raise ArkOptError(rc, lib().ark_opt_last_error().decode())
    return rc


def current_stream(t=None):
    """torch's current HIP stream (of t's device when t is given), as the
    void* the C ABI takes."""
    import torch
    s = torch.cuda.current_stream(t.device) if t is not None else torch.cuda.current_stream()
    return C.c_void_p(s.cuda_stream)


def exported_symbols():
    """Function names declared in include/*.h (every one must be exported)."""
    import re
    names = []
    for h in sorted(os.listdir(INCLUDE)):
        if not h.endswith(".h"):
            continue
        text = open(os.path.join(INCLUDE, h)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names += re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(ark_\w+)\s*\(", text, flags=re.M)
    return names
