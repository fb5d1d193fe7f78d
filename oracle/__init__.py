"""TEST INFRASTRUCTURE ONLY: ctypes binding of the CPU oracle (ark_oracle.c).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module, and only to check or time the reference arithmetic on the CPU.
The product package (ark_amd) never imports it.

The oracle restates (paths relative to proyecto_ark/ark01/ of the reference):
  asm/opti.s:192-360            ark_asm_adam_step_f16
  src/optimizer.rs:126-228      clip_all_grads + step_all
  src/training.rs:10-13,228-326 AMP loss-scale state machine
Parity pins for each function are listed in tests/test_oracle_*.py.
"""
import ctypes as C
import os
import subprocess

import numpy as np

from ark_amd import _abi

_HERE = os.path.dirname(os.path.abspath(__file__))
# ARK_ORACLE_LIB names another build of ark_oracle.c to load instead (the
# mutant builds of tests/test_oracle_mutants.py); it must exist.
LIB_PATH = os.environ.get("ARK_ORACLE_LIB") or os.path.join(_HERE, "_build", "libark_oracle.so")

_lib = None


def build(force=False):
    """Compile the oracle with its Makefile (gcc)."""
    args = ["make", "-C", _HERE]
    if force:
        args.insert(1, "-B")
    subprocess.run(args, check=True, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        build()
    L = C.CDLL(LIB_PATH)
    P = C.c_void_p
    u16p = C.POINTER(C.c_uint16)
    f32p = C.POINTER(C.c_float)
    L.ark_ref_f16_to_f32.argtypes = [C.c_uint16]
    L.ark_ref_f16_to_f32.restype = C.c_float
    L.ark_ref_f32_to_f16.argtypes = [C.c_float]
    L.ark_ref_f32_to_f16.restype = C.c_uint16
    L.ark_ref_f16_to_f32_array.argtypes = [P, P, C.c_uint64]
    L.ark_ref_f32_to_f16_array.argtypes = [P, P, C.c_uint64]
    L.ark_ref_check_f16_to_f32_f16c.restype = C.c_int64
    L.ark_ref_check_f32_to_f16_f16c.argtypes = [C.c_uint64, C.c_uint64, C.c_int]
    L.ark_ref_check_f32_to_f16_f16c.restype = C.c_int64
    L.ark_ref_compare_f32_to_f16_range.argtypes = [C.c_uint64, C.c_uint64, P, C.c_int,
                                                   C.POINTER(C.c_uint64)]
    L.ark_ref_compare_f32_to_f16_range.restype = C.c_int64
    L.ark_ref_set_vector.argtypes = [C.c_int]
    L.ark_ref_set_vector.restype = C.c_int
    L.ark_ref_grad_accumulate.argtypes = [P, P, C.c_uint64]
    L.ark_ref_grad_accumulate.restype = None
    L.ark_ref_embed_scatter.argtypes = [P, C.c_uint32, C.c_uint32, P, P, C.c_uint32]
    L.ark_ref_embed_scatter.restype = None
    L.ark_ref_pow_binary.argtypes = [C.c_float, C.c_uint32]
    L.ark_ref_pow_binary.restype = C.c_float
    L.ark_ref_prologue.argtypes = [C.c_float, C.c_float, C.c_float, C.c_float,
                                   C.c_uint32, C.POINTER(Scalars)]
    L.ark_ref_adam_step_f32.argtypes = [P, P, P, P, C.c_uint64, C.c_float, C.c_float,
                                        C.c_float, C.c_float, C.c_float, C.c_uint32]
    L.ark_ref_adam_step_f16.argtypes = [P, P, P, P, C.c_uint64, C.c_float, C.c_float,
                                        C.c_float, C.c_float, C.c_float, C.c_uint32]
    L.ark_ref_sumsq.argtypes = [C.POINTER(_abi.Tensor), C.c_int32, C.c_uint32, C.c_float,
                                C.c_int, C.POINTER(C.c_int32)]
    L.ark_ref_sumsq.restype = C.c_double
    L.ark_ref_pairwise.argtypes = [P, C.c_uint64]
    L.ark_ref_pairwise.restype = C.c_double
    L.ark_ref_state_init.argtypes = [C.POINTER(_abi.HParams), C.POINTER(_abi.State)]
    L.ark_ref_opt_step.argtypes = [C.POINTER(_abi.Tensor), C.c_int32, C.POINTER(_abi.HParams),
                                   C.POINTER(_abi.State), C.c_float, C.c_int,
                                   C.POINTER(_abi.StepInfo)]
    L.ark_ref_finalize.argtypes = [C.POINTER(_abi.HParams), C.POINTER(_abi.State), C.c_double,
                                   C.c_int, C.c_float, C.POINTER(_abi.StepInfo)]
    L.ark_ref_apply_given.argtypes = [C.POINTER(_abi.Tensor), C.c_int32, C.POINTER(_abi.HParams),
                                      C.c_uint32, C.c_float, C.POINTER(_abi.StepInfo), C.c_int]
    L.ark_ref_record_overflow.argtypes = [C.POINTER(_abi.HParams), C.POINTER(_abi.State),
                                          C.POINTER(_abi.StepInfo)]
    L.ark_ref_amp_replay.argtypes = [C.POINTER(_abi.HParams), C.POINTER(_abi.State), P,
                                     C.c_uint64, P]
    L.ark_ref_grad_clip_literal.argtypes = [P, C.c_uint64, C.c_float]
    L.ark_ref_grad_clip_literal.restype = C.c_float
    L.ark_ref_grad_clip.argtypes = [P, C.c_uint64, C.c_float, C.c_int]
    L.ark_ref_grad_clip.restype = C.c_float
    L.ark_ref_mix64.argtypes = [C.c_uint64]
    L.ark_ref_mix64.restype = C.c_uint64
    L.ark_ref_splitmix64_next.argtypes = [C.POINTER(C.c_uint64)]
    L.ark_ref_splitmix64_next.restype = C.c_uint64
    L.ark_ref_synth_base.argtypes = [C.c_uint64, C.c_uint32, C.c_uint32]
    L.ark_ref_synth_base.restype = C.c_uint64
    L.ark_ref_synth_normal_f32.argtypes = [P, C.c_uint64, C.c_uint64, C.c_uint32, C.c_uint32,
                                           C.c_float]
    L.ark_ref_synth_normal_f16.argtypes = [P, C.c_uint64, C.c_uint64, C.c_uint32, C.c_uint32,
                                           C.c_float]
    del u16p, f32p
    _lib = L
    return L


class Scalars(C.Structure):
    _fields_ = [(k, C.c_float) for k in ("decay", "bc1", "bc2", "lr_eff", "c1", "c2")]


def _ptr(a):
    return a.ctypes.data_as(C.c_void_p)


# ---- conversions -----------------------------------------------------------

def f16_to_f32(bits):
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(bits.shape, np.float32)
    lib().ark_ref_f16_to_f32_array(_ptr(bits), _ptr(out), bits.size)
    return out


def f32_to_f16(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().ark_ref_f32_to_f16_array(_ptr(x), _ptr(out), x.size)
    return out


def compare_f32_to_f16_range(lo, got, nthreads=8):
    """Mismatches of got (uint16, one per fp32 pattern lo, lo+1, ...) against
    the conversion of those patterns, and the first mismatching pattern."""
    got = np.ascontiguousarray(got, dtype=np.uint16)
    first = C.c_uint64()
    bad = lib().ark_ref_compare_f32_to_f16_range(lo, lo + got.size, _ptr(got), nthreads,
                                                 C.byref(first))
    return bad, (None if first.value == 2 ** 64 - 1 else first.value)


def set_vector(on):
    """Run the optimizer step's loops 8-wide (AVX2/F16C) -- only to time the
    CPU baseline; the checker uses the scalar restatement.  Returns the mode
    in effect."""
    return lib().ark_ref_set_vector(1 if on else 0)


def grad_accumulate(dst, src):
    """In place: dst (float32) += src (float32), i ascending."""
    assert dst.dtype == np.float32 and src.dtype == np.float32 and dst.flags.c_contiguous
    src = np.ascontiguousarray(src)
    assert dst.size == src.size
    lib().ark_ref_grad_accumulate(_ptr(dst), _ptr(src), dst.size)


def embed_scatter(embed_grad, tokens, dx0):
    """In place on embed_grad (vocab x d float32): the loop of
    objc/bridge.m:922-928 over tokens (uint32) and dx0 (batch x d float32)."""
    assert embed_grad.dtype == np.float32 and embed_grad.flags.c_contiguous
    vocab, d = embed_grad.shape
    tokens = np.ascontiguousarray(tokens, dtype=np.uint32)
    dx0 = np.ascontiguousarray(dx0, dtype=np.float32)
    assert dx0.shape == (tokens.size, d)
    lib().ark_ref_embed_scatter(_ptr(embed_grad), vocab, d, _ptr(tokens), _ptr(dx0), tokens.size)


def pow_binary(beta, t):
    return lib().ark_ref_pow_binary(beta, t)


def prologue(lr, beta1, beta2, wd, t):
    s = Scalars()
    lib().ark_ref_prologue(lr, beta1, beta2, wd, t, C.byref(s))
    return {k: getattr(s, k) for k, _ in Scalars._fields_}


def adam_step_f16(w, g, m, v, lr, beta1, beta2, eps, wd, t):
    """In place on numpy arrays: w uint16, g/m/v float32 (opti.s:192-360)."""
    for a, dt in ((w, np.uint16), (g, np.float32), (m, np.float32), (v, np.float32)):
        assert a.dtype == dt and a.flags.c_contiguous
    assert w.size == g.size == m.size == v.size
    lib().ark_ref_adam_step_f16(_ptr(w), _ptr(g), _ptr(m), _ptr(v), w.size, lr, beta1,
                                beta2, eps, wd, t)


def adam_step_f32(w, g, m, v, lr, beta1, beta2, eps, wd, t):
    """In place on float32 numpy arrays (opti.s:20-177, fp32 weights)."""
    for a in (w, g, m, v):
        assert a.dtype == np.float32 and a.flags.c_contiguous
    assert w.size == g.size == m.size == v.size
    lib().ark_ref_adam_step_f32(_ptr(w), _ptr(g), _ptr(m), _ptr(v), w.size, lr, beta1,
                                beta2, eps, wd, t)


def pairwise(x):
    x = np.ascontiguousarray(x, dtype=np.float64)
    return lib().ark_ref_pairwise(_ptr(x), x.size)


# ---- host parameter sets ----------------------------------------------------

class HostTensor:
    """One tensor's host arrays: w (uint16 fp16 bits), g (uint16 or float32),
    m, v (float32)."""

    def __init__(self, w, g, m, v, weight_decay=0.0, flags=0):
        self.w, self.g, self.m, self.v = w, g, m, v
        self.weight_decay = float(weight_decay)
        self.flags = int(flags)

    @property
    def n(self):
        return self.w.size

    def copy(self):
        return HostTensor(self.w.copy(), self.g.copy(), self.m.copy(), self.v.copy(),
                          self.weight_decay, self.flags)


def table(tensors):
    arr = (_abi.Tensor * max(1, len(tensors)))()
    for i, t in enumerate(tensors):
        assert t.w.dtype == np.uint16 and t.m.dtype == np.float32 and t.v.dtype == np.float32
        for a in (t.w, t.g, t.m, t.v):
            assert a.flags.c_contiguous and a.size == t.w.size
        arr[i].w = t.w.ctypes.data
        arr[i].g = t.g.ctypes.data
        arr[i].m = t.m.ctypes.data
        arr[i].v = t.v.ctypes.data
        arr[i].n = t.w.size
        arr[i].weight_decay = t.weight_decay
        arr[i].flags = t.flags
    return arr


def sumsq(tensors, grad_dtype, inv_scale, nthreads=1):
    tab = table(tensors)
    bad = C.c_int32(0)
    r = lib().ark_ref_sumsq(tab, len(tensors), grad_dtype, inv_scale, nthreads, C.byref(bad))
    return r, bool(bad.value)


class Optimizer:
    """Host oracle of one handle: hparams + state, stepping HostTensors in place."""

    def __init__(self, tensors, hp, nthreads=1):
        self.tensors = tensors
        self.hp = hp
        self.nthreads = nthreads
        self.state = _abi.State()
        lib().ark_ref_state_init(C.byref(hp), C.byref(self.state))
        self._tab = table(tensors)

    def step(self, lr):
        info = _abi.StepInfo()
        st = lib().ark_ref_opt_step(self._tab, len(self.tensors), C.byref(self.hp),
                                    C.byref(self.state), lr, self.nthreads, C.byref(info))
        return st, info

    def apply_given(self, lr, t, given):
        return lib().ark_ref_apply_given(self._tab, len(self.tensors), C.byref(self.hp), t, lr,
                                         C.byref(given), self.nthreads)

    def record_overflow(self):
        info = _abi.StepInfo()
        st = lib().ark_ref_record_overflow(C.byref(self.hp), C.byref(self.state), C.byref(info))
        return st, info


def finalize(hp, state, sumsq, nonfinite, lr):
    """The scalar half of a step (ark_ref_finalize): skip / clip / t /
    loss-scale decisions from a given canonical sum of squares and
    non-finite flag; `state` is updated in place.  Returns (status, info)."""
    info = _abi.StepInfo()
    st = lib().ark_ref_finalize(C.byref(hp), C.byref(state), sumsq, 1 if nonfinite else 0, lr,
                                C.byref(info))
    return st, info


def amp_replay(hp, state, events):
    """Run the oracle's AMP state machine over step outcomes (True = skip);
    returns (status, scales after each step); `state` is updated in place."""
    ev = np.ascontiguousarray(events, dtype=np.uint8)
    scales = np.empty(ev.size, np.float32)
    st = lib().ark_ref_amp_replay(C.byref(hp), C.byref(state), _ptr(ev), ev.size, _ptr(scales))
    return st, scales


def grad_clip_literal(g, threshold):
    """In place on a float32 array: ark_asm_grad_clip (opti.s:369-432)
    instruction by instruction.  Returns the pre-clip norm."""
    assert g.dtype == np.float32 and g.flags.c_contiguous
    return lib().ark_ref_grad_clip_literal(_ptr(g), g.size, threshold)


def grad_clip(g, threshold, nthreads=1):
    """In place on a float32 array: the build's clip (canonical-tree norm,
    then the reference's compare, division and multiply).  Returns the
    pre-clip norm."""
    assert g.dtype == np.float32 and g.flags.c_contiguous
    return lib().ark_ref_grad_clip(_ptr(g), g.size, threshold, nthreads)


def default_hparams():
    """The reference's defaults (AdamConfig::default, training.rs:10-13,
    config.rs:69), built here independently of the product library."""
    hp = _abi.HParams()
    hp.beta1, hp.beta2, hp.eps, hp.grad_clip = 0.9, 0.999, 1e-8, 1.0
    hp.loss_scale_init, hp.loss_scale_min, hp.loss_scale_max = 256.0, 1.0, 8192.0
    hp.scale_up_every, hp.max_consecutive_nonfinite = 2000, 200
    hp.grad_dtype = _abi.GRAD_F16
    return hp


# ---- generator ---------------------------------------------------------------

def mix64(z):
    return lib().ark_ref_mix64(z)


def splitmix64_seq(state, n):
    s = C.c_uint64(state)
    return [lib().ark_ref_splitmix64_next(C.byref(s)) for _ in range(n)]


def synth_normal_f16(n, seed, tensor_id, step, sigma_scale):
    out = np.empty(n, np.uint16)
    lib().ark_ref_synth_normal_f16(_ptr(out), n, seed, tensor_id, step, sigma_scale)
    return out


def synth_normal_f32(n, seed, tensor_id, step, sigma_scale):
    out = np.empty(n, np.float32)
    lib().ark_ref_synth_normal_f32(_ptr(out), n, seed, tensor_id, step, sigma_scale)
    return out
