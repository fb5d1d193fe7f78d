"""Host-side mirror of ARK's optimizer interface over the gfx950 library.

Mirrors (paths relative to proyecto_ark/ark01/ of the reference):
  AdamConfig            src/optimizer.rs:44-66
  Optimizer.new         src/optimizer.rs:74
  Optimizer.lr_now      src/optimizer.rs:80-92
  Optimizer.step_all    src/optimizer.rs:171-228 + the AMP block of
                        src/training.rs:289-326 (one fused device step)
  Optimizer.record_overflow   src/training.rs:228-241
  Optimizer.restaurar_momentos  src/optimizer.rs:237-313
  ModelWeights / ParamSet       src/memory.rs:202-255 (device arenas)
  adam_step_zero_copy   src/optimizer.rs:27-40 (one ark_asm_adam_step_f16 call)
  adam_step             src/ffi.rs:98-101 (one ark_asm_adam_step call, fp32 w)

Device memory and streams come from torch; every optimizer computation runs
in the HIP library through its C ABI.
"""
import ctypes as C
import math
from dataclasses import dataclass

import numpy as np

from . import _abi
from ._lib import check, lib


@dataclass
class AdamConfig:
    """optimizer.rs:44-66 (defaults of AdamConfig::default)."""
    lr: float = 3e-4
    beta1: float = 0.9
    beta2: float = 0.999
    eps: float = 1e-8
    weight_decay: float = 0.01
    grad_clip: float = 1.0
    warmup_steps: int = 100


@dataclass
class AmpConfig:
    """AMP scaler constants: training.rs:10-13, config.rs:36/69, and the
    early-stop limit of training.rs:235/298."""
    loss_scale_init: float = 256.0
    loss_scale_min: float = 1.0
    loss_scale_max: float = 8192.0
    scale_up_every: int = 2000
    max_consecutive_nonfinite: int = 200


def hparams(cfg: AdamConfig, amp: AmpConfig, grad_dtype=_abi.GRAD_F16):
    hp = _abi.HParams()
    hp.beta1, hp.beta2, hp.eps = cfg.beta1, cfg.beta2, cfg.eps
    hp.grad_clip = cfg.grad_clip
    hp.loss_scale_init = amp.loss_scale_init
    hp.loss_scale_min = amp.loss_scale_min
    hp.loss_scale_max = amp.loss_scale_max
    hp.scale_up_every = amp.scale_up_every
    hp.max_consecutive_nonfinite = amp.max_consecutive_nonfinite
    hp.grad_dtype = grad_dtype
    return hp


def cos_f32(x) -> np.float32:
    """The fp32 cosine of `f32::cos` (optimizer.rs:89), taken as the
    correctly rounded result: libm's double cos, rounded once to fp32.  Over
    every argument lr_now can pass (pi * d / 800000 in fp32, d = 0..800000)
    this equals the exactly rounded cosine; the C++ mirror computes it the
    same way."""
    return np.float32(math.cos(float(np.float32(x))))


def lr_now(cfg: AdamConfig, step: int) -> float:
    """optimizer.rs:80-92 in fp32, with `step` the already-incremented
    Optimizer::step (step_all increments before calling it, :172-173)."""
    f32 = np.float32
    lr = f32(cfg.lr)
    if step < cfg.warmup_steps:
        return float(lr * (f32(step) + f32(1.0)) / f32(cfg.warmup_steps))
    decay_steps = f32(step - cfg.warmup_steps)
    progress = min(decay_steps / f32(800_000.0), f32(1.0))
    cosine = f32(0.5) * (f32(1.0) + cos_f32(f32(np.pi) * progress))
    lr_min = lr * f32(0.1)
    return float(lr_min + (lr - lr_min) * cosine)


def _single_tensor_args(w, g, m, v, w_bytes):
    import torch
    ts = (w, g, m, v)
    if not all(isinstance(t, torch.Tensor) and t.is_cuda and t.is_contiguous() for t in ts):
        raise ValueError("w, g, m and v must be contiguous device tensors")
    if len({t.device for t in ts}) != 1:
        raise ValueError("w, g, m and v must be on one device")
    if w_bytes == 4 and w.dtype != torch.float32:
        raise ValueError("w must hold float32 elements")
    if w_bytes == 2 and (w.element_size() != 2 or w.dtype == torch.bfloat16):
        raise ValueError("w must hold float16 elements (or their bits as 16-bit integers)")
    if not all(t.dtype == torch.float32 for t in (g, m, v)):
        raise ValueError("g, m and v must be float32")
    # optimizer.rs:32-33 (debug_assert_eq on the lengths)
    if not (w.numel() == g.numel() == m.numel() == v.numel()):
        raise ValueError(f"lengths differ: w {w.numel()}, g {g.numel()}, m {m.numel()}, "
                         f"v {v.numel()}")
    return (w.data_ptr(), g.data_ptr(), m.data_ptr(), v.data_ptr(), g.numel(),
            C.c_void_p(torch.cuda.current_stream(w.device).cuda_stream))


def adam_step_zero_copy(w_fp16, g, m, v, lr, beta1, beta2, eps, wd, t):
    """optimizer.rs:27-40: AdamW over one tensor, fp16 weights (or their
    16-bit bits) updated in place from fp32 g, m, v (ark_hip_adam_step_f16,
    the drop-in of ark_asm_adam_step_f16, opti.s:192-360), queued on torch's
    current stream of w's device."""
    wp, gp, mp, vp, n, st = _single_tensor_args(w_fp16, g, m, v, 2)
    check(lib().ark_hip_adam_step_f16(wp, gp, mp, vp, n, lr, beta1, beta2, eps, wd, t, st))


def adam_step(w, g, m, v, lr, beta1, beta2, eps, wd, t):
    """ffi.rs:98-101: the same over fp32 weights (ark_hip_adam_step, the
    drop-in of ark_asm_adam_step, opti.s:20-177)."""
    wp, gp, mp, vp, n, st = _single_tensor_args(w, g, m, v, 4)
    check(lib().ark_hip_adam_step(wp, gp, mp, vp, n, lr, beta1, beta2, eps, wd, t, st))


def grad_clip_global(grads, threshold, wait=True):
    """ffi.rs:206-213 (grad_clip_global, over ark_asm_grad_clip,
    opti.s:369-432): the L2 norm of the float32 GPU tensor grads and, when it
    exceeds threshold, grads scaled in place by threshold / norm
    (ark_hip_grad_clip), on torch's current stream of its device.  Returns
    the pre-clip norm (0.0 for an empty tensor, as the reference); with
    wait=False the work is only queued and None is returned."""
    import torch
    if not (grads.is_cuda and grads.is_contiguous() and grads.dtype == torch.float32):
        raise ValueError("grads must be a contiguous float32 GPU tensor")
    st = C.c_void_p(torch.cuda.current_stream(grads.device).cuda_stream)
    norm = C.c_float()
    check(lib().ark_hip_grad_clip(grads.data_ptr(), grads.numel(), threshold,
                                  C.byref(norm) if wait else None, st))
    return norm.value if wait else None


def grad_clip(grads, threshold):
    """ffi.rs:216-220: the reference's alias of grad_clip_global."""
    return grad_clip_global(grads, threshold)


class ParamSet:
    """Parameter-buffer set on one device: fp16 weights, gradients (fp16 or
    fp32, already multiplied by the loss scale), fp32 m and v.  Each array
    kind is one arena; every tensor starts on a 256-byte boundary so the
    kernels use 16-byte accesses throughout."""

    ALIGN_ELEMS = 128  # 256 B of fp16, 512 B of fp32

    def __init__(self, specs, weight_decay, device="cuda", grad_dtype=_abi.GRAD_F16,
                 no_unscale=()):
        import torch
        self.specs = list(specs)
        self.grad_dtype = grad_dtype
        self.weight_decay = float(weight_decay)
        offs, o = [], 0
        for s in self.specs:
            offs.append(o)
            o += (s.n + self.ALIGN_ELEMS - 1) // self.ALIGN_ELEMS * self.ALIGN_ELEMS
        self.total = max(o, 1)
        self.offsets = offs
        self.w_arena = torch.zeros(self.total, dtype=torch.float16, device=device)
        gdt = torch.float16 if grad_dtype == _abi.GRAD_F16 else torch.float32
        self.g_arena = torch.zeros(self.total, dtype=gdt, device=device)
        self.m_arena = torch.zeros(self.total, dtype=torch.float32, device=device)
        self.v_arena = torch.zeros(self.total, dtype=torch.float32, device=device)
        self.no_unscale = set(no_unscale)

    def __len__(self):
        return len(self.specs)

    @property
    def n_params(self):
        return sum(s.n for s in self.specs)

    def view(self, arena, i):
        o, n = self.offsets[i], self.specs[i].n
        return arena[o:o + n]

    def w(self, i): return self.view(self.w_arena, i)
    def g(self, i): return self.view(self.g_arena, i)
    def m(self, i): return self.view(self.m_arena, i)
    def v(self, i): return self.view(self.v_arena, i)

    def table(self):
        arr = (_abi.Tensor * len(self.specs))()
        for i, s in enumerate(self.specs):
            arr[i].w = self.w(i).data_ptr()
            arr[i].g = self.g(i).data_ptr()
            arr[i].m = self.m(i).data_ptr()
            arr[i].v = self.v(i).data_ptr()
            arr[i].n = s.n
            arr[i].weight_decay = self.weight_decay if s.decay else 0.0
            arr[i].flags = _abi.TENSOR_NO_UNSCALE if s.name in self.no_unscale else 0
        return arr


class Optimizer:
    """Optimizer { cfg, step } over a ParamSet, with the AMP loss scaler state
    kept on the device next to it."""

    def __init__(self, cfg: AdamConfig, params: ParamSet, amp: AmpConfig = None,
                 stream=None, table=None):
        import torch
        self.cfg = cfg
        self.amp = amp or AmpConfig()
        self.params = params
        self.hp = hparams(cfg, self.amp, params.grad_dtype if params else _abi.GRAD_F16)
        if stream is None:
            stream = torch.cuda.current_stream()
        self._stream = stream
        self._table = table if table is not None else params.table()
        h = C.c_void_p()
        check(lib().ark_opt_create(self._table, len(self._table), C.byref(self.hp),
                                   C.c_void_p(stream.cuda_stream), C.byref(h)))
        self._h = h

    @property
    def handle(self):
        """The ark_opt_handle* (for the gradient hand-off's final calls)."""
        return self._h

    # -- lifecycle ----------------------------------------------------------
    def close(self):
        if self._h:
            lib().ark_opt_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- state ----------------------------------------------------------------
    def get_state(self):
        st = _abi.State()
        check(lib().ark_opt_get_state(self._h, C.byref(st)))
        return st

    def set_state(self, **kw):
        st = self.get_state()
        for k, v in kw.items():
            setattr(st, k, v)
        check(lib().ark_opt_set_state(self._h, C.byref(st)))

    @property
    def step(self):
        """Optimizer::step (applied AdamW steps)."""
        return self.get_state().t

    @property
    def loss_scale(self):
        return self.get_state().loss_scale

    # -- the step ---------------------------------------------------------------
    def lr_now(self, step):
        return lr_now(self.cfg, step)

    def step_all(self, lr=None, info=False, schedule=False):
        """One fused step.  lr: this step's learning rate (default cfg.lr);
        schedule=True evaluates lr_now at the step number this step would
        take (waits for the device to read t).  Returns (status, StepInfo)
        when info is True, else the status without waiting."""
        if schedule:
            lr = self.lr_now(self.get_state().t + 1)
        elif lr is None:
            lr = self.cfg.lr
        if info:
            out = _abi.StepInfo()
            rc = check(lib().ark_opt_step(self._h, lr, C.byref(out)))
            return rc, out
        return check(lib().ark_opt_step(self._h, lr, None))

    def step_lr_dev(self, lr_dev, info=False):
        """One fused step whose lr the finalize kernel reads from the
        one-element float32 GPU tensor lr_dev when it runs (graph replays
        that follow a schedule).  Returns (status, StepInfo) when info is
        True, else the status without waiting."""
        import torch
        assert lr_dev.is_cuda and lr_dev.dtype == torch.float32 and lr_dev.numel() == 1
        if info:
            out = _abi.StepInfo()
            rc = check(lib().ark_opt_step_lr_dev(self._h, lr_dev.data_ptr(), C.byref(out)))
            return rc, out
        return check(lib().ark_opt_step_lr_dev(self._h, lr_dev.data_ptr(), None))

    def record_overflow(self, info=True):
        out = _abi.StepInfo()
        rc = check(lib().ark_opt_record_overflow(self._h, C.byref(out) if info else None))
        return (rc, out) if info else rc

    # -- timing -------------------------------------------------------------------
    def set_timing(self, on):
        check(lib().ark_opt_set_timing(self._h, 1 if on else 0))

    def get_timing(self):
        t = _abi.Timing()
        check(lib().ark_opt_get_timing(self._h, C.byref(t)))
        return t

    # -- checkpoint resume ----------------------------------------------------------
    def restaurar_momentos(self, momentos_m, momentos_v, adam_step):
        """optimizer.rs:237-313.  momentos_m/_v: host float32 arrays in
        checkpoint order: embed, 9 per layer (wq, wk, wv, wo, w1, w2, w3, g1,
        g2), then gamma_final when present (271 or 272 for EKO-237M).  Same
        tolerance as the reference: a count mismatch restores nothing, an
        embed or layer size mismatch stops there (what was copied stays) and
        leaves `step` unchanged, a gamma_final size mismatch is skipped.
        Returns True when the step was set."""
        import torch
        specs = self.params.specs
        names = [s.name for s in specs]
        if "embed" not in names or "gamma_final" not in names:
            raise ValueError("restaurar_momentos needs an EKO parameter set")
        layers = [i for i, s in enumerate(specs) if s.name not in ("embed", "gamma_final")]
        esperados = 1 + len(layers)
        if (len(momentos_m) not in (esperados, esperados + 1)
                or len(momentos_v) not in (esperados, esperados + 1)):
            return False

        def put(ti, k):
            mk = np.ascontiguousarray(momentos_m[k], np.float32).ravel()
            vk = np.ascontiguousarray(momentos_v[k], np.float32).ravel()
            if mk.size != specs[ti].n:
                return False
            if vk.size != specs[ti].n:  # copy_from_slice asserts (memory.rs:60)
                raise ValueError(f"momento v {k}: {vk.size} != {specs[ti].n}")
            self.params.m(ti).copy_(torch.from_numpy(mk))
            self.params.v(ti).copy_(torch.from_numpy(vk))
            return True

        if not put(names.index("embed"), 0):                       # :260-266
            return False
        if len(momentos_m) == esperados + 1:                       # :269-275
            put(names.index("gamma_final"), esperados)
        for k, ti in enumerate(layers, start=1):                   # :278-306
            if not put(ti, k):
                return False
        self.set_state(t=int(adam_step))                           # :308
        return True
