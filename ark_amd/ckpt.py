"""ARK checkpoints (include/ark_ckpt.h) written from and read into
device-resident optimizer buffers.

``CheckpointV3.save_fp16`` takes the arguments of the reference's
CheckpointV3::save_fp16 (proyecto_ark/ark01/src/io.rs:432-446) as torch
tensors on the GPU and writes the same V4 file byte for byte;
``CheckpointV3.load`` is CheckpointV3::load (io.rs:504-671) into device
buffers given in file order.  ``save_params`` / ``load_params`` do the same
for a ParamSet and its Optimizer, in the tensor order of
Trainer::guardar_checkpoint (training.rs:536-604), with the loss-scaler
state carried in the trailer the reference's loader skips.  ``PackPlan``
repeats the device half of a save (the V4 image in device memory) with the
tables uploaded once and no host wait per save.
"""
import ctypes as C
import os
from dataclasses import dataclass

from . import _abi
from ._lib import check, lib, current_stream as _stream


class Records:
    """The ark_ckpt_record table of a list of tensors (file order), built
    once: fp16-sized elements -> ARK_CKPT_F16, fp32-sized -> ARK_CKPT_F32.
    Keeps the tensors alive."""

    def __init__(self, tensors):
        self.tensors = list(tensors)
        self.arr = (_abi.CkptRecord * max(1, len(self.tensors)))()
        for i, t in enumerate(self.tensors):
            assert t.is_cuda and t.is_contiguous(), f"record {i}: contiguous GPU tensor expected"
            es = t.element_size()
            assert es in (2, 4), f"record {i}: 2- or 4-byte elements expected"
            self.arr[i] = _abi.CkptRecord(t.data_ptr(), t.numel(),
                                          _abi.CKPT_F16 if es == 2 else _abi.CKPT_F32, 0)
        self.types = (C.c_uint32 * max(1, len(self.tensors)))(
            *[self.arr[i].dtype for i in range(len(self.tensors))])

    def __len__(self):
        return len(self.tensors)


def _records(tensors):
    return tensors if isinstance(tensors, Records) else Records(tensors)


@dataclass
class CkptInfo:
    version: int
    has_moments: bool
    global_step: int
    adam_step: int
    n_tensors: int
    file_bytes: int
    has_amp: bool


def _info(ci):
    return CkptInfo(ci.version, bool(ci.has_moments), ci.global_step, ci.adam_step,
                    ci.n_tensors, ci.file_bytes, bool(ci.has_amp))


def probe(path):
    """(CkptInfo, [(n, type)]) of a checkpoint file without reading its data."""
    ci = _abi.CkptInfo()
    check(lib().ark_ckpt_probe(os.fsencode(path), C.byref(ci), None, None, 0))
    k = ci.n_tensors
    ns = (C.c_uint64 * max(1, k))()
    ts = (C.c_uint32 * max(1, k))()
    check(lib().ark_ckpt_probe(os.fsencode(path), C.byref(ci), ns, ts, k))
    return _info(ci), [(ns[i], ts[i]) for i in range(k)]


def save(path, tensors, global_step, adam_step, amp_state=None):
    """Write the V4 file of `tensors` (file order; fp16 -> type 0, fp32 -> 1)."""
    recs = _records(tensors)
    amp = C.byref(amp_state) if amp_state is not None else None
    check(lib().ark_ckpt_save_v4(os.fsencode(path), global_step, adam_step, recs.arr, len(recs),
                                 amp, _stream()))


def load(path, tensors):
    """Fill `tensors` (file order, element counts as in the file) from a V2,
    V3 or V4 file; returns (CkptInfo, ark_opt_state or None)."""
    recs = _records(tensors)
    ci, st = _abi.CkptInfo(), _abi.State()
    check(lib().ark_ckpt_load(os.fsencode(path), recs.arr, len(recs), C.byref(ci), C.byref(st),
                              _stream()))
    info = _info(ci)
    return info, (st if info.has_amp else None)


def image_bytes(tensors, with_amp=False):
    out = C.c_uint64()
    recs = _records(tensors)
    check(lib().ark_ckpt_v4_image_bytes(recs.arr, len(recs), int(with_amp), C.byref(out)))
    return out.value


def pack(tensors, image, global_step, adam_step, amp_state=None):
    """Write the V4 image of `tensors` into the uint8 GPU tensor `image`."""
    amp = C.byref(amp_state) if amp_state is not None else None
    recs = _records(tensors)
    check(lib().ark_ckpt_v4_pack(recs.arr, len(recs), global_step, adam_step, amp,
                                 image.data_ptr(), image.numel(), _stream()))


class PackPlan:
    """Repeated V4 saves of the same tensors into the same uint8 GPU tensor
    `image` (ark_ckpt_v4_pack_plan_*): the tables are uploaded once, and each
    run queues the headers and data on the plan's stream without waiting.
    with_amp: the image carries the AMP trailer, and every run passes the
    state.  The tensors and the image must outlive the plan."""

    def __init__(self, tensors, image, with_amp=False, stream=None):
        import torch
        self._recs = _records(tensors)
        self._image = image
        if stream is None:
            stream = torch.cuda.current_stream()
        self._stream = stream
        h = C.c_void_p()
        check(lib().ark_ckpt_v4_pack_plan_create(self._recs.arr, len(self._recs), int(with_amp),
                                                 image.data_ptr(), image.numel(),
                                                 C.c_void_p(stream.cuda_stream), C.byref(h)))
        self._h = h

    def run(self, global_step, adam_step, amp_state=None):
        amp = C.byref(amp_state) if amp_state is not None else None
        check(lib().ark_ckpt_v4_pack_plan_run(self._h, global_step, adam_step, amp))

    def close(self):
        if self._h:
            check(lib().ark_ckpt_plan_destroy(self._h))
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def unpack(image, tensors, file_types=None):
    """Scatter a V4 image (uint8 GPU tensor) into `tensors`; file_types
    defaults to each tensor's own type."""
    recs = _records(tensors)
    ft = recs.types if file_types is None else (C.c_uint32 * max(1, len(recs)))(*file_types)
    check(lib().ark_ckpt_v4_unpack(image.data_ptr(), image.numel(), recs.arr, len(recs), ft,
                                   _stream()))


class CheckpointV3:
    """The reference's checkpoint entry points (io.rs:417-671), GPU side."""

    @staticmethod
    def save_fp16(path, global_step, adam_step, embed_w_f16, embed_m_f32, embed_v_f32,
                  gamma_f_f16, gamma_f_m_f32, gamma_f_v_f32, layer_w_f16, layer_m_f32,
                  layer_v_f32, amp_state=None):
        """io.rs:432-500: embed w/m/v, per layer 9 w, 9 m, 9 v, gamma_final w/m/v."""
        tensors = [embed_w_f16, embed_m_f32, embed_v_f32]
        for w, m, v in zip(layer_w_f16, layer_m_f32, layer_v_f32):
            tensors += list(w) + list(m) + list(v)
        tensors += [gamma_f_f16, gamma_f_m_f32, gamma_f_v_f32]
        save(path, tensors, global_step, adam_step, amp_state)

    @staticmethod
    def load(path, tensors):
        return load(path, tensors)


def param_tensors(params, with_moments=True):
    """A ParamSet's buffers in the V4 file order of guardar_checkpoint
    (training.rs:536-604): embed w, m, v; per layer wq..g2 weights, then
    their m, then their v; gamma_final w, m, v.  with_moments=False gives
    the weights-only V2 order (embed, then each layer's 9)."""
    idx = {s.name: i for i, s in enumerate(params.specs)}
    layers = sorted({int(n[1:].split(".")[0]) for n in idx if n.startswith("l")})
    names = ["wq", "wk", "wv", "wo", "w1", "w2", "w3", "g1", "g2"]
    out = []
    if "embed" in idx:
        i = idx["embed"]
        out += [params.w(i)] + ([params.m(i), params.v(i)] if with_moments else [])
    for l in layers:
        ids = [idx[f"l{l}.{k}"] for k in names]
        out += [params.w(i) for i in ids]
        if with_moments:
            out += [params.m(i) for i in ids] + [params.v(i) for i in ids]
    if "gamma_final" in idx and with_moments:
        i = idx["gamma_final"]
        out += [params.w(i), params.m(i), params.v(i)]
    return out


def save_params(path, params, opt, global_step):
    """guardar_checkpoint: the ParamSet's w/m/v, adam_step = the optimizer's
    t, and the loss-scaler state in the trailer."""
    st = opt.get_state()
    save(path, param_tensors(params), global_step, st.t, st)


def file_tensors(params, version, n_tensors):
    """The ParamSet buffers a file of this version and tensor count fills, in
    file order, as the reference reads them:
    * V4 / V3: param_tensors(params), without gamma_final's w, m, v when the
      file has 3 + 27 L tensors (io.rs:560-565 tells the two apart by the
      count; V3 never has it, io.rs:614-616), which then stay as they are;
    * V2: the weights only, embed and each layer's 9 (the 1 + 9 L tensors
      training.rs:488-509 accepts)."""
    has_gf = any(s.name == "gamma_final" for s in params.specs)
    if version == 2:
        return param_tensors(params, with_moments=False)
    full = param_tensors(params)
    if has_gf and n_tensors == len(full) - 3:
        return full[:-3]
    return full


def load_params(path, params, opt=None):
    """Resume: fill the ParamSet from the file (the tensors file_tensors
    names; the library refuses a file whose count or sizes differ).  With
    opt, set its t to the file's adam_step (optimizer.rs:308) and restore
    the loss-scaler state when the file carries it.  A V2 file holds weights
    only: the reference starts the optimizer from zero after it
    (training.rs:488-509), so the moments are zeroed and t set to 0."""
    head, _ = probe(path)
    info, amp = load(path, file_tensors(params, head.version, head.n_tensors))
    if info.version == 2:
        params.m_arena.zero_()
        params.v_arena.zero_()
    if opt is not None:
        if amp is not None:
            opt.set_state(**{k: getattr(amp, k) for k, _ in _abi.State._fields_
                             if k != "reserved"})
        opt.set_state(t=info.adam_step)
    return info, amp
