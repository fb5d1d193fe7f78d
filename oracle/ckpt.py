"""CPU restatement of the ARK checkpoint format -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
this module, as the checker of the GPU checkpoint path; the product never
does.

Follows proyecto_ark/ark01/src/io.rs:
  save_fp16  io.rs:432-500  (V4 writer: header :453-456, tensor records
                             :459-471, order :473-494)
  load       io.rs:504-671  (magic dispatch :516-520; V4 :520-595 with the
                             type test :534 and the gamma_final detection
                             :560-565; V3 :597-636; V2 :638-662; bad magic
                             :665-668)
The fp16 -> fp32 of load is half::f16::to_f32 (memory.rs:111-113, half
2.7.1 per eko_infer/Cargo.lock): IEEE exact widening, NaNs quieted with
their payload, which oracle.f16_to_f32 restates.

V3 and V2 files have no writer in the reference; ``write_v3`` / ``write_v2``
build the byte layouts its loader reads (io.rs:597-662).  ``amp_trailer`` is
this build's extension (40 bytes after the last tensor), which ``load``
ignores exactly as the reference's loader does.
"""
import struct

import numpy as np

from . import f16_to_f32

MAGIC_V2 = 0x4B325241  # "ARK2"  io.rs:412
MAGIC_V3 = 0x4B335241  # "ARK3"  io.rs:413
MAGIC_V4 = 0x4B345241  # "ARK4"  io.rs:414
MAGIC_AMP = 0x53504D41  # "AMPS"  (extension)


def _u16(a):
    a = np.asarray(a)
    assert a.dtype in (np.uint16, np.int16, np.float16), a.dtype
    return np.ascontiguousarray(a).view(np.uint16)


def _f32(a):
    a = np.asarray(a)
    assert a.dtype in (np.float32, np.uint32, np.int32), a.dtype
    return np.ascontiguousarray(a).view(np.float32)


def _rec_f16(data):  # write_tensor_f16, io.rs:459-464
    d = _u16(data)
    return struct.pack("<QQ", d.size, 0) + d.astype("<u2").tobytes()


def _rec_f32(data):  # write_tensor_f32, io.rs:466-471
    d = _f32(data)
    return struct.pack("<QQ", d.size, 1) + d.astype("<f4").tobytes()


def save_fp16(global_step, adam_step, embed_w_f16, embed_m_f32, embed_v_f32,
              gamma_f_f16, gamma_f_m_f32, gamma_f_v_f32, layer_w_f16, layer_m_f32, layer_v_f32):
    """The bytes CheckpointV3::save_fp16 writes (io.rs:432-500)."""
    n_layers = len(layer_w_f16)
    n_tensors = 3 + n_layers * 27 + 3  # io.rs:448
    out = [struct.pack("<IQQQ", MAGIC_V4, global_step, adam_step, n_tensors)]
    out += [_rec_f16(embed_w_f16), _rec_f32(embed_m_f32), _rec_f32(embed_v_f32)]
    for l in range(n_layers):
        out += [_rec_f16(t) for t in layer_w_f16[l]]
        out += [_rec_f32(t) for t in layer_m_f32[l]]
        out += [_rec_f32(t) for t in layer_v_f32[l]]
    out += [_rec_f16(gamma_f_f16), _rec_f32(gamma_f_m_f32), _rec_f32(gamma_f_v_f32)]
    return b"".join(out)


def write_v4(global_step, adam_step, tensors):
    """A V4 file of arbitrary tensors in the given order (uint16/float16 ->
    type 0, float32 -> type 1), the record format of io.rs:459-471."""
    out = [struct.pack("<IQQQ", MAGIC_V4, global_step, adam_step, len(tensors))]
    for t in tensors:
        t = np.asarray(t)
        out.append(_rec_f16(t) if t.dtype.itemsize == 2 else _rec_f32(t))
    return b"".join(out)


def write_v3(global_step, adam_step, tensors_f32):
    out = [struct.pack("<IQQQ", MAGIC_V3, global_step, adam_step, len(tensors_f32))]
    for t in tensors_f32:
        d = _f32(t)
        out.append(struct.pack("<Q", d.size) + d.astype("<f4").tobytes())
    return b"".join(out)


def write_v2(global_step, tensors_f32):
    out = [struct.pack("<IQQ", MAGIC_V2, global_step, len(tensors_f32))]
    for t in tensors_f32:
        d = _f32(t)
        out.append(struct.pack("<Q", d.size) + d.astype("<f4").tobytes())
    return b"".join(out)


def amp_trailer(state_bytes):
    """The 40-byte AMP trailer: magic, version 1, the 32-byte ark_opt_state."""
    assert len(state_bytes) == 32
    return struct.pack("<II", MAGIC_AMP, 1) + bytes(state_bytes)


class Truncated(ValueError):
    pass


def _take(buf, off, n):
    if off + n > len(buf):
        raise Truncated(f"need bytes [{off}, {off + n}) of {len(buf)}")
    return buf[off:off + n], off + n


def records(buf):
    """Walk a V2/V3/V4 file: (header dict, [(n, type, raw ndarray)]) with
    type 0 (F16, uint16 array) or 1 (F32, float32 array), in file order."""
    buf = memoryview(buf)
    b, off = _take(buf, 0, 4)
    (magic,) = struct.unpack("<I", b)
    b, off = _take(buf, off, 8)
    (global_step,) = struct.unpack("<Q", b)
    if magic in (MAGIC_V4, MAGIC_V3):
        b, off = _take(buf, off, 16)
        adam_step, n_tensors = struct.unpack("<QQ", b)
        version = 4 if magic == MAGIC_V4 else 3
    elif magic == MAGIC_V2:
        b, off = _take(buf, off, 8)
        (n_tensors,) = struct.unpack("<Q", b)
        adam_step, version = 0, 2
    else:
        raise ValueError(f"Magic signature 0x{magic:08X} invalida")  # io.rs:665-668
    out = []
    for _ in range(n_tensors):
        b, off = _take(buf, off, 8)
        (n,) = struct.unpack("<Q", b)
        tipo = 1
        if version == 4:
            b, off = _take(buf, off, 8)
            (tipo,) = struct.unpack("<Q", b)
        if version == 4 and tipo == 0:  # io.rs:534: 0 = F16, anything else F32
            b, off = _take(buf, off, 2 * n)
            out.append((n, 0, np.frombuffer(b, dtype="<u2").copy()))
        else:
            b, off = _take(buf, off, 4 * n)
            out.append((n, 1, np.frombuffer(b, dtype="<f4").copy()))
    head = dict(version=version, global_step=global_step, adam_step=adam_step,
                n_tensors=n_tensors, end=off)
    return head, out


def load(buf):
    """CheckpointV3::load on the file bytes (io.rs:504-671): a dict with
    global_step, adam_step, pesos, momentos_m, momentos_v (float32 arrays)
    and tiene_momentos."""
    head, recs = records(buf)
    v = head["version"]
    tens = [r[2].astype(np.float32) if r[1] == 1 else f16_to_f32(r[2]) for r in recs]
    if v == 2:  # io.rs:638-662
        return dict(global_step=head["global_step"], adam_step=0, pesos=tens,
                    momentos_m=[], momentos_v=[], tiene_momentos=False)
    n_tensors = head["n_tensors"]
    if v == 4:  # io.rs:560-565
        has_gamma_final = (n_tensors - 3) % 27 == 3
        n_layers = (n_tensors - 6) // 27 if has_gamma_final else (n_tensors - 3) // 27
    else:  # io.rs:614-616
        has_gamma_final = False
        n_layers = (n_tensors - 3) // 27
    pesos, m, vv = [tens[0]], [tens[1]], [tens[2]]
    rem = tens[3:3 + n_layers * 27]
    for l in range(n_layers):
        base = l * 27
        pesos += rem[base:base + 9]
        m += rem[base + 9:base + 18]
        vv += rem[base + 18:base + 27]
    if has_gamma_final:
        g = 3 + n_layers * 27
        pesos.append(tens[g])
        m.append(tens[g + 1])
        vv.append(tens[g + 2])
    return dict(global_step=head["global_step"], adam_step=head["adam_step"], pesos=pesos,
                momentos_m=m, momentos_v=vv, tiene_momentos=True)
