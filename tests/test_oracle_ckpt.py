"""Pins of the checkpoint oracle (oracle/ckpt.py) against the reference's
format (proyecto_ark/ark01/src/io.rs:12-24, :412-414, :432-671): a
known-answer file typed byte by byte from the format description, the
loader's tensor regrouping and gamma_final detection, the V3 / V2 layouts,
and its failure modes.  The reference ships no checkpoint to compare with
(its entren/ directory holds only a JSONL file)."""
import struct

import numpy as np
import pytest

import oracle
from oracle import ckpt as K

# 0 layers: embed w (2 x f16), m (1 x f32), v (0); gamma_final w (1 x f16),
# m (1 x f32), v (1 x f32).  global_step 258, adam_step 7, n_tensors 6.
KNOWN = bytes.fromhex(
    "4152344b" "0201000000000000" "0700000000000000" "0600000000000000"
    "0200000000000000" "0000000000000000" "003c00c0"           # embed w: 1.0, -2.0
    "0100000000000000" "0100000000000000" "0000003f"           # embed m: 0.5
    "0000000000000000" "0100000000000000"                      # embed v: empty
    "0100000000000000" "0000000000000000" "007e"               # gamma w: qNaN
    "0100000000000000" "0100000000000000" "00000080"           # gamma m: -0.0
    "0100000000000000" "0100000000000000" "01000000"           # gamma v: 2^-149
)


def _known_args():
    return dict(global_step=258, adam_step=7,
                embed_w_f16=np.array([0x3C00, 0xC000], np.uint16),
                embed_m_f32=np.array([0.5], np.float32),
                embed_v_f32=np.zeros(0, np.float32),
                gamma_f_f16=np.array([0x7E00], np.uint16),
                gamma_f_m_f32=np.array([-0.0], np.float32),
                gamma_f_v_f32=np.array([1], np.uint32).view(np.float32),
                layer_w_f16=[], layer_m_f32=[], layer_v_f32=[])


def test_known_answer_bytes():
    assert K.save_fp16(**_known_args()) == KNOWN
    # u32 0x4B345241 little endian: the file starts with the bytes "AR4K"
    assert KNOWN[:4] == b"AR4K"


def test_known_answer_load():
    r = K.load(KNOWN)
    assert r["global_step"] == 258 and r["adam_step"] == 7 and r["tiene_momentos"]
    p, m, v = r["pesos"], r["momentos_m"], r["momentos_v"]
    assert len(p) == len(m) == len(v) == 2  # embed, gamma_final (6 = 3 + 0*27 + 3)
    assert p[0].tolist() == [1.0, -2.0]
    assert np.isnan(p[1][0]) and p[1].view(np.uint32)[0] == 0x7FC00000
    assert m[0].tolist() == [0.5] and m[1].view(np.uint32)[0] == 0x80000000
    assert v[0].size == 0 and v[1].view(np.uint32)[0] == 1


def _rand_layers(rng, n_layers, d, h):
    sizes = [d * d] * 4 + [d * h, h * d, d * h, d, d]
    w = [[rng.integers(0, 65536, s, dtype=np.uint32).astype(np.uint16) for s in sizes]
         for _ in range(n_layers)]
    m = [[rng.standard_normal(s).astype(np.float32) for s in sizes] for _ in range(n_layers)]
    v = [[rng.random(s, dtype=np.float32) for s in sizes] for _ in range(n_layers)]
    return w, m, v


@pytest.mark.parametrize("n_layers", [1, 3])
def test_regrouping_with_gamma_final(n_layers):
    rng = np.random.default_rng(n_layers)
    d, h, vocab = 5, 7, 11
    w, m, v = _rand_layers(rng, n_layers, d, h)
    ew = rng.integers(0, 65536, vocab * d, dtype=np.uint32).astype(np.uint16)
    em, ev = rng.standard_normal(vocab * d).astype(np.float32), rng.random(vocab * d, np.float32)
    gw = rng.integers(0, 65536, d, dtype=np.uint32).astype(np.uint16)
    gm, gv = rng.standard_normal(d).astype(np.float32), rng.random(d, np.float32)
    buf = K.save_fp16(3, 2, ew, em, ev, gw, gm, gv, w, m, v)
    head, recs = K.records(buf)
    assert head["n_tensors"] == 3 + 27 * n_layers + 3 == len(recs)
    assert head["end"] == len(buf)
    r = K.load(buf)
    # pesos: embed, then each layer's 9, then gamma_final (io.rs:569-586)
    want_p = [ew] + [t for l in w for t in l] + [gw]
    assert len(r["pesos"]) == 1 + 9 * n_layers + 1
    for a, b in zip(r["pesos"], want_p):
        np.testing.assert_array_equal(a.view(np.uint32), oracle.f16_to_f32(b).view(np.uint32))
    for a, b in zip(r["momentos_m"], [em] + [t for l in m for t in l] + [gm]):
        np.testing.assert_array_equal(a, b)
    for a, b in zip(r["momentos_v"], [ev] + [t for l in v for t in l] + [gv]):
        np.testing.assert_array_equal(a, b)


def test_v4_without_gamma_final():
    """30 = 3 + 27 tensors: (30 - 3) % 27 == 0, so no gamma_final and one layer."""
    rng = np.random.default_rng(9)
    tens = [rng.integers(0, 65536, 4, dtype=np.uint32).astype(np.uint16) if (i < 3 and i == 0)
            or (i >= 3 and (i - 3) % 27 < 9) else rng.standard_normal(4).astype(np.float32)
            for i in range(30)]
    r = K.load(K.write_v4(1, 1, tens))
    assert len(r["pesos"]) == 10 and len(r["momentos_m"]) == 10


def test_v3_and_v2_layouts():
    rng = np.random.default_rng(3)
    t = [rng.standard_normal(n).astype(np.float32) for n in (6, 6, 6)]
    v3 = K.write_v3(11, 4, t)
    assert v3[:4] == b"AR3K" and struct.unpack("<QQQ", v3[4:28]) == (11, 4, 3)
    assert len(v3) == 28 + 3 * (8 + 24)
    r = K.load(v3)
    assert r["adam_step"] == 4 and r["tiene_momentos"] and len(r["pesos"]) == 1
    np.testing.assert_array_equal(r["momentos_v"][0], t[2])
    v2 = K.write_v2(12, t[:2])
    assert v2[:4] == b"AR2K" and len(v2) == 20 + 2 * (8 + 24)
    r = K.load(v2)
    assert r["adam_step"] == 0 and not r["tiene_momentos"] and len(r["pesos"]) == 2


def test_failures_and_trailer():
    with pytest.raises(ValueError, match="0x12345678"):
        K.load(struct.pack("<IQ", 0x12345678, 0) + b"\0" * 40)
    with pytest.raises(K.Truncated):
        K.load(KNOWN[:-1])
    with pytest.raises(K.Truncated):
        K.load(KNOWN[:20])
    # the reference loader stops after n_tensors: a trailer changes nothing
    tr = K.amp_trailer(bytes(range(32)))
    assert len(tr) == 40 and tr[:4] == b"AMPS"
    a, b = K.load(KNOWN), K.load(KNOWN + tr)
    for k in ("pesos", "momentos_m", "momentos_v"):
        for x, y in zip(a[k], b[k]):
            np.testing.assert_array_equal(x.view(np.uint32), y.view(np.uint32))


def test_nonzero_type_reads_as_f32():
    """io.rs:534 tests type == 0 only: any other type is read as F32."""
    buf = bytearray(K.write_v4(0, 0, [np.array([1.5, 2.5], np.float32)] * 3))
    struct.pack_into("<Q", buf, 28 + 8, 7)  # first record's type := 7
    head, recs = K.records(bytes(buf))
    assert recs[0][1] == 1 and recs[0][2].tolist() == [1.5, 2.5]
