"""The library's checkpoint header parser and image sizing on the CPU (no
device call): ark_ckpt_probe on files the oracle writes in the reference's
formats (V4 with and without the AMP trailer, V3, V2), its failures on a bad
magic and on truncation (io.rs:665-668, read_exact), and
ark_ckpt_v4_image_bytes against the oracle's file length."""
import ctypes as C
import struct

import numpy as np
import pytest

from ark_amd import _abi
from ark_amd._lib import lib
from oracle import ckpt as K


def _probe(path, max_n=64):
    ci = _abi.CkptInfo()
    ns = (C.c_uint64 * max_n)()
    ts = (C.c_uint32 * max_n)()
    rc = lib().ark_ckpt_probe(str(path).encode(), C.byref(ci), ns, ts, max_n)
    return rc, ci, list(ns[:ci.n_tensors]), list(ts[:ci.n_tensors])


def _tensors(rng):
    return [rng.integers(0, 65536, 5, dtype=np.uint32).astype(np.uint16),
            rng.standard_normal(3).astype(np.float32),
            rng.integers(0, 65536, 1, dtype=np.uint32).astype(np.uint16),
            np.zeros(0, np.float32),
            rng.standard_normal(4097).astype(np.float32)]


def test_probe_v4_and_trailer(tmp_path):
    rng = np.random.default_rng(1)
    t = _tensors(rng)
    p = tmp_path / "a.bin"
    p.write_bytes(K.write_v4(123, 45, t))
    rc, ci, ns, ts = _probe(p)
    assert rc == 0 and (ci.version, ci.global_step, ci.adam_step, ci.n_tensors) == (4, 123, 45, 5)
    assert ci.has_moments == 1 and ci.has_amp == 0 and ci.file_bytes == p.stat().st_size
    assert ns == [x.size for x in t]
    assert ts == [0 if x.dtype == np.uint16 else 1 for x in t]
    st = _abi.State(t=45, loss_scale=2048.0, clean_steps=7, consecutive_nonfinite=0,
                    skipped_steps=3, early_stop=0, reserved=0)
    p.write_bytes(K.write_v4(123, 45, t) + K.amp_trailer(bytes(st)))
    rc, ci, _, _ = _probe(p)
    assert rc == 0 and ci.has_amp == 1
    # a trailer with a wrong magic is ignored, as the reference ignores any tail
    p.write_bytes(K.write_v4(123, 45, t) + b"XXXX" + bytes(36))
    rc, ci, _, _ = _probe(p)
    assert rc == 0 and ci.has_amp == 0


def test_probe_v3_v2(tmp_path):
    rng = np.random.default_rng(2)
    t = [rng.standard_normal(n).astype(np.float32) for n in (7, 1, 300)]
    p = tmp_path / "b.bin"
    p.write_bytes(K.write_v3(9, 8, t))
    rc, ci, ns, ts = _probe(p)
    assert rc == 0 and (ci.version, ci.adam_step, ci.has_moments) == (3, 8, 1)
    assert ns == [7, 1, 300] and ts == [1, 1, 1]
    p.write_bytes(K.write_v2(9, t))
    rc, ci, ns, ts = _probe(p)
    assert rc == 0 and (ci.version, ci.adam_step, ci.has_moments) == (2, 0, 0)
    assert ns == [7, 1, 300]


def test_probe_failures(tmp_path):
    p = tmp_path / "c.bin"
    p.write_bytes(struct.pack("<IQ", 0xDEADBEEF, 0) + bytes(32))
    rc, _, _, _ = _probe(p)
    assert rc == _abi.EIO and "0xDEADBEEF" in lib().ark_opt_last_error().decode()
    good = K.write_v4(1, 1, [np.zeros(5, np.uint16), np.zeros(3, np.float32)])
    for cut in (1, 8, 16, 20, len(good) - 30):
        p.write_bytes(good[:len(good) - cut])
        rc, _, _, _ = _probe(p)
        assert rc == _abi.EIO, cut
    # a tensor count no file of this size could hold
    bad = bytearray(good)
    struct.pack_into("<Q", bad, 20, 1 << 40)
    p.write_bytes(bytes(bad))
    rc, _, _, _ = _probe(p)
    assert rc == _abi.EIO
    rc, _, _, _ = _probe(tmp_path / "missing.bin")
    assert rc == _abi.EIO


@pytest.mark.parametrize("amp", [0, 1])
def test_image_bytes_matches_oracle_length(amp):
    rng = np.random.default_rng(3)
    t = _tensors(rng)
    recs = (_abi.CkptRecord * len(t))()
    for i, x in enumerate(t):
        recs[i] = _abi.CkptRecord(0x1000 * (i + 1), x.size,
                                  _abi.CKPT_F16 if x.dtype == np.uint16 else _abi.CKPT_F32, 0)
    out = C.c_uint64()
    assert lib().ark_ckpt_v4_image_bytes(recs, len(t), amp, C.byref(out)) == 0
    assert out.value == len(K.write_v4(0, 0, t)) + 40 * amp


def _layout_fits(ci, ns, ts):
    """The probed layout inside the file: headers plus data no longer than it."""
    head = {4: 28, 3: 28, 2: 20}[ci.version]
    rec = 16 if ci.version == 4 else 8
    total = head + sum(rec + n * (2 if t == _abi.CKPT_F16 else 4) for n, t in zip(ns, ts))
    return total <= ci.file_bytes


@pytest.mark.parametrize("version", [4, 3, 2])
def test_probe_survives_corrupted_and_truncated_files(tmp_path, version):
    """Random truncations and byte overwrites of a valid file (headers, sizes,
    types, data): the parser either rejects the file with EIO or reports a
    layout that fits inside it -- never a crash, never an out-of-file read."""
    from hypothesis import given, settings, HealthCheck
    from hypothesis import strategies as st

    rng = np.random.default_rng(version)
    t = [rng.standard_normal(n).astype(np.float32) for n in (5, 1, 0, 33)]
    if version == 4:
        t[0] = rng.integers(0, 65536, 5, dtype=np.uint32).astype(np.uint16)
        good = K.write_v4(7, 6, t) + K.amp_trailer(bytes(40 - 8))
    elif version == 3:
        good = K.write_v3(7, 6, t)
    else:
        good = K.write_v2(7, t)
    p = tmp_path / f"f{version}.bin"

    @settings(max_examples=300, deadline=None, suppress_health_check=list(HealthCheck))
    @given(cut=st.integers(0, len(good)), off=st.integers(0, len(good) - 1),
           junk=st.binary(min_size=1, max_size=12))
    def check(cut, off, junk):
        b = bytearray(good)
        b[off:off + len(junk)] = junk
        b = bytes(b[:len(b) - cut])
        p.write_bytes(b)
        rc, ci, ns, ts = _probe(p, max_n=8)
        assert rc in (0, _abi.EIO)
        if rc == 0:
            assert ci.file_bytes == len(b)
            if ci.n_tensors <= 8:
                assert _layout_fits(ci, ns, ts)

    check()
