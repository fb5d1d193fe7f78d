"""The C ABI library on the CPU (no GPU calls): it loads, exports every
function include/*.h declares with matching struct layouts, and rejects bad
arguments before touching the device."""
import ctypes as C
import os
import re

from ark_amd import _abi
from ark_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    names = _lib.exported_symbols()
    assert len(names) >= 17
    for n in names:
        assert hasattr(L, n), n
    # and the header list is complete: every ark_* symbol of the .so is declared
    syms = os.popen(f"nm -D --defined-only {_lib.LIB_PATH}").read()
    exported = set(re.findall(r" T (ark_\w+)", syms))
    assert exported == set(names)


def test_struct_layouts_match():
    L = _lib.lib()
    sizes = (C.c_size_t * 5)()
    assert L.ark_opt_struct_sizes(sizes, 5) == 5
    assert list(sizes) == [C.sizeof(s) for s in _abi.STRUCTS]
    k = len(_abi.ALL_STRUCTS)
    sizes = (C.c_size_t * (k + 3))()
    assert L.ark_opt_struct_sizes(sizes, k + 3) == k  # no more than it knows
    assert list(sizes)[:k] == [C.sizeof(s) for s in _abi.ALL_STRUCTS]
    assert [C.sizeof(s) for s in _abi.ALL_STRUCTS[5:]] == [24, 24, 48, 24]
    assert L.ark_opt_abi_version() == _abi.ABI_VERSION
    assert L.ark_opt_struct_sizes(None, 5) == _abi.EINVAL


def _hp():
    hp = _abi.HParams()
    _lib.lib().ark_opt_default_hparams(C.byref(hp))
    return hp


def _create(table, n, hp):
    h = C.c_void_p()
    rc = _lib.lib().ark_opt_create(table, n, C.byref(hp) if hp is not None else None, None,
                                   C.byref(h))
    return rc, h, _lib.lib().ark_opt_last_error().decode()


def test_create_rejects_bad_arguments_before_device_calls():
    t = (_abi.Tensor * 1)()
    t[0].w, t[0].g, t[0].m, t[0].v, t[0].n = 0x1000, 0x2000, 0x3000, 0x4000, 10
    assert _create(None, 1, _hp())[0] == _abi.EINVAL
    assert _create(t, 0, _hp())[0] == _abi.EINVAL
    rc, h, msg = _create(t, 1, None)
    assert rc == _abi.EINVAL and "hparams" in msg
    for field, value, word in [("grad_clip", 0.0, "grad_clip"), ("grad_clip", -1.0, "grad_clip"),
                               ("grad_clip", float("nan"), "grad_clip"),
                               ("beta1", float("nan"), "finite"),
                               ("loss_scale_init", float("inf"), "loss_scale_init"),
                               ("loss_scale_min", 0.0, "loss_scale_min"),
                               ("grad_dtype", 7, "grad_dtype")]:
        hp = _hp()
        setattr(hp, field, value)
        rc, h, msg = _create(t, 1, hp)
        assert rc == _abi.EINVAL and word in msg, (field, msg)
    t[0].w = 0x1001  # odd address for fp16
    rc, h, msg = _create(t, 1, _hp())
    assert rc == _abi.EINVAL and "aligned" in msg
    t[0].w = 0x1000
    t[0].weight_decay = float("nan")
    rc, h, msg = _create(t, 1, _hp())
    assert rc == _abi.EINVAL and "weight_decay" in msg
    t[0].weight_decay = 0.0
    for n in (2 ** 64 - 1, 2 ** 63, 2 ** 48 + 1):  # segment count and byte sizes would wrap
        t[0].n = n
        rc, h, msg = _create(t, 1, _hp())
        assert rc == _abi.EINVAL and "too large" in msg, (n, msg)


def _table(rows):
    """A tensor table of fake device addresses: rows of (w, g, m, v, n)."""
    t = (_abi.Tensor * len(rows))()
    for i, (w, g, m, v, n) in enumerate(rows):
        t[i].w, t[i].g, t[i].m, t[i].v, t[i].n = w, g, m, v, n
    return t


MB = 1 << 20


def test_create_rejects_aliased_buffers_before_device_calls():
    """The reference steps distinct per-tensor fields (optimizer.rs:171,
    memory.rs:202-255); a table whose written buffers (w, m, v) share a byte
    with each other or with a gradient is refused, naming both, before any
    device query (the addresses here are not memory at all)."""
    ok = [(1 * MB, 2 * MB, 3 * MB, 4 * MB, 1000), (5 * MB, 6 * MB, 7 * MB, 8 * MB, 1000)]
    cases = {
        "duplicate entry": ([ok[0], ok[1], ok[0]], ["tensor 0 w", "tensor 2 w"]),
        "partial w overlap": ([ok[0], (1 * MB + 1998, 6 * MB, 7 * MB, 8 * MB, 1000)],
                              ["tensor 0 w", "tensor 1 w"]),
        "m equal to v": ([ok[0], (5 * MB, 6 * MB, 7 * MB, 7 * MB, 1000)],
                         ["tensor 1 m", "tensor 1 v"]),
        "g inside w": ([(1 * MB, 1 * MB + 400, 3 * MB, 4 * MB, 1000), ok[1]],
                       ["tensor 0 g", "tensor 0 w"]),
        "g of one tensor on another's v": ([ok[0], (5 * MB, 4 * MB + 3996, 7 * MB, 8 * MB, 1000)],
                                           ["tensor 1 g", "tensor 0 v"]),
    }
    for name, (rows, words) in cases.items():
        rc, h, msg = _create(_table(rows), len(rows), _hp())
        assert rc == _abi.EINVAL and not h.value, (name, msg)
        assert "overlaps" in msg and all(w in msg for w in words), (name, msg)
    # touching but disjoint spans, an empty tensor on top of another and two
    # tensors sharing one read-only gradient pass the check (and then fail the
    # device query, since the addresses are fake)
    for rows in ([(1 * MB, 2 * MB, 3 * MB, 4 * MB, 1000), (1 * MB + 2000, 2 * MB, 3 * MB + 4000,
                                                           4 * MB + 4000, 1000)],
                 [ok[0], (1 * MB, 1 * MB, 1 * MB, 1 * MB, 0)]):
        rc, h, msg = _create(_table(rows), len(rows), _hp())
        assert rc != _abi.OK and "overlaps" not in msg, msg


def test_single_tensor_dropin_rejects_aliased_buffers():
    L = _lib.lib()
    msg = lambda: L.ark_opt_last_error().decode()
    args = (3e-4, 0.9, 0.999, 1e-8, 0.01, 1, None)
    for (w, g, m, v), words in [((1 * MB, 2 * MB, 3 * MB, 3 * MB), ("m", "v")),
                                ((1 * MB, 1 * MB + 8, 3 * MB, 4 * MB), ("g", "w")),
                                ((1 * MB, 2 * MB, 1 * MB + 1996, 4 * MB), ("w", "m")),
                                ((1 * MB, 4 * MB + 3996, 3 * MB, 4 * MB), ("g", "v"))]:
        assert L.ark_hip_adam_step_f16(w, g, m, v, 1000, *args) == _abi.EINVAL
        assert "overlaps" in msg() and all(f"0 {x}" in msg() for x in words), msg()
    assert L.ark_hip_adam_step_f16(1 * MB, 2 * MB, 3 * MB, 3 * MB + 4000, 1000, *args) != 0
    assert "overlaps" not in msg()


def test_fp32_weight_dropin_argument_checks():
    L = _lib.lib()
    msg = lambda: L.ark_opt_last_error().decode()
    args = (3e-4, 0.9, 0.999, 1e-8, 0.01, 1, None)
    assert L.ark_hip_adam_step(None, None, None, None, 0, *args) == _abi.OK
    assert L.ark_hip_adam_step(0x1002, 0x2000, 0x3000, 0x4000, 10, *args) == _abi.EINVAL
    assert "aligned" in msg()
    for n in (2 ** 64 - 1, 2 ** 48 + 1):
        assert L.ark_hip_adam_step(0x1000, 0x2000, 0x3000, 0x4000, n, *args) == _abi.EINVAL
        assert "too large" in msg()
    # fp32 w spans 4 B per element: w at 1 MiB reaches into m placed 3996 B on
    assert L.ark_hip_adam_step(1 * MB, 2 * MB, 1 * MB + 3996, 3 * MB, 1000, *args) == _abi.EINVAL
    assert "overlaps" in msg() and "0 w" in msg() and "0 m" in msg(), msg()
    assert L.ark_hip_adam_step(1 * MB, 2 * MB, 1 * MB + 4000, 3 * MB, 1000, *args) != _abi.OK
    assert "overlaps" not in msg()


def test_single_tensor_dropin_argument_checks():
    L = _lib.lib()
    assert L.ark_hip_adam_step_f16(None, None, None, None, 0, 3e-4, 0.9, 0.999, 1e-8, 0.01, 1,
                                   None) == _abi.OK
    rc = L.ark_hip_adam_step_f16(0x1001, 0x2000, 0x3000, 0x4000, 10, 3e-4, 0.9, 0.999, 1e-8,
                                 0.01, 1, None)
    assert rc == _abi.EINVAL
    rc = L.ark_hip_adam_step_f16(0x1000, 0x2002, 0x3000, 0x4000, 10, 3e-4, 0.9, 0.999, 1e-8,
                                 0.01, 1, None)
    assert rc == _abi.EINVAL
    for n in (2 ** 64 - 1, 2 ** 64 - 100, 2 ** 48 + 1):  # the grid-size test would wrap
        rc = L.ark_hip_adam_step_f16(0x1000, 0x2000, 0x3000, 0x4000, n, 3e-4, 0.9, 0.999, 1e-8,
                                     0.01, 1, None)
        assert rc == _abi.EINVAL and "too large" in L.ark_opt_last_error().decode(), n


def test_grad_clip_dropin_argument_checks():
    L = _lib.lib()
    msg = lambda: L.ark_opt_last_error().decode()
    norm = C.c_float(7.0)
    # no values: norm 0 and nothing queued (the Rust wrapper's empty slice)
    assert L.ark_hip_grad_clip(None, 0, 1.0, C.byref(norm), None) == _abi.OK and norm.value == 0.0
    assert L.ark_hip_grad_clip(None, 0, 1.0, None, None) == _abi.OK
    norm.value = 7.0
    assert L.ark_hip_grad_clip(0x1002, 10, 1.0, C.byref(norm), None) == _abi.EINVAL
    assert "aligned" in msg() and norm.value == 0.0
    for n in (2 ** 64 - 1, 2 ** 32 + 1):
        assert L.ark_hip_grad_clip(0x1000, n, 1.0, None, None) == _abi.EINVAL
        assert "exceeds" in msg()
    # aligned and in range: the buffer check (no GPU here) refuses it
    assert L.ark_hip_grad_clip(0x1000, 10, 1.0, C.byref(norm), None) != _abi.OK


def test_synth_argument_checks():
    L = _lib.lib()
    assert L.ark_synth_copy(0x1000, 0x2008, 64, None) == -1
    assert L.ark_synth_copy(0x1000, 0x2000, 17, None) == -1
    assert L.ark_synth_copy(None, None, 0, None) == 0
    assert L.ark_synth_normal_f16(None, 0, 1, 2, 3, 1.0, None) == 0
    assert L.ark_synth_normal_f16(None, 5, 1, 2, 3, 1.0, None) == -1
    sm = L.ark_synth_stream_mix
    assert sm(None, None, None, None, 0, 0, 0, None) == 0
    assert sm(0x1000, 0x2000, 0x3000, 0x4000, 300, 0, 0, None) == -1  # not a multiple of 256
    assert sm(0x1000, 0x2008, 0x3000, 0x4000, 256, 0, 0, None) == -1  # not 16-byte aligned
    assert sm(None, 0x2000, 0x3000, 0x4000, 256, 0, 0, None) == -1
    assert sm(0x1000, 0x2000, 0x3000, 0x4000, 2 ** 50, 0, 0, None) == -1  # grid too large
    assert sm(0x1000, 0x2000, 0x3000, 0x4000, 256, 0, 33, None) == -1  # more than 32 per CU


def test_handle_calls_reject_null():
    L = _lib.lib()
    assert L.ark_opt_step(None, 1e-3, None) == _abi.EINVAL
    assert L.ark_opt_record_overflow(None, None) == _abi.EINVAL
    assert L.ark_opt_get_state(None, None) == _abi.EINVAL
    assert L.ark_opt_set_state(None, None) == _abi.EINVAL
    assert L.ark_opt_destroy(None) == _abi.OK


def test_headers_cite_reference_interfaces():
    text = open(os.path.join(ROOT, "include", "ark_opt.h")).read()
    for cite in ("opti.s:189-193", "optimizer.rs:171-228", "training.rs:289-326",
                 "training.rs:228-241", "optimizer.rs:237-313", "opti.s:369-432"):
        assert cite in text


def test_next_rows_reject_bad_arguments_before_device_calls():
    """The codec, gradient and checkpoint entry points refuse NULL buffers,
    misalignment and unknown enums with EINVAL and a message, before any
    HIP call."""
    L = _lib.lib()
    msg = lambda: L.ark_opt_last_error().decode()
    assert L.ark_hip_dequant_f16_to_f32(None, None, 0, None) == 0  # n == 0 is a no-op
    assert L.ark_hip_dequant_f16_to_f32(None, None, 8, None) == _abi.EINVAL and "NULL" in msg()
    assert L.ark_hip_quant_f32_to_f16(2, 16, 8, None) == _abi.EINVAL and "aligned" in msg()
    h = C.c_void_p()
    assert L.ark_codec_plan_create(None, 1, 0, None, C.byref(h)) == _abi.EINVAL
    assert L.ark_codec_plan_create(None, 0, 7, None, C.byref(h)) == _abi.EINVAL and "direction" in msg()
    assert L.ark_grad_accumulate(None, None, 4, None) == _abi.EINVAL
    assert L.ark_grad_accumulate(6, 8, 4, None) == _abi.EINVAL and "aligned" in msg()
    assert L.ark_grad_embed_scatter(None, 0, 4, None, None, 3, None) == _abi.EINVAL and "vocab" in msg()
    assert L.ark_grad_embed_scatter(None, 10, 4, None, None, 0, None) == 0  # empty batch
    assert (L.ark_grad_embed_scatter_noalloc(None, 0, 4, None, None, 3, None) == _abi.EINVAL
            and "vocab" in msg())
    assert L.ark_grad_embed_scatter_noalloc(None, 10, 4, None, None, 0, None) == 0
    # one 256-lane block per token: 2^24 tokens would be 2^32 work-items
    for f in (L.ark_grad_embed_scatter, L.ark_grad_embed_scatter_noalloc):
        assert f(1 << 20, 10, 4, 2 << 20, 3 << 20, 1 << 24, None) == _abi.EINVAL
        assert "too large" in msg(), msg()
    recs = (_abi.CkptRecord * 1)()
    recs[0] = _abi.CkptRecord(0, 4, 9, 0)
    out = C.c_uint64()
    assert L.ark_ckpt_v4_image_bytes(recs, 1, 0, C.byref(out)) == _abi.EINVAL and "dtype" in msg()
    assert L.ark_ckpt_save_v4(None, 0, 0, recs, 1, None, None) == _abi.EINVAL
    assert L.ark_ckpt_probe(None, None, None, None, 0) == _abi.EINVAL


def test_plans_reject_overlapping_spans_before_device_calls():
    """A gradient or codec plan runs every span in one launch, so a dst that
    shares a byte with another span's dst or src would race; such tables are
    refused, naming both spans, before any device query (the addresses are
    not memory at all).  Sources may overlap each other."""
    L = _lib.lib()
    msg = lambda: L.ark_opt_last_error().decode()
    h = C.c_void_p()

    def grad(rows):
        arr = (_abi.GradSpan * len(rows))()
        for i, (d, s_, n) in enumerate(rows):
            arr[i] = _abi.GradSpan(d, s_, n)
        return L.ark_grad_plan_create(arr, len(rows), None, C.byref(h))

    def codec(rows, direction=_abi.CODEC_F16_TO_F32):
        arr = (_abi.CodecSpan * len(rows))()
        for i, (s_, d, n) in enumerate(rows):
            arr[i] = _abi.CodecSpan(s_, d, n)
        return L.ark_codec_plan_create(arr, len(rows), direction, None, C.byref(h))

    # gradient spans (dst, src, n), 4 B per element
    bad = {
        "same dst twice": [(1 * MB, 2 * MB, 1000), (1 * MB, 3 * MB, 1000)],
        "dst inside another dst": [(1 * MB, 2 * MB, 1000), (1 * MB + 400, 3 * MB, 10)],
        "dst on another span's src": [(1 * MB, 2 * MB, 1000), (2 * MB + 3996, 3 * MB, 10)],
    }
    for name, rows in bad.items():
        assert grad(rows) == _abi.EINVAL and not h.value, name
        assert "overlaps" in msg() and "span 0" in msg() and "span 1" in msg(), (name, msg())
    # shared sources, touching spans and an empty span on top pass the check
    for rows in ([(1 * MB, 3 * MB, 1000), (2 * MB, 3 * MB, 1000)],
                 [(1 * MB, 3 * MB, 1000), (1 * MB + 4000, 4 * MB, 1000)],
                 [(1 * MB, 3 * MB, 1000), (1 * MB, 1 * MB, 0)]):
        assert grad(rows) != _abi.OK and "overlaps" not in msg(), msg()
    # codec spans (src, dst, n): f16 -> f32 reads 2 B and writes 4 B per element
    bad = {
        "same dst twice": [(1 * MB, 2 * MB, 1000), (3 * MB, 2 * MB, 1000)],
        "dst on another span's src": [(1 * MB, 2 * MB, 1000), (3 * MB, 1 * MB + 1996, 10)],
        "dst partly over another dst": [(1 * MB, 2 * MB, 1000), (3 * MB, 2 * MB + 3996, 10)],
    }
    for name, rows in bad.items():
        assert codec(rows) == _abi.EINVAL and not h.value, name
        assert "overlaps" in msg() and "span 0" in msg() and "span 1" in msg(), (name, msg())
    for rows in ([(1 * MB, 2 * MB, 1000), (1 * MB, 3 * MB, 1000)],
                 [(1 * MB, 2 * MB, 1000), (3 * MB, 2 * MB + 4000, 1000)]):
        assert codec(rows) != _abi.OK and "overlaps" not in msg(), msg()


def test_checkpoint_calls_reject_overlapping_buffers_before_device_calls():
    """Unpack and load write every record in one launch, so their records
    must be pairwise disjoint; pack writes the image and unpack reads it, so
    the image must not overlap any record.  Refused before any device query
    (the addresses are not memory); pack's records may overlap each other."""
    L = _lib.lib()
    msg = lambda: L.ark_opt_last_error().decode()

    def recs(rows):
        arr = (_abi.CkptRecord * len(rows))()
        for i, (p, n, dt) in enumerate(rows):
            arr[i] = _abi.CkptRecord(p, n, dt, 0)
        return arr

    F16, F32 = _abi.CKPT_F16, _abi.CKPT_F32
    overlapping = recs([(1 * MB, 1000, F16), (1 * MB + 1000, 1000, F32)])
    disjoint = recs([(1 * MB, 1000, F16), (2 * MB, 1000, F32)])
    types = (C.c_uint32 * 2)(F16, F32)
    # unpack: records written
    assert L.ark_ckpt_v4_unpack(8 * MB, 1 * MB, overlapping, 2, types, None) == _abi.EINVAL
    assert "record 0 data overlaps record 1 data" in msg(), msg()
    assert L.ark_ckpt_v4_unpack(2 * MB - 16, 64, disjoint, 2, types, None) == _abi.EINVAL
    assert "record 1 data overlaps the image" in msg(), msg()
    assert L.ark_ckpt_v4_unpack(8 * MB, 1 * MB, disjoint, 2, types, None) != _abi.OK
    assert "overlaps" not in msg(), msg()
    # pack: the image written, records read (they may overlap each other)
    assert L.ark_ckpt_v4_pack(disjoint, 2, 0, 0, None, 1 * MB + 512, 1 * MB, None) == _abi.EINVAL
    assert "record 0 data overlaps the image" in msg(), msg()
    assert L.ark_ckpt_v4_pack(overlapping, 2, 0, 0, None, 8 * MB, 1 * MB, None) != _abi.OK
    assert "overlaps" not in msg(), msg()
    # load: records written
    assert L.ark_ckpt_load(b"/nonexistent", overlapping, 2, None, None, None) == _abi.EINVAL
    assert "overlaps" in msg(), msg()


def test_pack_plan_rejects_bad_arguments_before_device_calls():
    """The pack plan checks its arguments as ark_ckpt_v4_pack does (the
    image's size with or without the trailer, its alignment, overlap with a
    record) before any device query, and its run refuses a NULL plan and an
    AMP state that does not match the plan (the addresses are not memory)."""
    L = _lib.lib()
    msg = lambda: L.ark_opt_last_error().decode()
    arr = (_abi.CkptRecord * 2)()
    arr[0] = _abi.CkptRecord(1 * MB, 1000, _abi.CKPT_F16, 0)
    arr[1] = _abi.CkptRecord(2 * MB, 1000, _abi.CKPT_F32, 0)
    size = 28 + 16 + 2000 + 16 + 4000
    h = C.c_void_p(12345)
    assert L.ark_ckpt_v4_pack_plan_create(arr, 2, 0, 8 * MB, size, None, None) == _abi.EINVAL
    assert "out is NULL" in msg(), msg()
    assert L.ark_ckpt_v4_pack_plan_create(arr, 2, 0, 8 * MB, size - 1, None,
                                          C.byref(h)) == _abi.EINVAL
    assert "needs %d" % size in msg() and h.value is None, msg()
    assert L.ark_ckpt_v4_pack_plan_create(arr, 2, 1, 8 * MB, size, None,
                                          C.byref(h)) == _abi.EINVAL
    assert "needs %d" % (size + 40) in msg(), msg()
    assert L.ark_ckpt_v4_pack_plan_create(arr, 2, 0, 8 * MB + 8, size, None,
                                          C.byref(h)) == _abi.EINVAL
    assert "16-byte aligned" in msg(), msg()
    assert L.ark_ckpt_v4_pack_plan_create(arr, 2, 0, 1 * MB + 512, size, None,
                                          C.byref(h)) == _abi.EINVAL
    assert "record 0 data overlaps the image" in msg(), msg()
    assert L.ark_ckpt_v4_pack_plan_create(None, 2, 0, 8 * MB, size, None,
                                          C.byref(h)) == _abi.EINVAL
    assert L.ark_ckpt_v4_pack_plan_run(None, 0, 0, None) == _abi.EINVAL
    assert "plan is NULL" in msg(), msg()
    assert L.ark_ckpt_plan_destroy(None) == _abi.OK


def test_missing_library_fails_loudly(tmp_path):
    """No fallback path: with the library absent, the loader and the entry
    points above it raise, naming the missing file (run in a fresh process so
    this process's loaded library is untouched)."""
    import subprocess
    import sys
    missing = str(tmp_path / "libark_opt.so")
    code = (
        "import sys\n"
        "from ark_amd import _lib, ckpt\n"
        "_lib.LIB_PATH = sys.argv[1]\n"
        "_lib._lib = None\n"
        "for f in (_lib.lib, lambda: ckpt.probe(sys.argv[1]), lambda: _lib.check(-1)):\n"
        "    try:\n"
        "        f()\n"
        "    except ImportError as e:\n"
        "        assert sys.argv[1] in str(e), e\n"
        "    else:\n"
        "        raise SystemExit('no error')\n"
        "print('ok')\n")
    r = subprocess.run([sys.executable, "-c", code, missing], cwd=ROOT, capture_output=True,
                       text=True, timeout=300)
    assert r.returncode == 0 and r.stdout.strip() == "ok", r.stdout + r.stderr
