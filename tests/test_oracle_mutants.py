"""The oracle's pins catch plausible mistakes.  Each mutant is a copy of
oracle/ark_oracle.c, or of the checkpoint format's oracle/ckpt.py, with one
planted error -- a swapped or dropped operand, a wrong sign, comparison,
constant or index, a rounding shortcut.  The C mutants are compiled on the
CPU with the oracle's own flags.  The pin tests named beside each mutant must
fail against it.  Those pins are the independent checks: the second
restatement in Python with an exact-rational fma, closed forms, exhaustive
conversions against F16C and numpy, brute force on small inputs, the
reference's own loss-scale trajectory, and a checkpoint file typed byte by
byte from the format.  Self-consistency checks (the vectorised loops against
the scalar ones, fixtures the oracle wrote) are not run here.  An unmutated
copy built the same way must pass them."""
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "oracle", "ark_oracle.c")
CFLAGS = ["-O2", "-std=c11", "-fPIC", "-ffp-contract=off", "-fno-math-errno", "-mfma",
          "-mf16c", "-mavx2", "-pthread", "-shared"]

# name: (text in ark_oracle.c, planted replacement, pin files tests/test_oracle_<x>.py)
MUTANTS = {
    # AdamW element update and prologue (opti.s:210-308)
    "first_moment_takes_beta2": ('float mm = *m * beta1;             /* fmul v1, v1, v16     :286 */',
        'float mm = *m * beta2;             /* fmul v1, v1, v16     :286 */', ["adam"]),
    "second_moment_drops_the_square": ('vv = fmaf(s->c2, gg, vv);          /* fmla v2, v19, v4     :293 */',
        'vv = fmaf(s->c2, g, vv);          /* fmla v2, v19, v4     :293 */', ["adam"]),
    "first_moment_not_fused": ('mm = fmaf(s->c1, g, mm);           /* fmla v1, v18, v0     :287 */',
        'mm = s->c1 * g + mm;           /* fmla v1, v18, v0     :287 */', ["adam"]),
    "eps_inside_the_root": ('d = d + eps;                       /* fadd v5, v5, v20     :298 */',
        'd = sqrtf(vv + eps);                       /* fadd v5, v5, v20     :298 */', ["adam"]),
    "update_not_scaled": ('u = u * s->lr_eff;                 /* fmul v6, v6, v21     :300 */',
        'u = u * s->c1;                 /* fmul v6, v6, v21     :300 */', ["adam"]),
    "decay_sign": ("out->decay = 1.0f - lw;", "out->decay = 1.0f + lw;", ["adam"]),
    "bias_correction_without_root": ("float r = sqrtf(out->bc2);", "float r = out->bc2;",
                                     ["adam"]),
    "t0_not_coerced": ("if (t == 0) t = 1;", "if (t == 0) t = 0;", ["adam"]),
    # the fp32-weight element (opti.s:105-131)
    "fp32_weight_decay_skipped": ('w = w * s->decay;                  /* fmul v3, v3, v22     :128 */',
        'w = w * 1.0f;                  /* fmul v3, v3, v22     :128 */', ["adam"]),
    "fp32_first_moment_not_fused": ('mm = fmaf(s->c1, g, mm);           /* fmla v1, v18, v0     :115 */',
        'mm = s->c1 * g + mm;           /* fmla v1, v18, v0     :115 */', ["adam"]),
    "power_multiplies_beta": ("if (k & 1u) res = res * base;", "if (k & 1u) res = res * beta;",
                              ["adam"]),
    # norm and finite flag (optimizer.rs:127-145, training.rs:291)
    "norm_not_unscaled": ("float gu = grad_f32(T->g, c->dtype, st + j) * inv_t;",
                          "float gu = grad_f32(T->g, c->dtype, st + j);", ["norm"]),
    "tree_pairs_strided": ("for (uint64_t i = 0; i < w; ++i) b[i] = b[2 * i] + b[2 * i + 1];",
                           "for (uint64_t i = 0; i < w; ++i) b[i] = b[i] + b[i + w];", ["norm"]),
    "finite_flag_misses_infinity": ("return (((const uint16_t *)g)[i] & 0x7C00u) == 0x7C00u;",
                                    "return (((const uint16_t *)g)[i] & 0x7E00u) == 0x7E00u;",
                                    ["norm"]),
    # clip (optimizer.rs:145-165)
    "clip_at_equality": ("int clipped = (norm > hp->grad_clip) && (norm > 0.0f);",
                         "int clipped = (norm >= hp->grad_clip) && (norm > 0.0f);", ["clip"]),
    "clip_coefficient_inverted": ("float coef = clipped ? hp->grad_clip / norm : 1.0f;",
                                  "float coef = clipped ? norm / hp->grad_clip : 1.0f;", ["clip"]),
    # AMP state machine (training.rs:293-326)
    "skip_does_not_halve": ("float s = st->loss_scale * 0.5f;", "float s = st->loss_scale;",
                            ["amp"]),
    "growth_one_step_late": ("if (st->clean_steps >= hp->scale_up_every) {",
                             "if (st->clean_steps > hp->scale_up_every) {", ["amp"]),
    "capped_growth_keeps_counting": ("    st->clean_steps = 0;                                   /* :325 */",
                                     "    if (nueva > scale) st->clean_steps = 0;", ["amp"]),
    "early_stop_at_200": ("if (st->consecutive_nonfinite > hp->max_consecutive_nonfinite) {",
                          "if (st->consecutive_nonfinite >= hp->max_consecutive_nonfinite) {",
                          ["amp"]),
    # fp16 conversions (opti.s:279, :307)
    "narrowing_ties_round_down": ("if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u;",
                                  "if (rem > 0x1000u) h += 1u;", ["fp16"]),
    "widening_subnormal_unit": ("float mag = (float)mant * 5.9604644775390625e-08f;",
                                "float mag = (float)mant * 1.1920928955078125e-07f;", ["fp16"]),
    # gradient hand-off (bridge.m:922-928)
    "out_of_range_token_to_last_row": ("uint32_t t = (tokens[i] < vocab) ? tokens[i] : 0;",
                                       "uint32_t t = (tokens[i] < vocab) ? tokens[i] : vocab - 1;",
                                       ["grad"]),
    "scatter_in_reverse": ("for (uint32_t i = 0; i < batch_seq; ++i) {",
                           "for (uint32_t i = batch_seq; i-- > 0;) {", ["grad"]),
    # per-tensor clip (opti.s:369-432)
    "grad_clip_at_equality": ("if (!(norm > thr)) return;", "if (!(norm >= thr)) return;",
                              ["grad_clip"]),
    "grad_clip_coefficient_inverted": ("const float c = thr / norm;",
                                       "const float c = norm / thr;", ["grad_clip"]),
    "grad_clip_pairs_folded_in_order": ("float s = (acc[0] + acc[1]) + (acc[2] + acc[3]);",
                                        "float s = ((acc[0] + acc[1]) + acc[2]) + acc[3];",
                                        ["grad_clip"]),
    "grad_clip_tail_unfused": ("for (; i < n; ++i) s = fmaf(g[i], g[i], s);",
                               "for (; i < n; ++i) s = g[i] * g[i] + s;", ["grad_clip"]),
    "grad_clip_norm_in_f64": ("const float norm = sqrtf((float)sum);",
                              "const float norm = (float)sqrt(sum);", ["grad_clip"]),
}
PINS = sorted({f for _, _, files in MUTANTS.values() for f in files})

# The checkpoint format's restatement (oracle/ckpt.py, io.rs:432-671), pinned
# by tests/test_oracle_ckpt.py (a known-answer file typed byte by byte from
# the format, the loader's regrouping rules, V3/V2 layouts, failures).
CKPT = os.path.join(ROOT, "oracle", "ckpt.py")
CKPT_MUTANTS = {
    "magic_in_reading_order": ("MAGIC_V4 = 0x4B345241", "MAGIC_V4 = 0x41524B34"),
    "header_steps_swapped": ("MAGIC_V4, global_step, adam_step, n_tensors)]",
                             "MAGIC_V4, adam_step, global_step, n_tensors)]"),
    "f16_record_tagged_f32": ('return struct.pack("<QQ", d.size, 0)',
                              'return struct.pack("<QQ", d.size, 1)'),
    "gamma_final_moments_swapped": ("_rec_f32(gamma_f_m_f32), _rec_f32(gamma_f_v_f32)]",
                                    "_rec_f32(gamma_f_v_f32), _rec_f32(gamma_f_m_f32)]"),
    "unknown_type_read_as_f16": ("if version == 4 and tipo == 0:", "if version == 4 and tipo != 1:"),
    "gamma_final_test": ("has_gamma_final = (n_tensors - 3) % 27 == 3",
                         "has_gamma_final = (n_tensors - 3) % 27 == 0"),
    "layer_m_slice": ("m += rem[base + 9:base + 18]", "m += rem[base + 8:base + 17]"),
}

_CKPT_DRIVER = """
import importlib.util, sys
sys.path.insert(0, {root!r})
import oracle
spec = importlib.util.spec_from_file_location("oracle.ckpt", {mutant!r})
mod = importlib.util.module_from_spec(spec)
sys.modules["oracle.ckpt"] = mod
spec.loader.exec_module(mod)
oracle.ckpt = mod
import pytest
sys.exit(pytest.main(["-q", "-x", "-p", "no:cacheprovider", "-m", "not gpu", {test!r}]))
"""


def _run_ckpt_mutant(tmp, name, old, new):
    src = open(CKPT).read()
    if old is not None:
        assert src.count(old) == 1, f"{name}: the text to mutate is not in oracle/ckpt.py once"
        src = src.replace(old, new)
    path = os.path.join(tmp, f"ckpt_{name}.py")
    with open(path, "w") as f:
        f.write(src)
    code = _CKPT_DRIVER.format(root=ROOT, mutant=path,
                               test=os.path.join(ROOT, "tests", "test_oracle_ckpt.py"))
    r = subprocess.run([sys.executable, "-c", code], cwd=ROOT, capture_output=True, text=True,
                       timeout=600)
    return r.returncode, (r.stdout + r.stderr)[-1500:]


def _build_and_run(tmp, name, old, new, files):
    """Build ark_oracle.c with `old` replaced by `new` (None: unchanged) and
    run the pin files against it; returns (pytest exit code, output tail)."""
    src = open(SRC).read()
    if old is not None:
        assert src.count(old) == 1, f"{name}: the text to mutate is not in ark_oracle.c once"
        src = src.replace(old, new)
    d = os.path.join(tmp, name)
    os.makedirs(os.path.join(d, "oracle"))
    os.symlink(os.path.join(ROOT, "include"), os.path.join(d, "include"))
    shutil.copy(os.path.join(ROOT, "oracle", "ark_oracle.h"), os.path.join(d, "oracle"))
    with open(os.path.join(d, "oracle", "ark_oracle.c"), "w") as f:
        f.write(src)
    so = os.path.join(d, "libark_oracle.so")
    cc = subprocess.run(["gcc", *CFLAGS, "-o", so, os.path.join(d, "oracle", "ark_oracle.c"),
                         "-lm"], capture_output=True, text=True)
    assert cc.returncode == 0, f"{name}: build failed\n{cc.stderr[-2000:]}"
    env = dict(os.environ, ARK_ORACLE_LIB=so, OMP_NUM_THREADS="2")
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider",
                        "-m", "not gpu"] + [os.path.join(ROOT, "tests", f"test_oracle_{f}.py")
                                            for f in files],
                       cwd=ROOT, env=env, capture_output=True, text=True, timeout=600)
    return r.returncode, (r.stdout + r.stderr)[-1500:]


@pytest.fixture(scope="module")
def results(tmp_path_factory):
    tmp = str(tmp_path_factory.mktemp("mutants"))
    jobs = {"unmutated": (None, None, PINS)}
    jobs.update(MUTANTS)
    with ThreadPoolExecutor(max_workers=4) as ex:
        futs = {n: ex.submit(_build_and_run, tmp, n, *job) for n, job in jobs.items()}
        futs["ckpt:unmutated"] = ex.submit(_run_ckpt_mutant, tmp, "unmutated", None, None)
        for n, (old, new) in CKPT_MUTANTS.items():
            futs["ckpt:" + n] = ex.submit(_run_ckpt_mutant, tmp, n, old, new)
        return {n: f.result() for n, f in futs.items()}


def test_unmutated_copy_passes_the_pins(results):
    rc, out = results["unmutated"]
    assert rc == 0, out
    rc, out = results["ckpt:unmutated"]
    assert rc == 0, out


@pytest.mark.parametrize("name", sorted(MUTANTS))
def test_pins_catch_the_mutant(results, name):
    rc, out = results[name]
    assert rc == 1, f"{name}: pins {MUTANTS[name][2]} did not fail (exit {rc})\n{out}"


@pytest.mark.parametrize("name", sorted(CKPT_MUTANTS))
def test_pins_catch_the_checkpoint_mutant(results, name):
    rc, out = results["ckpt:" + name]
    assert rc == 1, f"{name}: tests/test_oracle_ckpt.py did not fail (exit {rc})\n{out}"
