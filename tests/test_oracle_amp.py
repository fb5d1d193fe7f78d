"""Pins of the oracle's AMP loss-scale state machine (training.rs:10-13,
:228-241, :289-326) by known answers and by the reference's own logged
trajectory (index.html:374, extracted to tests/golden/)."""
import ctypes as C
import json
import os

import numpy as np

import oracle
from ark_amd import _abi

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "amp_trajectory_index_html.json")


def _hp(**kw):
    hp = oracle.default_hparams()
    for k, v in kw.items():
        setattr(hp, k, v)
    return hp


def _state(hp):
    st = _abi.State()
    oracle.lib().ark_ref_state_init(C.byref(hp), C.byref(st))
    return st


def test_defaults_match_reference_constants():
    """LOSS_SCALE_INIT 256, MIN 1, SCALE_UP_EVERY 2000 (training.rs:10-13);
    loss_scale_max 8192 (config.rs:69); AdamConfig::default betas/eps/clip
    (optimizer.rs:54-66); and the library's defaults agree."""
    from ark_amd._lib import lib
    hp = _abi.HParams()
    lib().ark_opt_default_hparams(C.byref(hp))
    ref = oracle.default_hparams()
    for k, _ in _abi.HParams._fields_:
        assert getattr(hp, k) == getattr(ref, k), k
    assert _state(hp).loss_scale == 256.0


def test_growth_exactly_every_2000_clean_steps():
    hp = _hp()
    st = _state(hp)
    _, sc = oracle.amp_replay(hp, st, np.zeros(9000, bool))
    # scale after applied step k (1-based) = min(256 * 2^(k // 2000), 8192)
    k = np.arange(1, 9001)
    assert np.array_equal(sc, np.minimum(256.0 * 2.0 ** (k // 2000), 8192.0).astype(np.float32))
    assert st.t == 9000 and st.clean_steps == 9000 % 2000


def test_cap_resets_counter_and_never_exceeds_max():
    """training.rs:319-326: at the cap min(2S, max) == S, the scale stays and
    clean_steps still resets (Q4)."""
    hp = _hp(loss_scale_init=4096.0)
    st = _state(hp)
    _, sc = oracle.amp_replay(hp, st, np.zeros(6001, bool))
    assert sc.max() == 8192.0 and sc[1999] == 8192.0 and sc[-1] == 8192.0
    assert st.clean_steps == 1


def test_config3_start_above_default_cap_never_grows():
    """Configuration c3 starts at 65536 > the default cap 8192: min(2S, max) < S,
    so the scale never grows (Q3) until loss_scale_max is raised."""
    hp = _hp(loss_scale_init=65536.0)
    st = _state(hp)
    _, sc = oracle.amp_replay(hp, st, np.zeros(5000, bool))
    assert np.all(sc == 65536.0)
    hp = _hp(loss_scale_init=65536.0, loss_scale_max=2.0 ** 24)
    st = _state(hp)
    _, sc = oracle.amp_replay(hp, st, np.zeros(5000, bool))
    assert sc[1998] == 65536.0 and sc[1999] == 131072.0 and sc[3999] == 262144.0


def test_skip_halves_floors_and_keeps_t():
    hp = _hp(loss_scale_init=8.0)
    st = _state(hp)
    ev = np.array([0, 0, 1, 1, 1, 1, 1, 0], bool)
    _, sc = oracle.amp_replay(hp, st, ev)
    assert sc.tolist() == [8, 8, 4, 2, 1, 1, 1, 1]  # floor LOSS_SCALE_MIN = 1
    assert st.t == 3 and st.skipped_steps == 5 and st.consecutive_nonfinite == 0


def test_skip_resets_clean_counter():
    hp = _hp()
    st = _state(hp)
    ev = np.zeros(4100, bool)
    ev[1500] = True  # a skip after 1500 clean steps restarts the count
    _, sc = oracle.amp_replay(hp, st, ev)
    assert sc[1499] == 256.0 and sc[1500] == 128.0
    # growth 2000 applied steps after the skip (indices 1501..3500)
    assert sc[3499] == 128.0 and sc[3500] == 256.0


def test_early_stop_after_more_than_200_consecutive():
    """training.rs:298-301: the 201st consecutive skip stops; later calls
    keep reporting it and change nothing."""
    hp = _hp()
    st = _state(hp)
    rc, _ = oracle.amp_replay(hp, st, np.ones(200, bool))
    assert rc == _abi.OK and st.early_stop == 0
    rc, _ = oracle.amp_replay(hp, st, np.ones(1, bool))
    assert rc == _abi.EARLY_STOP and st.early_stop == 1 and st.skipped_steps == 201
    rc, _ = oracle.amp_replay(hp, st, np.zeros(5, bool))
    assert rc == _abi.EARLY_STOP and st.t == 0 and st.skipped_steps == 201


def test_record_overflow_is_the_same_skip():
    hp = _hp()
    a, b = _state(hp), _state(hp)
    info = _abi.StepInfo()
    for _ in range(3):
        oracle.lib().ark_ref_record_overflow(C.byref(hp), C.byref(a), C.byref(info))
    oracle.amp_replay(hp, b, np.ones(3, bool))
    assert a.as_dict() == b.as_dict()


def test_replay_matches_full_steps():
    """ark_ref_amp_replay and ark_ref_opt_step share the bookkeeping: a run
    of full steps over real gradients with injected infs equals the replay
    of its outcomes."""
    rng = np.random.default_rng(3)
    n = 64
    g = np.zeros(n, np.uint16)
    t = oracle.HostTensor(np.zeros(n, np.uint16), g, np.zeros(n, np.float32),
                          np.zeros(n, np.float32), 0.1)
    hp = _hp(scale_up_every=7, loss_scale_init=64.0, max_consecutive_nonfinite=4)
    opt = oracle.Optimizer([t], hp)
    ref = _state(hp)
    outcomes = rng.random(400) < 0.15
    for bad in outcomes:
        g[:] = oracle.f32_to_f16(rng.standard_normal(n).astype(np.float32))
        if bad:
            g[rng.integers(n)] = 0x7C00
        rc, _ = opt.step(1e-3)
        rrc, _ = oracle.amp_replay(hp, ref, np.array([bad]))
        assert rc == rrc
        assert opt.state.as_dict() == ref.as_dict()


def _segments(rows):
    """Split the logged rows into training runs, as (base, rows) with base the
    checkpoint step R the run resumed from.  A run restarts the AMP state at
    LOSS_SCALE_INIT (training.rs:120; the scale is not checkpointed) and logs
    at local steps 1, 100, 200, ... (training.rs:444).  A restart shows as a
    row off the 100-step grid of the current run, a drop of the cumulative
    skip count, or a drop of the scale with no new skip; in the last case the
    local-step-1 row is missing from the dashboard and the run resumed from
    the last 500-step checkpoint (training.rs:454-456) before the row."""
    segs = []
    for step, scale, skips in rows:
        if segs:
            base, seg = segs[-1]
            prev = seg[-1]
            on_grid = (step - base) % 100 == 0
            if on_grid and skips >= prev[2] and not (scale < prev[1] and skips == prev[2]):
                seg.append((step, scale, skips))
                continue
            if on_grid:  # restart whose local-step-1 row is missing
                segs.append(((step - 1) // 500 * 500, [(step, scale, skips)]))
                continue
        segs.append((step - 1, [(step, scale, skips)]))  # this row is local step 1
    return segs


def test_reference_trajectory_growth_cadence_and_cap():
    """Every logged scale of the reference's training runs without skips is
    reproduced by replaying clean steps from LOSS_SCALE_INIT with the default
    cap 8192: doubling exactly every 2000 applied steps, capped."""
    rows = json.load(open(GOLDEN))["rows"]
    segs = _segments(rows)
    assert sum(len(s) for _, s in segs) == len(rows)
    checked = 0
    for base, seg in segs:
        clean = [r for r in seg if r[2] == 0]
        k_max = clean[-1][0] - base
        hp = _hp()
        st = _state(hp)
        _, sc = oracle.amp_replay(hp, st, np.zeros(k_max, bool))
        for step, scale, _ in clean:
            assert sc[step - base - 1] == scale, (base, step)
            checked += 1
    assert checked == 4429  # every row not preceded by a skip in its run


def test_reference_trajectory_skip_events_are_explained():
    """The one run with skips (restart at 432650) logs a halving 8192 -> 4096
    with skips 0 -> 1 between local steps 10200 and 10300 and 4096 -> 2048
    with skips 1 -> 2 between 12200 and 12300.  A brute-force search over
    where each skip fell finds placements under which the oracle's state
    machine reproduces every later logged scale, including the regrowth to
    4096 and 8192; placements a whole interval off do not fit."""
    rows = json.load(open(GOLDEN))["rows"]
    base, seg = _segments(rows)[-1]
    assert base == 432650
    last = seg[-1][0] - base
    logged = {step - base: scale for step, scale, _ in seg}
    skip_rows = [(a[0] - base, b[0] - base) for a, b in zip(seg, seg[1:]) if b[2] > a[2]]
    assert skip_rows == [(10200, 10300), (12200, 12300)]

    def fits(p1, p2):
        # p: number of applied steps before the skip
        ev = np.zeros(last + 2, bool)
        ev[p1] = True
        ev[p2 + 1] = True
        hp = _hp()
        st = _state(hp)
        _, sc = oracle.amp_replay(hp, st, ev)
        applied = np.cumsum(~ev)
        for k, scale in logged.items():
            i = int(np.searchsorted(applied, k))  # index of the k-th applied step
            if sc[i] != scale:
                return False
        return True

    ok = [(p1, p2) for p1 in range(10200, 10300, 7) for p2 in range(12200, 12300, 7)
          if fits(p1, p2)]
    assert ok, "no skip placement reproduces the logged trajectory"
    assert not fits(8000, 12250) and not fits(10250, 14000)
