"""Share scheduler (scope_amd/scheduler.py): the roofline model's balance
point, capacity cap, choice and calibration, checked against brute force over
r and against closed forms."""
import numpy as np
import pytest

from scope_amd.scheduler import (ShareController, ShareScheduler, Side, fit_side,
                                 fit_side_report)


def _sched(**kw):
    return ShareScheduler(gpu=Side(20e-6, 6.0e12), host=Side(60e-6, 130e9), **kw)


def test_balance_point_equalises_the_two_sides():
    s = _sched()
    for W in (1e6, 5e7, 3e8, 2e9):
        r = s.balance_share(W)
        t = s.predict(r, W) if r < 1 else None
        if 0 < r < 1:
            assert t["gpu"] == pytest.approx(t["host"], rel=1e-9)


def test_choice_is_the_brute_force_minimum():
    for budget in (None, 1e9, 5e9, 2e10):
        s = _sched(hbm_budget_bytes=budget)
        for W in (1e6, 3e7, 3e8, 1e9):
            for layers in (1, 27):
                r = s.choose(W, layers)
                cap = s.capacity_share(W, layers)
                assert 0.0 <= r <= cap + 1e-12
                grid = np.linspace(0.0, cap, 2001)
                best = min(s.predict(float(x), W)["layer"] for x in grid)
                assert s.predict(r, W)["layer"] <= best + 1e-12


def test_all_in_hbm_when_it_fits_and_capacity_bound_otherwise():
    s = _sched(hbm_budget_bytes=8e9)
    W = 2.5e8  # 27 layers: 6.75 GB, fits
    assert s.choose(W, 27) == 1.0
    W = 1e9    # 27 GB does not fit: r is the capacity share
    assert s.choose(W, 27) == pytest.approx(8e9 / 27e9)


def test_slow_host_moves_balance_towards_the_gpu():
    fast = ShareScheduler(gpu=Side(0, 6e12), host=Side(0, 6e12), xfer_s=0)
    assert fast.balance_share(1e9) == pytest.approx(0.5)
    slow = ShareScheduler(gpu=Side(0, 6e12), host=Side(0, 6e10), xfer_s=0)
    assert slow.balance_share(1e9) == pytest.approx(6e12 / (6e12 + 6e10))


def test_granularity_rounds_down_within_capacity():
    s = _sched(hbm_budget_bytes=2.9e9)   # capacity share 0.725
    r = s.choose(1e9, 4, granularity=0.125)
    assert r == pytest.approx(0.625)      # largest multiple of 0.125 below 0.725
    assert r <= s.capacity_share(1e9, 4)
    s = _sched(hbm_budget_bytes=3e9)     # capacity share 0.75 is on the grid
    assert s.choose(1e9, 4, granularity=0.125) == pytest.approx(0.75)


# A measured share sweep of the 27-layer DeepSeek-V2-Lite decode (B 32,
# lognormal lengths, 16 host threads) on one MI355X box: tokens on each side
# and the per-layer times of each partial and of the whole layer, at shares
# 0.1, 0.3, 0.5, 0.7, 0.9 and 1.0.  Its r = 0.1 point is slow on both sides:
# the GPU partial (30 MB in 37.9 us, 790 GB/s) ran on clocks that dropped
# while the GPU waited ~3 ms per layer for the host, and the host partial ran
# at 94 GB/s against 139-151 GB/s at the neighbouring shares.
SWEEP_GPU_TOKENS = [26008, 78052, 130105, 182142, 234186, 260221]
SWEEP_GPU_US = [37.9, 26.9, 36.2, 45.8, 54.9, 59.5]
SWEEP_HOST_TOKENS = [234213, 182169, 130116, 78079, 26035]
SWEEP_HOST_US = [2876.2, 1393.6, 1019.2, 647.7, 276.1]
SWEEP_LAYER_US = [3129.4, 1455.4, 1075.7, 698.6, 325.8, 68.7]
SWEEP_SHARES = [0.1, 0.3, 0.5, 0.7, 0.9, 1.0]
SWEEP_HOST_READ_GBS = 202.2


def test_bounded_fit_of_a_measured_sweep_stays_physical():
    """The plain least-squares fit of the sweep's GPU points gives a rate
    above the 8 TB/s HBM peak (9.8 TB/s); the bounded, outlier-robust fit
    leaves the r = 0.1 points out, keeps both rates below their physical
    bounds and predicts every other share's layer time within 10%."""
    gpts = [(t * 1152.0, u * 1e-6) for t, u in zip(SWEEP_GPU_TOKENS, SWEEP_GPU_US)]
    hpts = [(t * 1152.0, u * 1e-6) for t, u in zip(SWEEP_HOST_TOKENS, SWEEP_HOST_US)]
    assert fit_side(gpts).rate_bps > 8e12  # the unbounded fit is unphysical
    g = fit_side_report(gpts, max_rate_bps=8e12, reject_rel=0.15)
    h = fit_side_report(hpts, max_rate_bps=SWEEP_HOST_READ_GBS * 1e9, reject_rel=0.15)
    assert g.side.rate_bps <= 8e12 and h.side.rate_bps <= SWEEP_HOST_READ_GBS * 1e9
    assert g.rejected == [gpts[0]] and h.rejected == [hpts[0]]
    assert 6.0e12 < g.side.rate_bps < 7.0e12 and 150e9 < h.side.rate_bps < 170e9
    resid = [m - max(a, b) for m, a, b in zip(SWEEP_LAYER_US, SWEEP_GPU_US, SWEEP_HOST_US)]
    sched = ShareScheduler(gpu=g.side, host=h.side, xfer_s=float(np.median(resid)) * 1e-6,
                           merge_s=0.0,
                           merge_gpu_only_s=(SWEEP_LAYER_US[-1] - SWEEP_GPU_US[-1]) * 1e-6)
    W = sum(SWEEP_GPU_TOKENS[-1:]) * 1152.0
    for r, m in zip(SWEEP_SHARES[1:], SWEEP_LAYER_US[1:]):
        assert abs(sched.predict(r, W)["layer"] * 1e6 / m - 1.0) < 0.10, r


def test_bounded_fit_caps_the_rate_and_floors_the_intercept():
    # points on a line steeper than the cap: the rate is the cap, the
    # intercept the median residual
    true = Side(5e-6, 10e12)
    pts = [(b, true.time(b)) for b in (1e8, 2e8, 4e8, 8e8)]
    r = fit_side_report(pts, max_rate_bps=8e12)
    assert r.rate_capped and r.side.rate_bps == pytest.approx(8e12)
    assert r.side.max_rate_bps == 8e12
    # a negative least-squares intercept is floored and the slope refitted
    pts = [(1e8, 10e-6), (2e8, 30e-6), (3e8, 50e-6)]
    r = fit_side_report(pts, min_fixed_s=2e-6)
    assert r.side.fixed_s == pytest.approx(2e-6)
    assert r.side.time(2e8) == pytest.approx(30e-6, rel=0.15)
    # an online update cannot take a bounded side above its bound
    s = ShareScheduler(gpu=Side(0.0, 6e12, max_rate_bps=8e12), host=Side(0, 1e11))
    for _ in range(50):
        s.observe("gpu", 1e9, 1e9 / 20e12)
    assert s.gpu.rate_bps <= 8e12
    # with three points nothing is rejected; clean points are all kept
    clean = [(b, Side(1e-5, 5e12).time(b)) for b in (1e8, 2e8, 3e8, 5e8, 8e8)]
    assert fit_side_report(clean, reject_rel=0.05).rejected == []
    assert fit_side_report(pts, reject_rel=0.01).rejected == []


def test_fit_recovers_affine_sides_and_ema_tracks_rate():
    true = Side(25e-6, 5.5e12)
    pts = [(b, true.time(b)) for b in (1e8, 3e8, 6e8, 1.2e9)]
    f = fit_side(pts)
    assert f.fixed_s == pytest.approx(25e-6, rel=1e-6)
    assert f.rate_bps == pytest.approx(5.5e12, rel=1e-6)
    s = ShareScheduler(gpu=Side(25e-6, 1e12), host=Side(0, 1e11))
    for _ in range(60):
        s.observe("gpu", 5e8, true.time(5e8))
    assert s.gpu.rate_bps == pytest.approx(5.5e12, rel=1e-3)
    with pytest.raises(ValueError):
        fit_side([(1e8, 1e-3)])
    with pytest.raises(ValueError):
        s.predict(1.5, 1e8)


def _simulate(ctl, lens, host, steps, bw_g=6e12, bw_h=100e9, fixed_g=15e-6, fixed_h=40e-6,
              bpt=1152):
    """Decode loop of a modelled two-sided cache: per layer the sides take
    fixed + bytes / rate; lengths grow by one token a step (on the GPU side);
    moves apply the controller's targets."""
    lens = list(lens)
    host = list(host)
    trace = []
    for _ in range(steps):
        for _l in range(ctl.layers):
            g_tok = sum(L - h for L, h in zip(lens, host))
            h_tok = sum(host)
            ctl.observe_layer(g_tok * bpt, fixed_g + g_tok * bpt / bw_g, h_tok * bpt,
                              (fixed_h + h_tok * bpt / bw_h) if h_tok else 0.0)
        lens = [L + 1 for L in lens]
        t = ctl.decide(lens, host)
        if t is not None:
            ctl.record_move(ctl.share_of(lens, host), ctl.share_of(lens, t),
                            sum(abs(a - b) for a, b in zip(t, host)) // ctl.page_size, 0.0)
            host = t
        trace.append(ctl.share_of(lens, host))
    return lens, host, trace


def test_controller_converges_to_the_hbm_budget_and_holds():
    """A cache twice the HBM budget, starting at r = 0.1 (a host-heavy split):
    the first decision moves to the capacity share, later steps move only when
    growth shifts it by a page per sequence, and the share never exceeds the
    budget."""
    rng = np.random.default_rng(5)
    lens = [int(x) for x in np.clip(rng.lognormal(np.log(4096), 1.0, 32), 256, 65536)]
    layers, bpt, ps = 27, 1152, 64
    W = sum(lens) * bpt
    budget = 0.5 * W * layers
    # fixed costs as modelled, rates off by 1.5x / 2x: the EMA must find them
    sched = ShareScheduler(gpu=Side(15e-6, 4e12), host=Side(40e-6, 50e9), xfer_s=30e-6,
                           hbm_budget_bytes=budget)
    ctl = ShareController(sched, bpt, layers, ps)
    host0 = ctl.targets_for(0.1, lens)
    lens_end, host_end, trace = _simulate(ctl, lens, host0, steps=40)
    # first decision: to the capacity share (within a page per sequence)
    assert ctl.moves and ctl.moves[0].step == 1
    assert abs(ctl.moves[0].share_to - 0.5) < 0.01
    assert abs(trace[0] - 0.5) < 0.01
    # then it holds: no move while growth shifts the boundary by less than a
    # page per sequence, and the GPU side never exceeds the budget
    assert len(ctl.moves) <= 2
    for r, n in zip(trace, range(1, 41)):
        W_n = sum(L + n for L in lens) * bpt
        assert r <= sched.capacity_share(W_n, layers) + 1e-9
    # the EMA learned the modelled rates (fixed costs are the scheduler's)
    assert abs(sched.gpu.rate_bps / 6e12 - 1) < 0.02
    assert abs(sched.host.rate_bps / 100e9 - 1) < 0.02


def test_controller_without_budget_goes_all_gpu_and_stops_moving():
    lens = [3000, 5000, 700]
    sched = ShareScheduler(gpu=Side(10e-6, 6e12), host=Side(10e-6, 100e9))
    ctl = ShareController(sched, 4096, 32, 64)
    _, host, trace = _simulate(ctl, lens, ctl.targets_for(0.25, lens), steps=5, bpt=4096)
    assert host == [0, 0, 0] and trace[-1] == 1.0
    assert len(ctl.moves) == 1 and all(c == 1.0 for c in ctl.chosen)


def test_controller_hysteresis_ignores_sub_page_moves():
    lens = [4096] * 8
    # budget just above the current GPU side: the capacity share differs from
    # the current one by less than a page per sequence
    sched = ShareScheduler(gpu=Side(10e-6, 6e12), host=Side(10e-6, 100e9),
                           hbm_budget_bytes=0.5 * sum(lens) * 1152 * 4 + 10 * 1152 * 4)
    ctl = ShareController(sched, 1152, 4, 64)
    host = ctl.targets_for(0.5, lens)
    assert ctl.decide(lens, host) is None
    assert ctl.moves == [] and ctl.shares == [0.5]
    # once appends push the GPU side over the budget, it must move (a page
    # per sequence, rounding the host side up), however small the move
    lens2 = [L + 3 for L in lens]
    t = ctl.decide(lens2, host)
    assert t == [2112] * 8 and ctl.shares[-1] <= 0.5


def test_controller_records_but_does_not_move_while_a_move_is_in_flight():
    lens = [3000, 5000, 700]
    sched = ShareScheduler(gpu=Side(10e-6, 6e12), host=Side(10e-6, 100e9))
    ctl = ShareController(sched, 4096, 32, 64)
    host = ctl.targets_for(0.25, lens)
    assert ctl.decide(lens, host, moving=True) is None     # would move to r = 1 otherwise
    assert ctl.steps == 1 and ctl.chosen == [1.0]
    assert ctl.shares == [ctl.share_of(lens, host)]       # the current boundaries
    assert ctl.decide(lens, host) == [0, 0, 0]
    # a move the cache ran under later steps: its own step, wall and stall times
    ctl.record_move(0.25, 1.0, 40, 0.07, stall_seconds=0.008, step=1, copy_seconds=0.056)
    m = ctl.moves[-1]
    assert (m.step, m.seconds, m.stall_seconds, m.copy_seconds) == (1, 0.07, 0.008, 0.056)
    ctl.record_move(1.0, 0.5, 10, 0.02)                   # waited for: all of it is stall
    m = ctl.moves[-1]
    assert m.step == 2 and m.stall_seconds == m.copy_seconds == 0.02
