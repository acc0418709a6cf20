"""Share scheduler (scope_amd/scheduler.py): the roofline model's balance
point, capacity cap, choice and calibration, checked against brute force over
r and against closed forms."""
import numpy as np
import pytest

from scope_amd.scheduler import ShareController, ShareScheduler, Side, fit_side


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
