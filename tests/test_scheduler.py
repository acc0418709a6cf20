"""Share scheduler (scope_amd/scheduler.py): the roofline model's balance
point, capacity cap, choice and calibration, checked against brute force over
r and against closed forms."""
import numpy as np
import pytest

from scope_amd.scheduler import ShareScheduler, Side, fit_side


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
