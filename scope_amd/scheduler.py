"""Share scheduler: which fraction r of every sequence's KV lives in HBM.

The reference picks its split from calibrated tables (KV_LEN_GS_TABLE,
system/deepseek.py:127-142; batch/length ladders, system/qwenoffload.py:
1291-1327 and system/deepseek.py:846-864) and nudges it online with an EMA
toward the point where GPU and CPU finish together (system/qwenoffload.py:
1160-1165, system/mixoffload.py:1466-1474).  Here the choice comes from a
roofline model of the two partials that the same measurements calibrate:

  GPU partial   t_g(r) = a_g + r * W / bw_g        (HBM stream, W = KV bytes
                                                    of one layer, all sequences)
  host partial  t_h(r) = a_h + (1 - r) * W / bw_h  (host DRAM stream / AVX-512)
  transfers     t_x    = q to the host + the host partial back (PCIe latency
                         dominated; only when r < 1)
  layer         T(r) = max(t_g(r), t_h(r) + t_x) + t_m   for r < 1
                T(1) = t_g(1) + t_m1                      (no host partial)

T is minimised where the two sides meet, r_bal = (a_h + t_x - a_g + W/bw_h) /
(W/bw_g + W/bw_h), or at r = 1 when the whole cache fits, since the host side
then disappears.  HBM capacity caps r: r <= hbm_budget / (layers * W).  With
MI355X's HBM at ~6 TB/s against a host at ~0.1 TB/s, r_bal is above 0.97 for
every realistic W, so in practice the choice is "as much as fits": the host
partition exists for capacity, and its speed sets the step time once the
cache outgrows HBM.

Rates are tracked online with the reference's EMA form (new = (1 - w) * old
+ w * observed), per side, from (bytes, seconds) observations.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field


@dataclass
class Side:
    """Affine time model of one partial: seconds = fixed + bytes / rate.

    max_rate_bps, when set, is the side's physical bound (the HBM peak for
    the GPU partial, the measured host read bandwidth for the host partial):
    no fit or online update takes the rate above it."""
    fixed_s: float
    rate_bps: float
    max_rate_bps: float | None = None

    def time(self, nbytes: float) -> float:
        return self.fixed_s + nbytes / self.rate_bps

    def bounded(self, rate_bps: float) -> float:
        return rate_bps if self.max_rate_bps is None else min(rate_bps, self.max_rate_bps)


@dataclass
class ShareScheduler:
    gpu: Side
    host: Side
    xfer_s: float = 30e-6        # q to the host + partial back, per layer
    merge_s: float = 5e-6        # merge launch with a host partial
    merge_gpu_only_s: float = 5e-6
    hbm_budget_bytes: float | None = None
    ema_weight: float = 0.2
    history: list = field(default_factory=list)

    # ------------------------------------------------------------------ model

    def predict(self, r: float, layer_bytes: float) -> dict:
        """Per-layer times (seconds) at share r for a layer of layer_bytes KV."""
        if not 0.0 <= r <= 1.0:
            raise ValueError(f"share {r} outside [0, 1]")
        tg = self.gpu.time(r * layer_bytes)
        if r >= 1.0:
            return {"gpu": tg, "host": 0.0, "layer": tg + self.merge_gpu_only_s}
        th = self.host.time((1.0 - r) * layer_bytes) + self.xfer_s
        return {"gpu": tg, "host": th, "layer": max(tg, th) + self.merge_s}

    def balance_share(self, layer_bytes: float) -> float:
        """Share where the GPU partial and the host partial (+ transfers) take
        equally long, clamped to [0, 1]."""
        if layer_bytes <= 0:
            return 1.0
        wg = layer_bytes / self.gpu.rate_bps
        wh = layer_bytes / self.host.rate_bps
        r = (self.host.fixed_s + self.xfer_s - self.gpu.fixed_s + wh) / (wg + wh)
        return min(1.0, max(0.0, r))

    def capacity_share(self, layer_bytes: float, layers: int = 1) -> float:
        """Largest share whose GPU pages fit the HBM budget."""
        if self.hbm_budget_bytes is None or layer_bytes <= 0:
            return 1.0
        return min(1.0, max(0.0, self.hbm_budget_bytes / (layers * layer_bytes)))

    def choose(self, layer_bytes: float, layers: int = 1, granularity: float = 0.0) -> float:
        """The share minimising the per-layer time within the HBM budget.

        Candidates: the balance point, the capacity limit and r = 1; T is
        piecewise linear in r with its minimum at one of them.  granularity
        > 0 rounds the result down to a multiple of it (a coarser policy
        table), never above the capacity limit.
        """
        cap = self.capacity_share(layer_bytes, layers)
        cands = {min(cap, self.balance_share(layer_bytes)), cap}
        if cap >= 1.0:
            cands.add(1.0)
        best = min(cands, key=lambda r: (self.predict(r, layer_bytes)["layer"], -r))
        if granularity > 0:
            best = min(cap, math.floor(best / granularity + 1e-9) * granularity)
        return best

    def choose_for_lengths(self, lens, bytes_per_token: int, layers: int = 1,
                           granularity: float = 0.0) -> float:
        """choose() for a batch of sequence lengths (bytes of every token of one
        layer: 1152 for the absorbed MLA latent, Hkv*2*D*2 for GQA)."""
        return self.choose(float(sum(int(x) for x in lens)) * bytes_per_token, layers,
                           granularity)

    # ------------------------------------------------------------- calibration

    def observe(self, side: str, nbytes: float, seconds: float) -> None:
        """Folds one measured partial into that side's rate (EMA over the rate
        implied by the current fixed cost)."""
        s = self.gpu if side == "gpu" else self.host
        eff = seconds - s.fixed_s
        if nbytes <= 0 or eff <= 0:
            return
        w = self.ema_weight
        s.rate_bps = s.bounded((1.0 - w) * s.rate_bps + w * s.bounded(nbytes / eff))
        self.history.append((side, nbytes, seconds))


@dataclass
class SideFit:
    """A fitted side with the points it kept and the ones it left out."""
    side: Side
    used: list            # (bytes, seconds) points of the final fit
    rejected: list        # points dropped as outliers
    rate_capped: bool     # the least-squares rate exceeded max_rate_bps


def _affine(pts, max_rate_bps, min_fixed_s):
    """seconds = fixed + bytes / rate over pts by least squares, the rate
    capped at max_rate_bps (the intercept then refitted as the median
    residual) and the intercept floored at min_fixed_s (the slope then
    refitted through it)."""
    n = len(pts)
    mb = sum(b for b, _ in pts) / n
    mt = sum(t for _, t in pts) / n
    sbb = sum((b - mb) ** 2 for b, _ in pts)
    slope = sum((b - mb) * (t - mt) for b, t in pts) / sbb
    if slope <= 0:
        raise ValueError("time does not grow with bytes; cannot fit a rate")
    fixed = mt - slope * mb
    capped = max_rate_bps is not None and 1.0 / slope > max_rate_bps
    if capped:
        slope = 1.0 / max_rate_bps
        res = sorted(t - b * slope for b, t in pts)
        fixed = 0.5 * (res[(n - 1) // 2] + res[n // 2])
    if fixed < min_fixed_s:
        fixed = min_fixed_s
        slope = sum(b * (t - fixed) for b, t in pts) / sum(b * b for b, _ in pts)
        if slope <= 0:
            raise ValueError("time does not grow with bytes; cannot fit a rate")
        if max_rate_bps is not None and 1.0 / slope > max_rate_bps:
            slope, capped = 1.0 / max_rate_bps, True
    return Side(fixed_s=fixed, rate_bps=1.0 / slope, max_rate_bps=max_rate_bps), capped


def fit_side_report(points, max_rate_bps: float | None = None, min_fixed_s: float = 0.0,
                    reject_rel: float | None = None) -> SideFit:
    """Affine fit seconds = fixed + bytes / rate over (bytes, seconds) points,
    physically bounded and robust to single bad points.

    max_rate_bps caps the rate (a slope flatter than the hardware allows is a
    measurement artefact, e.g. a short partial slowed by idle clocks making a
    long one look fast); min_fixed_s floors the intercept (the launch floor).
    With reject_rel, one point at a time is left out while more than three
    remain: the one whose removal lets the fit explain the others best
    (smallest largest relative error), if the fit of the others misses it by
    more than reject_rel of its own time.  Judging each point by a fit that
    excludes it keeps a single bad point from dragging the line towards
    itself and getting good points rejected instead."""
    pts = [(float(b), float(t)) for b, t in points if b > 0]
    if len(pts) < 2 or len({b for b, _ in pts}) < 2:
        raise ValueError("need two or more distinct byte counts to fit a side")
    rejected = []
    side, capped = _affine(pts, max_rate_bps, min_fixed_s)
    while reject_rel is not None and len(pts) > 3:
        best = None
        for i in range(len(pts)):
            rest = pts[:i] + pts[i + 1:]
            if len({b for b, _ in rest}) < 2:
                continue
            try:
                s_i, c_i = _affine(rest, max_rate_bps, min_fixed_s)
            except ValueError:
                continue
            fit_err = max(abs(t - s_i.time(b)) / t for b, t in rest)
            b_i, t_i = pts[i]
            cand = (fit_err, i, s_i, c_i, abs(t_i - s_i.time(b_i)) / t_i)
            if best is None or cand[0] < best[0]:
                best = cand
        if best is None or best[4] <= reject_rel:
            break
        rejected.append(pts.pop(best[1]))
        side, capped = best[2], best[3]
    return SideFit(side, pts, rejected, capped)


def fit_side(points, max_rate_bps: float | None = None, min_fixed_s: float = 0.0,
             reject_rel: float | None = None) -> Side:
    """The side of fit_side_report: least squares by default, bounded and
    outlier-robust when asked."""
    return fit_side_report(points, max_rate_bps, min_fixed_s, reject_rel).side


# --------------------------------------------------------------------------
# Online control of a two-sided paged cache


@dataclass
class ShareMove:
    """One boundary move made by the controller."""
    step: int
    share_from: float
    share_to: float
    pages: int          # pages moved, summed over sequences (per layer)
    seconds: float      # wall time of the move (all layers), from its start to the switch
    # time the decode loop spent on it: all of `seconds` when the loop waits
    # for the copies, only the issue and the switch when they run under the
    # following steps
    stall_seconds: float = 0.0
    copy_seconds: float = 0.0  # the page copies alone


class ShareController:
    """Keeps a two-sided paged cache (scope_amd.paged) at the share the
    scheduler chooses, from the times the decode loop measures.

    Per layer the cache reports the GPU partial's event time and the host
    partial's wall time with the bytes each side streamed (observe_layer),
    which the scheduler folds into its rates with the reference's EMA form
    (system/qwenoffload.py:1160-1165, system/mixoffload.py:1466-1474).  After
    the last layer of a decode step, decide() asks the scheduler for the share
    of the current lengths within the HBM budget and returns new host-token
    targets per sequence when they move the boundary by at least
    min_move_pages pages per sequence on average (smaller moves are not worth
    their copies, and this hysteresis keeps the share from oscillating);
    the cache then moves its pages (set_boundaries).

    The reference adapts a split ratio toward equal GPU and CPU times and
    clamps it to [0.1, 0.9]; here the target comes from the roofline model of
    both sides plus the HBM capacity, so a cache larger than its HBM budget
    converges to the capacity share instead of oscillating around a balance
    point the budget does not allow.
    """

    def __init__(self, sched: ShareScheduler, bytes_per_token: int, layers: int,
                 page_size: int, min_move_pages: float = 1.0, granularity: float = 0.0):
        if bytes_per_token <= 0 or layers <= 0 or page_size <= 0:
            raise ValueError("bytes_per_token, layers and page_size must be positive")
        self.sched = sched
        self.bytes_per_token = bytes_per_token
        self.layers = layers
        self.page_size = page_size
        self.min_move_pages = min_move_pages
        self.granularity = granularity
        self.steps = 0
        self.moves: list[ShareMove] = []
        self.shares: list[float] = []   # share after each decide()
        self.chosen: list[float] = []   # the scheduler's choice at each decide()
        # moves decided but not made: (step, share_from, share_wanted, reason)
        self.skipped: list[tuple] = []

    def observe_layer(self, gpu_bytes: float, gpu_s: float, host_bytes: float,
                      host_s: float) -> None:
        """One layer's measured partials (bytes streamed, seconds)."""
        if gpu_bytes > 0 and gpu_s > 0:
            self.sched.observe("gpu", gpu_bytes, gpu_s)
        if host_bytes > 0 and host_s > 0:
            self.sched.observe("host", host_bytes, host_s)

    @staticmethod
    def share_of(lens, host_tokens) -> float:
        total = sum(int(x) for x in lens)
        return 1.0 if total == 0 else 1.0 - sum(int(h) for h in host_tokens) / total

    def targets_for(self, r: float, lens, round_up: bool = False) -> list[int]:
        """Host tokens per sequence at share r: L - floor(r L), rounded down to
        a page (the GPU takes the rest), as the cache's set_share does; with
        round_up, rounded up instead (at most L's last full page), so the GPU
        side stays within r L: the rounding used when HBM capacity sets r."""
        ps = self.page_size
        out = []
        for L in lens:
            L = int(L)
            h = L - int(math.floor(r * L))
            out.append(min(-(-h // ps) * ps, (L // ps) * ps) if round_up else (h // ps) * ps)
        return out

    def decide(self, lens, host_tokens, moving: bool = False):
        """After a decode step: host-token targets per sequence if the chosen
        share moves the boundary by at least min_move_pages pages per
        sequence, or if the GPU side has outgrown the HBM budget (decode
        appends land on the GPU side); else None.  With moving (a move of
        the cache is still in flight), the choice is recorded and None
        returned."""
        self.steps += 1
        W = float(sum(int(x) for x in lens)) * self.bytes_per_token
        r = self.sched.choose(W, self.layers, self.granularity)
        self.chosen.append(r)
        cap = self.sched.capacity_share(W, self.layers)
        targets = self.targets_for(r, lens, round_up=cap < 1.0 and r >= cap - 1e-12)
        budget = self.sched.hbm_budget_bytes
        gpu_bytes = (sum(int(x) for x in lens) - sum(int(h) for h in host_tokens)) \
            * self.bytes_per_token * self.layers
        over = budget is not None and gpu_bytes > budget
        moved = sum(abs(t - int(h)) for t, h in zip(targets, host_tokens)) // self.page_size
        same = all(t == int(h) for t, h in zip(targets, host_tokens))
        if moving or same or (moved < self.min_move_pages * max(1, len(lens)) and not over):
            self.shares.append(self.share_of(lens, host_tokens))
            return None
        self.shares.append(self.share_of(lens, targets))
        return targets

    def amend_last_share(self, r: float) -> None:
        """The share the last decide() led to, when the cache could make only
        part of the move (or none of it)."""
        if self.shares:
            self.shares[-1] = r

    def record_skip(self, share_from: float, share_wanted: float, reason: str) -> None:
        """A move decided after step self.steps that the cache could not start
        (pools or partition full); the decode step itself went on."""
        self.skipped.append((self.steps, share_from, share_wanted, reason))

    def record_move(self, share_from: float, share_to: float, pages: int,
                    seconds: float, stall_seconds: float | None = None,
                    step: int | None = None, copy_seconds: float | None = None) -> None:
        """A move the cache made: started after decode step `step` (default:
        the last decided), `seconds` to its switch, `stall_seconds` of them
        spent by the decode loop and `copy_seconds` by its page copies
        (default: all)."""
        self.moves.append(ShareMove(self.steps if step is None else step, share_from,
                                    share_to, pages, seconds,
                                    seconds if stall_seconds is None else stall_seconds,
                                    seconds if copy_seconds is None else copy_seconds))
