"""Boundary movement of the two-sided paged caches (scope_amd/paged.py), on
the CPU: both "sides" live in host memory here, the GPU pages are written
directly, and only the bookkeeping and page copies run.  After every move
the concatenation host tokens ++ GPU tokens must equal the original token
sequence bit for bit, every page must be accounted for, and both sides'
lengths and tables must agree."""
import time

import numpy as np
import pytest
import torch

from helpers import bf16_randn, bits
from scope_amd.paged import PagedKVCache, PagedMlaCache

PS = 32


def _fill_gpu(part, layer, b, payloads):
    """Write token rows into the GPU partition's pages of (layer, b) as the
    append kernels would (payload token axis: -2 for GQA pools, 0 for MLA)."""
    n = payloads[0].shape[-2] if payloads[0].dim() == 3 else payloads[0].shape[0]
    part.reserve(b, int(part.lens[layer, b]) + n)
    start = int(part.lens[layer, b])
    pools = [part.k, part.v] if hasattr(part, "k") else [part.latent]
    for t in range(n):
        pos = start + t
        pid = int(part.host_table[b, pos // part.page_size])
        off = pos % part.page_size
        for pool, pl in zip(pools, payloads):
            if pl.dim() == 3:  # [Hkv, n, D]
                pool[layer, pid, :, off] = pl[:, t]
            else:              # [n, 576]
                pool[layer, pid, off] = pl[t]
    part.lens[layer, b] += n
    part._len_bufs[:, layer, b] = int(part.lens[layer, b])


def _gather(cache, layer, b):
    """Token rows of sequence b in `layer`: host pages then GPU pages."""
    ps = cache.page_size
    h = int(cache.host.lens[b])
    g = cache.gpu
    gl = int(g.lens[layer, b])
    out = []
    for data_h, data_g in zip(cache.host.data, cache._gpu_payload()):
        rows = []
        for t in range(h):
            pid = int(cache.host.table[b, t // ps])
            rows.append(data_h[layer, pid, ..., t % ps, :] if data_h.dim() == 5
                        else data_h[layer, pid, t % ps])
        for t in range(gl):
            pid = int(g.host_table[b, t // ps])
            rows.append(data_g[layer, pid, ..., t % ps, :] if data_g.dim() == 5
                        else data_g[layer, pid, t % ps])
        out.append(torch.stack(rows, dim=-2) if rows[0].dim() == 2 else torch.stack(rows))
    return out


def _check_accounting(cache):
    g = cache.gpu
    used_g = sum(int(x) for x in g._pages_held)
    assert g.pool.free + used_g == g.num_pages
    used_h = sum(int(x) for x in cache.host.held)
    assert cache.host.pool.free + used_h == cache.host.num_pages
    for b in range(cache.batch):
        assert int(cache.host.held[b]) * cache.page_size == int(cache.host.lens[b])
        assert int(g._pages_held[b]) >= -(-int(g.lens[0, b]) // cache.page_size)
        held = int(g._pages_held[b])
        assert np.array_equal(g.page_table[b, :held].numpy(), g.host_table[b, :held])
        assert (g.host_table[b, held:] == -1).all()
        assert (g._len_bufs[:, :, b] == int(g.lens[0, b])).all()
        ids = list(g.host_table[b, :held])
        assert len(set(ids)) == len(ids)


def test_mla_boundary_moves_keep_every_token():
    layers, B = 2, 3
    lens = [5 * PS + 7, 3 * PS, 2 * PS + 1]
    hosts = [2 * PS, 1 * PS, 0]
    cache = PagedMlaCache(layers, B, max_tokens=8 * PS, page_size=PS, device="cpu", pin=False)
    cache.STAGE_BYTES = 2 * layers * PS * 576 * 2   # two pages per chunk: multi-chunk copies
    data = {}
    for layer in range(layers):
        for b, (L, h) in enumerate(zip(lens, hosts)):
            c = bf16_randn((L, 512), 100 * layer + b)
            pe = bf16_randn((L, 64), 100 * layer + b + 50)
            data[layer, b] = torch.cat([c, pe], dim=1)
            # host part through load(); the GPU part written directly
            cache.host.lens[b] = h if layer == 0 else cache.host.lens[b]
            if layer == 0:
                cache._host_reserve(b, h)
            for p in range(h // PS):
                cache.host.data[0][layer, int(cache.host.table[b, p])] = \
                    data[layer, b][p * PS:(p + 1) * PS]
            _fill_gpu(cache.gpu, layer, b, [data[layer, b][h:]])
    _check_accounting(cache)
    moves = [(0, 4 * PS), (0, 0), (1, 3 * PS), (2, 2 * PS), (0, 5 * PS), (2, 0), (1, 0)]
    for b, h_new in moves:
        cache.set_boundary(b, h_new)
        assert cache.host_tokens(b) == h_new
        _check_accounting(cache)
        for layer in range(layers):
            for bb in range(B):
                (got,) = _gather(cache, layer, bb)
                assert np.array_equal(bits(got), bits(data[layer, bb])), (b, h_new, layer, bb)
    with pytest.raises(ValueError):
        cache.set_boundary(0, PS + 1)          # not a page multiple
    with pytest.raises(ValueError):
        cache.set_boundary(1, 4 * PS)          # beyond the sequence
    cache.set_share(0.5)
    for b, L in enumerate(lens):
        h = L - int(np.floor(0.5 * L))
        assert cache.host_tokens(b) == (h // PS) * PS
    _check_accounting(cache)


def test_gqa_boundary_moves_keep_every_token():
    layers, B, Hkv, D = 2, 2, 2, 64
    lens = [4 * PS + 3, 2 * PS]
    cache = PagedKVCache(layers, B, Hkv, D, max_tokens=6 * PS, page_size=PS, device="cpu",
                         pin=False)
    cache.STAGE_BYTES = layers * Hkv * PS * D * 2    # one page per chunk
    data = {}
    for layer in range(layers):
        for b, L in enumerate(lens):
            k = bf16_randn((Hkv, L, D), 10 * layer + b)
            v = bf16_randn((Hkv, L, D), 10 * layer + b + 5)
            data[layer, b] = (k, v)
            _fill_gpu(cache.gpu, layer, b, [k, v])
    _check_accounting(cache)
    for b, h_new in [(0, 3 * PS), (1, 2 * PS), (0, PS), (1, 0), (0, 4 * PS), (0, 0)]:
        cache.set_boundary(b, h_new)
        _check_accounting(cache)
        for layer in range(layers):
            for bb in range(B):
                gk, gv = _gather(cache, layer, bb)
                k, v = data[layer, bb]
                assert np.array_equal(bits(gk), bits(k)) and np.array_equal(bits(gv), bits(v))


def test_gpu_capacity_is_checked_before_moving():
    cache = PagedMlaCache(1, 1, max_tokens=2 * PS, page_size=PS, device="cpu", pin=False)
    lat = bf16_randn((2 * PS, 576), 1)
    _fill_gpu(cache.gpu, 0, 0, [lat])
    cache.set_boundary(0, 2 * PS)      # everything to the host
    assert int(cache.gpu.lens[0, 0]) == 0 and cache.gpu.pool.free == cache.gpu.num_pages
    cache.set_boundary(0, 0)           # and back
    (got,) = _gather(cache, 0, 0)
    assert np.array_equal(bits(got), bits(lat))


def test_mixed_direction_batch_and_pool_exhaustion():
    layers, B = 2, 3
    lens = [4 * PS, 3 * PS + 5, 2 * PS]
    hosts = [0, 3 * PS, PS]
    # pools sized exactly: a move must find its free pages before releasing
    cache = PagedMlaCache(layers, B, max_tokens=5 * PS, page_size=PS, host_pages=7,
                          gpu_pages=9, device="cpu", pin=False)
    data = {}
    for layer in range(layers):
        for b, (L, h) in enumerate(zip(lens, hosts)):
            data[layer, b] = bf16_randn((L, 576), 70 + 10 * layer + b)
            if layer == 0:
                cache._host_reserve(b, h)
                cache.host.lens[b] = h
            for p in range(h // PS):
                cache.host.data[0][layer, int(cache.host.table[b, p])] = \
                    data[layer, b][p * PS:(p + 1) * PS]
            _fill_gpu(cache.gpu, layer, b, [data[layer, b][h:]])
    _check_accounting(cache)
    cache.set_boundaries([2 * PS, PS, 0])   # seq 0 down, seqs 1 and 2 up, in one batch
    assert [cache.host_tokens(b) for b in range(B)] == [2 * PS, PS, 0]
    _check_accounting(cache)
    for layer in range(layers):
        for b in range(B):
            (got,) = _gather(cache, layer, b)
            assert np.array_equal(bits(got), bits(data[layer, b]))
    with pytest.raises(MemoryError):          # 4 + 3 + 2 pages > 7 host pages
        cache.set_boundaries([4 * PS, 3 * PS, 2 * PS])
    _check_accounting(cache)                  # a refused move changes nothing
    assert [cache.host_tokens(b) for b in range(B)] == [2 * PS, PS, 0]


def _mla_cache_with(lens, hosts, layers, max_tokens, **kw):
    cache = PagedMlaCache(layers, len(lens), max_tokens=max_tokens, page_size=PS, device="cpu",
                          pin=False, **kw)
    data = {}
    for layer in range(layers):
        for b, (L, h) in enumerate(zip(lens, hosts)):
            data[layer, b] = bf16_randn((L, 576), 300 + 10 * layer + b)
            if layer == 0:
                cache._host_reserve(b, h)
                cache.host.lens[b] = h
            for p in range(h // PS):
                cache.host.data[0][layer, int(cache.host.table[b, p])] = \
                    data[layer, b][p * PS:(p + 1) * PS]
            _fill_gpu(cache.gpu, layer, b, [data[layer, b][h:]])
    return cache, data


def _append_all(cache, data, n, seed):
    """n decode appends to every sequence of every layer (GPU side)."""
    for (layer, b), rows in list(data.items()):
        new = bf16_randn((n, 576), seed + 10 * layer + b)
        _fill_gpu(cache.gpu, layer, b, [new])
        data[layer, b] = torch.cat([rows, new])


def _check_tokens(cache, data):
    for (layer, b), rows in data.items():
        (got,) = _gather(cache, layer, b)
        assert np.array_equal(bits(got), bits(rows)), (layer, b)


def test_begun_move_keeps_the_boundaries_until_the_switch():
    """begin_boundaries copies the pages but leaves both sides' tables and
    lengths alone; decode appends meanwhile; the switch uses the lengths of
    its own moment."""
    layers = 2
    lens, hosts = [5 * PS + 7, 3 * PS + 2, 2 * PS + 1], [2 * PS, 0, 2 * PS]
    cache, data = _mla_cache_with(lens, hosts, layers, max_tokens=9 * PS)
    targets = [4 * PS, 2 * PS, 0]            # seqs 0 and 1 toward the host, seq 2 to the GPU
    assert cache.begin_boundaries(targets) and cache.moving
    assert [cache.host_tokens(b) for b in range(3)] == hosts
    _check_tokens(cache, data)
    _append_all(cache, data, PS + 3, 900)    # steps go on over the current boundaries
    _check_tokens(cache, data)
    with pytest.raises(RuntimeError):
        cache.begin_boundaries(hosts)        # one move at a time
    with pytest.raises(RuntimeError, match="boundary move"):
        cache.load(0, 0, data[0, 0][:, :512], data[0, 0][:, 512:], 0)
    cache.gpu.lens[1, 0] += 1                # layer 1 mid-step: no switch, the move stays
    with pytest.raises(RuntimeError, match="mid-step"):
        cache.poll_boundaries()
    assert cache.moving
    cache.gpu.lens[1, 0] -= 1
    assert cache.poll_boundaries() and not cache.moving
    assert [cache.host_tokens(b) for b in range(3)] == targets and cache.last_kept == []
    _check_accounting(cache)
    _check_tokens(cache, data)
    assert not cache.poll_boundaries()       # nothing in flight
    assert not cache.begin_boundaries(targets)
    # set_boundaries finishes a begun move first
    cache.begin_boundaries([0, 0, 2 * PS])
    cache.set_boundaries([PS, 0, 0])
    assert [cache.host_tokens(b) for b in range(3)] == [PS, 0, 0]
    _check_accounting(cache)
    _check_tokens(cache, data)


def test_begun_move_to_the_gpu_is_kept_when_appends_fill_the_partition():
    layers = 1
    cache, data = _mla_cache_with([3 * PS], [2 * PS], layers, max_tokens=4 * PS, gpu_pages=8)
    free_g = cache.gpu.pool.free
    assert cache.begin_boundaries([0])       # 1 + 2 GPU pages fit in 4
    assert cache.gpu.pool.free == free_g - 2
    _append_all(cache, data, 2 * PS, 700)    # now 3 GPU pages: 3 + 2 > 4
    cache.finish_boundaries()
    assert cache.last_kept == [0] and cache.host_tokens(0) == 2 * PS
    assert cache.gpu.pool.free == free_g - 2  # the two appended pages; the move's came back
    _check_accounting(cache)
    _check_tokens(cache, data)


def test_a_move_whose_copies_fail_gives_its_pages_back():
    cache, data = _mla_cache_with([3 * PS + 5, 2 * PS], [PS, 2 * PS], 1, max_tokens=6 * PS)
    free = (cache.gpu.pool.free, cache.host.pool.free)

    def fail(*a):
        raise RuntimeError("copy failed")
    cache._pages_to_host = cache._pages_to_gpu = fail
    with pytest.raises(RuntimeError, match="copy failed"):
        cache.begin_boundaries([2 * PS, 0])
    assert not cache.moving and (cache.gpu.pool.free, cache.host.pool.free) == free
    _check_accounting(cache)
    _check_tokens(cache, data)


def _controlled(cache, budget_bytes=None):
    """A share controller on `cache` with the per-layer timing left out (no
    GPU here): _step_done() is the controller's part of a decode step."""
    from scope_amd.scheduler import ShareController, ShareScheduler, Side

    sched = ShareScheduler(gpu=Side(1e-6, 6e12, max_rate_bps=8e12), host=Side(1e-6, 1e11),
                           hbm_budget_bytes=budget_bytes)
    ctl = ShareController(sched, 1152, cache.num_layers, cache.page_size)
    cache.controller, cache.async_moves = ctl, False
    cache._layer_log, cache._step_end = [], None
    return ctl


def test_controller_moves_are_cut_to_the_free_pages_and_never_raise():
    """GPU pool sized exactly to the loaded layout plus 4 pages: the scheduler
    wants everything in HBM (no budget, a fast GPU), which needs 9 more GPU
    pages.  The move is cut to the free pages less one page per sequence
    kept for appends, the tokens survive bit for bit, and the controller
    records the share actually reached; with no page to spare the move is
    skipped and recorded, and a move that fails to start is recorded too,
    without raising out of the step."""
    layers = 2
    lens, hosts = [4 * PS + 3, 3 * PS + 5, 2 * PS], [3 * PS, 3 * PS, 2 * PS]
    gpu_need = sum(-(-(L - h) // PS) for L, h in zip(lens, hosts))
    cache, data = _mla_cache_with(lens, hosts, layers, 6 * PS, gpu_pages=gpu_need + 4)
    ctl = _controlled(cache)
    cache._step_done()
    # 4 free GPU pages, 3 kept for appends: one page moves up (sequence 0's)
    assert [cache.host_tokens(b) for b in range(3)] == [2 * PS, 3 * PS, 2 * PS]
    assert cache.gpu.pool.free == 3
    assert len(ctl.moves) == 1 and ctl.moves[0].pages == 1
    assert ctl.shares[-1] == pytest.approx(ctl.share_of(lens, [2 * PS, 3 * PS, 2 * PS]))
    _check_accounting(cache)
    _check_tokens(cache, data)
    # no GPU page to spare: skipped, recorded, nothing moves
    cache._step_done()
    assert [cache.host_tokens(b) for b in range(3)] == [2 * PS, 3 * PS, 2 * PS]
    assert len(ctl.moves) == 1 and len(ctl.skipped) == 1
    assert ctl.shares[-1] == pytest.approx(ctl.share_of(lens, [2 * PS, 3 * PS, 2 * PS]))
    # a move that fails to start is recorded as skipped, not raised
    cache.feasible_targets = lambda t, gpu_reserve=0: [PS, 3 * PS, 2 * PS]

    def refuse(targets):
        raise MemoryError("pool exhausted")
    cache.set_boundaries = refuse
    cache._step_done()
    assert len(ctl.skipped) == 2 and "pool exhausted" in ctl.skipped[-1][3]
    assert ctl.shares[-1] == pytest.approx(ctl.share_of(lens, [2 * PS, 3 * PS, 2 * PS]))
    _check_accounting(cache)
    _check_tokens(cache, data)


def test_feasible_targets_respect_capacity_and_host_pool():
    layers = 1
    lens, hosts = [5 * PS, 2 * PS], [4 * PS, 0]
    cache, _ = _mla_cache_with(lens, hosts, layers, 5 * PS, host_pages=5, gpu_pages=20)
    # sequence 0 can take 4 pages up; sequence 1 wants 2 pages down but the
    # host pool has 1 free page
    assert cache.feasible_targets([0, 2 * PS]) == [0, PS]
    # the partition capacity (5 pages per sequence) caps a move up
    cache.gpu.max_pages = 3
    assert cache.feasible_targets([0, 0], gpu_reserve=0) == [2 * PS, 0]
    # the GPU reserve leaves pages free
    cache.gpu.max_pages = 5
    free = cache.gpu.pool.free
    assert cache.feasible_targets([0, 0], gpu_reserve=free - 1) == [3 * PS, 0]

def test_paced_targets_cut_every_sequence_by_the_same_fraction():
    layers = 1
    lens, hosts = [8 * PS, 8 * PS, 4 * PS], [8 * PS, 0, 4 * PS]
    cache, _ = _mla_cache_with(lens, hosts, layers, 8 * PS, host_pages=30, gpu_pages=30)
    # sequence 0 wants 8 pages up, sequence 1 4 pages down, sequence 2 stays
    targets = [0, 4 * PS, 4 * PS]
    assert cache.paced_targets(targets, 12) == targets  # within the cap: unchanged
    assert cache.paced_targets(targets, 100) == targets
    # 6 of 12 pages: half of each way
    assert cache.paced_targets(targets, 6) == [4 * PS, 2 * PS, 4 * PS]
    # 5 of 12: 8*5//12 = 3 and 4*5//12 = 1, the leftover page to the first
    assert cache.paced_targets(targets, 5) == [4 * PS, PS, 4 * PS]
    # one page
    assert cache.paced_targets(targets, 1) == [7 * PS, 0, 4 * PS]
    # every result is a feasible boundary and moves no more than the cap
    for cap in range(1, 13):
        out = cache.paced_targets(targets, cap)
        moved = sum(abs(o - h) // PS for o, h in zip(out, hosts))
        assert moved == min(cap, 12)
        assert all(o % PS == 0 and 0 <= o <= L for o, L in zip(out, lens))
        # each sequence moves toward its target and not past it
        for o, h, t in zip(out, hosts, targets):
            assert min(h, t) <= o <= max(h, t)


def test_async_controller_paces_a_move_to_the_step_time():
    """With pacing on, an async controller whose copies could move only a
    few pages within half a step starts a move of that many pages."""
    layers = 2
    lens, hosts = [6 * PS, 6 * PS], [6 * PS, 6 * PS]
    cache, data = _mla_cache_with(lens, hosts, layers, 6 * PS, gpu_pages=40)
    ctl = _controlled(cache)
    cache.async_moves = True
    cache.MOVE_STEP_FRACTION = 0.5
    # copies of 4 pages per step, so half a step moves 2
    step_s = 1.0
    cache._move_rate = 4 * cache._page_bytes() / step_s
    cache._step_end = time.perf_counter() - step_s
    cache._step_done()
    assert cache.moving  # the move is in flight
    m = cache._move
    assert m.pages == 2
    cache.finish_boundaries()
    assert sum(hosts) - sum(cache.host_tokens(b) for b in range(2)) == 2 * PS
    _check_accounting(cache)
    _check_tokens(cache, data)
