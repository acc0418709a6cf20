"""Token-range-partitioned decode KV caches with both segments paged alike.

Sequence b keeps its leading h_b tokens in host pages and the rest in HBM
pages.  Both sides use the same page layout (GQA: [Hkv, page_size, D] per
page of K and of V; MLA: [page_size, 576] per page of latent), so the
boundary moves by copying whole pages: set_boundary() / set_share() turn the
GPU's leading pages into host pages (share down) or the host's trailing pages
into GPU pages (share up), for every layer, and rewrite both page tables.
The reference fixes its boundary when the cache is allocated
(system/deepseek.py:161-166) and has no migration; this is the missing piece
that lets the share follow the scheduler (scope_amd.scheduler) as lengths
grow.

h_b is always a multiple of the page size: a host page is full, and decode
appends go to the GPU side only (the new token is at position L_b >= h_b), as
in the reference's boundary split (system/deepseek.py:181-188).

A decode step per layer is one call of the native layer driver
(scope_amd/layer.py, libwslayer.so), with the GIL released: q to pinned host
memory by a copy kernel; the GPU split step (append + partial over the HBM
pages); the native host partial over the host pages in the calling thread
while the GPU runs (bf16 out, fp32 lse, pinned); the merge, which reads it in
place (ws_merge_split, or ws_mla_merge_split_uv with the W_UV epilogue).
Lengths are the same in every layer between steps; migrate only then.
set_boundaries() waits for a move's page copies; begin_boundaries() lets
them run on a side stream under the following steps, which keep the
current boundaries until poll_boundaries() / finish_boundaries() switches
both sides over.
"""
from __future__ import annotations

import time

import numpy as np
import torch

from . import ops
from .layer import WlError, WlGqaLayer, WlMlaLayer
from .layer import lib as layer_lib
from .layer import run as run_layer
from .cache import GqaGpuPartition, MlaGpuPartition, PagePool
from .partition import pages_for


class _HostPages:
    """Host page pools (one tensor per payload, [num_layers, num_pages, *page])
    and the host segment's page table and lengths (shared by all layers)."""

    def __init__(self, num_layers, batch, max_pages, num_pages, page_shapes, pin):
        self.num_pages = num_pages
        self.pool = PagePool(num_pages)
        self.data = [torch.empty((num_layers, num_pages, *shape), dtype=torch.bfloat16,
                                 pin_memory=pin) for shape in page_shapes]
        self.table = np.zeros((batch, max_pages), np.int32)
        self.table_t = torch.from_numpy(self.table)  # shares memory with `table`
        self.held = np.zeros(batch, np.int64)
        self.lens = np.zeros(batch, np.int32)
        self.lens_t = torch.from_numpy(self.lens)


class _Move:
    """A boundary move whose page copies have been issued: per sequence
    (b, h, h_new, k, GPU page ids, host page ids), for moves toward the host
    (`downs`) and toward the GPU (`ups`); `event` follows the copies on the
    GPU's side stream (None: they are done)."""

    def __init__(self):
        self.downs, self.ups, self.kept = [], [], []
        self.event = self.start = None
        self.pages = self.bytes = 0
        self.t_begin = 0.0
        self.info = None  # the controller's record of the move


class _PagedTwoSided:
    """Shared bookkeeping of the two-sided caches; subclasses name the
    payload tensors of each side and the decode step."""

    gpu: GqaGpuPartition | MlaGpuPartition

    def __init__(self, num_layers, batch, max_tokens, page_size, host_pages, pin):
        self.num_layers = num_layers
        self.batch = batch
        self.page_size = page_size
        self.max_pages = max(1, pages_for(max_tokens, page_size))
        if host_pages is None:
            host_pages = batch * self.max_pages
        self.host = _HostPages(num_layers, batch, self.max_pages, host_pages,
                               self._page_shapes(), pin)
        # the side stream of boundary moves (default priority), used once here
        # so that its first-use costs (its queue, the allocator's first block
        # for it) are not paid by the first move
        dev = self.gpu.device
        self._move_stream = None
        if dev.type == "cuda":
            self._move_stream = torch.cuda.Stream(device=dev)
            with torch.cuda.stream(self._move_stream):
                torch.zeros(1, dtype=torch.int32, device=dev)
            self._move_stream.synchronize()

    # -- payload access (per subclass) -------------------------------------

    def _page_shapes(self):
        raise NotImplementedError

    def _gpu_payload(self):
        """GPU pool tensors [num_layers, num_pages, *page], in payload order."""
        raise NotImplementedError

    # -- lengths -------------------------------------------------------------

    def seq_len(self, b: int) -> int:
        """Tokens of sequence b (host + GPU); equal in every layer between steps."""
        g = self.gpu.lens[:, b]
        if (g != g[0]).any():
            raise RuntimeError("layers are mid-step (lengths differ across layers)")
        return int(self.host.lens[b]) + int(g[0])

    def host_tokens(self, b: int) -> int:
        return int(self.host.lens[b])

    def _host_reserve(self, b: int, n_tokens: int) -> None:
        need = pages_for(n_tokens, self.page_size)
        if need > self.max_pages:
            raise ValueError(f"sequence {b}: {n_tokens} host tokens exceed capacity")
        for p in range(int(self.host.held[b]), need):
            self.host.table[b, p] = self.host.pool.alloc()
        self.host.held[b] = max(int(self.host.held[b]), need)

    def _set_gpu_lens(self, b: int, n: int) -> None:
        g = self.gpu
        g.lens[:, b] = n
        g._len_bufs[:, :, b] = n

    def _write_gpu_row(self, b: int) -> None:
        g = self.gpu
        g.page_table[b].copy_(torch.from_numpy(g.host_table[b].copy()))

    def reserve_layout(self, lens, host_tokens) -> None:
        """Give every sequence b lens[b] tokens, host_tokens[b] of them (a page
        multiple) in host pages and the rest in HBM pages, in every layer,
        without writing any data: for callers that fill the page pools
        themselves (bulk prefill, benchmarks).  The cache must be empty."""
        ps = self.page_size
        g = self.gpu
        if len(lens) != self.batch or len(host_tokens) != self.batch:
            raise ValueError(f"need {self.batch} lengths and host token counts")
        self._check_no_move("reserve_layout")
        if self.host.lens.any() or g.lens.any():
            raise RuntimeError("reserve_layout needs an empty cache")
        for b, (L, h) in enumerate(zip(lens, host_tokens)):
            L, h = int(L), int(h)
            if h % ps or not 0 <= h <= L:
                raise ValueError(f"sequence {b}: host tokens {h} must be a page multiple "
                                 f"in [0, {L}]")
            self._host_reserve(b, h)
            self.host.lens[b] = h
            g.reserve(b, L - h)
            self._set_gpu_lens(b, L - h)

    # -- boundary movement ---------------------------------------------------

    def set_boundary(self, b: int, h_new: int) -> None:
        """Move sequence b's boundary to h_new host tokens (a multiple of the
        page size, at most its length), copying pages between the sides in
        every layer."""
        targets = [int(x) for x in self.host.lens]
        targets[b] = h_new
        self.set_boundaries(targets)

    def set_share(self, r: float) -> None:
        """GPU share r for every sequence: host tokens L - floor(r L), rounded
        down to a page multiple (the GPU takes the remainder)."""
        if not 0.0 <= r <= 1.0:
            raise ValueError(f"share {r} outside [0, 1]")
        targets = []
        for b in range(self.batch):
            L = self.seq_len(b)
            h = L - int(np.floor(r * L))
            targets.append((h // self.page_size) * self.page_size)
        self.set_boundaries(targets)

    def set_boundaries(self, targets) -> None:
        """Move every sequence's boundary to targets[b] host tokens in one
        batch: one page-copy launch per direction and payload, all layers at
        once (pinned host pools; unpinned ones go through pinned staging).
        New pages are taken before any page is given back, so no page is both
        read and written within a batch.  Returns when the copies are done and
        both sides use the new boundaries (a move in flight is finished
        first)."""
        self.finish_boundaries()
        if self.begin_boundaries(targets):
            self.finish_boundaries()

    _move = None  # the boundary move in flight (_Move), or None
    last_kept: list = []  # sequences the last switch left at their boundary
    last_copy_seconds = None  # GPU time of the last switched move's copies (side stream)

    @property
    def moving(self) -> bool:
        """A boundary move has been started and not yet switched to."""
        return self._move is not None

    def _check_no_move(self, what: str) -> None:
        if self._move is not None:
            raise RuntimeError(f"{what} during a boundary move: finish_boundaries() first")

    # Grid of a move's page copies: the host link bounds them, and 16
    # workgroups (512 KB of loads in flight) keep it as busy as 64 do, while
    # the decode kernels that run beside a begun move's copies are slowed far
    # less (their own loads wait behind fewer outstanding host-link reads).
    MOVE_WORKGROUPS = 16
    # At the end of a step, wait for a begun move's copies when they are
    # expected to end within this fraction of a step (at the copy rate last
    # measured in this process, _move_rate bytes/s; before any, a PCIe Gen5
    # x16 link's usual rate), instead of running one more step at the old
    # boundaries.
    MOVE_WAIT_FRACTION = 0.25
    _move_rate = 50e9
    # A move begun under the decode steps may be cut to the pages its copies
    # can move in this fraction of a step (at _move_rate): its copies then
    # end within the step that runs beside them, and the next decisions carry
    # the boundary on.  None (the default): the whole move at once, which
    # measured faster when the copies do not slow the steps beside them.
    MOVE_STEP_FRACTION = None

    def begin_boundaries(self, targets) -> bool:
        """Start moving every sequence's boundary to targets[b] host tokens
        and return without waiting for the copies.  The destination pages are
        taken from the pools now; with pinned host pools on a GPU the page
        copies queue on a side stream behind the work already queued on the
        current one (otherwise they run here, through pinned staging).
        Decode steps go on over the current boundaries meanwhile: the copies
        read full pages that decode appends never write (the host's trailing
        pages, or the GPU's leading pages below its newest token) and write
        pages that no table holds yet.  poll_boundaries() or
        finish_boundaries() switches both sides to the new boundaries, with
        the lengths of that moment.  One move at a time.  Returns False when
        no boundary moves."""
        if self._move is not None:
            raise RuntimeError("a boundary move is in flight: poll_boundaries() or "
                               "finish_boundaries() first")
        ps = self.page_size
        g = self.gpu
        if len(targets) != self.batch:
            raise ValueError(f"need {self.batch} targets")
        plan = []
        for b, h_new in enumerate(targets):
            h_new = int(h_new)
            L = self.seq_len(b)
            if h_new % ps or not 0 <= h_new <= L:
                raise ValueError(f"sequence {b}: boundary {h_new} must be a multiple of {ps} "
                                 f"in [0, {L}]")
            h = int(self.host.lens[b])
            if h_new != h:
                plan.append((b, h, h_new))
        if not plan:
            return False
        need_g = sum((h - hn) // ps for _, h, hn in plan if hn < h)
        need_h = sum((hn - h) // ps for _, h, hn in plan if hn > h)
        if need_g > g.pool.free or need_h > self.host.pool.free:
            raise MemoryError(f"boundary move needs {need_g} GPU / {need_h} host free pages, "
                              f"{g.pool.free} / {self.host.pool.free} available")
        for b, h, hn in plan:
            if hn < h and int(g._pages_held[b]) + (h - hn) // ps > g.max_pages:
                raise ValueError(f"sequence {b}: GPU partition capacity exceeded")
        m = _Move()
        for b, h, h_new in plan:
            k = abs(h_new - h) // ps
            if h_new > h:  # GPU's leading k pages -> new host pages
                pids_g = [int(x) for x in g.host_table[b, :k]]
                pids_h = [self.host.pool.alloc() for _ in range(k)]
                m.downs.append((b, h, h_new, k, pids_g, pids_h))
            else:  # host's trailing k pages -> new GPU pages
                hp1 = h // ps
                pids_h = [int(x) for x in self.host.table[b, hp1 - k:hp1]]
                pids_g = [g.pool.alloc() for _ in range(k)]
                m.ups.append((b, h, h_new, k, pids_g, pids_h))
        down_g = [x for e in m.downs for x in e[4]]
        down_h = [x for e in m.downs for x in e[5]]
        up_g = [x for e in m.ups for x in e[4]]
        up_h = [x for e in m.ups for x in e[5]]
        m.pages = len(down_g) + len(up_g)
        m.bytes = m.pages * self._page_bytes()
        m.t_begin = time.perf_counter()
        dev = g.device
        side = dev.type == "cuda" and all(hp.is_pinned() for hp in self.host.data)
        try:
            if side:
                ms = self._move_stream
                ms.wait_stream(torch.cuda.current_stream(dev))
                m.start = torch.cuda.Event(enable_timing=True)
                m.start.record(ms)
                with torch.cuda.stream(ms):
                    wg = self.MOVE_WORKGROUPS
                    for gp, hp in zip(self._gpu_payload(), self.host.data):  # all layers at once
                        if down_g:
                            ops.copy_pages(hp, down_h, gp, down_g, wg)
                        if up_g:
                            ops.copy_pages(gp, up_g, hp, up_h, wg)
                    m.event = torch.cuda.Event(enable_timing=True)
                    m.event.record(ms)
            else:
                for gp, hp in zip(self._gpu_payload(), self.host.data):
                    if down_g:
                        self._pages_to_host(gp, hp, down_g, down_h)
                    if up_g:
                        self._pages_to_gpu(gp, hp, up_g, up_h)
        except BaseException:
            if side:
                self._move_stream.synchronize()  # copies already queued end first
            for pid in down_h:
                self.host.pool.release(pid)
            for pid in up_g:
                g.pool.release(pid)
            raise
        self._move = m
        return True

    def poll_boundaries(self) -> bool:
        """Between decode steps: if the copies of the move in flight are done,
        switch both sides to its boundaries and return True; else False."""
        m = self._move
        if m is None or (m.event is not None and not m.event.query()):
            return False
        self._switch(m)
        return True

    def finish_boundaries(self) -> None:
        """Between decode steps: wait for the copies of the move in flight (if
        any) and switch both sides to its boundaries."""
        m = self._move
        if m is None:
            return
        if m.event is not None:
            m.event.synchronize()
        self._switch(m)

    def _switch(self, m) -> None:
        """The tables and lengths of both sides after the copies of move m,
        with the GPU lengths of now (decode appends may have added tokens
        since the move began).  A sequence whose GPU side can no longer take
        its new leading pages (appends filled the partition meanwhile) keeps
        its boundary; its pages go back to the pool (listed in last_kept)."""
        ps = self.page_size
        g = self.gpu
        # lengths first: between steps they agree across layers (else this
        # raises and the move stays in flight)
        lens = {e[0]: self.seq_len(e[0]) for e in m.downs + m.ups}
        self._move = None
        self.last_kept = m.kept
        self.last_copy_seconds = m.start.elapsed_time(m.event) * 1e-3 if m.event else None
        if self.last_copy_seconds and m.bytes:  # the host link's rate, for every cache
            _PagedTwoSided._move_rate = m.bytes / self.last_copy_seconds
        for b, h, h_new, k, pids_g, pids_h in m.downs:
            L = lens[b]
            held_g = int(g._pages_held[b])
            g.host_table[b, :held_g - k] = g.host_table[b, k:held_g].copy()
            g.host_table[b, held_g - k:held_g] = -1
            g._pages_held[b] = held_g - k
            hp0 = h // ps
            self.host.table[b, hp0:hp0 + k] = pids_h
            self.host.held[b] = hp0 + k
            self.host.lens[b] = h_new
            self._set_gpu_lens(b, L - h - k * ps)
            for pid in pids_g:
                g.pool.release(pid)
        for b, h, h_new, k, pids_g, pids_h in m.ups:
            L = lens[b]
            held_g = int(g._pages_held[b])
            if held_g + k > g.max_pages:
                m.kept.append(b)
                for pid in pids_g:
                    g.pool.release(pid)
                continue
            g.host_table[b, k:held_g + k] = g.host_table[b, :held_g].copy()
            g.host_table[b, :k] = pids_g
            g._pages_held[b] = held_g + k
            hp1 = h // ps
            self.host.table[b, hp1 - k:hp1] = 0
            self.host.held[b] = hp1 - k
            self.host.lens[b] = h_new
            self._set_gpu_lens(b, L - h + k * ps)
            for pid in pids_h:
                self.host.pool.release(pid)
        for b in sorted({e[0] for e in m.downs + m.ups}):
            self._write_gpu_row(b)

    # -- page copies through pinned staging ------------------------------------

    STAGE_BYTES = 32 << 20  # per staging buffer (two of them, allocated once)

    def _stages(self):
        """Two pinned staging buffers (page copies alternate between them so the
        host-side gather or scatter of one chunk overlaps the other's PCIe
        transfer)."""
        if getattr(self, "_stage", None) is None:
            pin = self.gpu.device.type == "cuda"
            self._stage = [torch.empty(self.STAGE_BYTES, dtype=torch.uint8, pin_memory=pin)
                           for _ in range(2)]
            self._stage_ev = [None, None]
        return self._stage

    def _chunks(self, hp, n):
        per_page = hp.shape[0] * hp[0, 0].numel() * hp.element_size()
        step = max(1, self.STAGE_BYTES // per_page)
        return [(i, min(n, i + step)) for i in range(0, n, step)]

    def _stage_view(self, k, hp, n):
        return self._stage[k][:hp.shape[0] * n * hp[0, 0].numel() * hp.element_size()].view(
            hp.dtype).view(hp.shape[0], n, *hp.shape[2:])

    def _wait_stage(self, k):
        ev = self._stage_ev[k]
        if ev is not None:
            ev.synchronize()
            self._stage_ev[k] = None

    def _record_stage(self, k):
        if self.gpu.device.type == "cuda":
            ev = torch.cuda.Event()
            ev.record()
            self._stage_ev[k] = ev

    def _pages_to_gpu(self, gp, hp, pids_g, pids_h):
        """gp[:, pids_g] = hp[:, pids_h] for every layer through pinned staging
        (an unpinned host pool; pinned pools are copied by the library's
        page-copy kernel in begin_boundaries)."""
        dev = self.gpu.device
        self._stages()
        ig = torch.tensor(pids_g, dtype=torch.int64, device=dev)
        ih = torch.tensor(pids_h, dtype=torch.int64)
        for c, (lo, hi) in enumerate(self._chunks(hp, len(pids_g))):
            k = c & 1
            self._wait_stage(k)  # its previous transfer has been read
            view = self._stage_view(k, hp, hi - lo)
            torch.index_select(hp, 1, ih[lo:hi], out=view)
            gp.index_copy_(1, ig[lo:hi], view.to(dev, non_blocking=True))
            self._record_stage(k)
        for k in (0, 1):
            self._wait_stage(k)

    def _pages_to_host(self, gp, hp, pids_g, pids_h):
        """hp[:, pids_h] = gp[:, pids_g] for every layer through pinned staging
        (an unpinned host pool)."""
        dev = self.gpu.device
        self._stages()
        ig = torch.tensor(pids_g, dtype=torch.int64, device=dev)
        ih = torch.tensor(pids_h, dtype=torch.int64)
        pending = None  # (stage index, lo, hi) copied but not yet scattered
        for c, (lo, hi) in enumerate(self._chunks(hp, len(pids_g))):
            k = c & 1
            view = self._stage_view(k, hp, hi - lo)
            view.copy_(gp.index_select(1, ig[lo:hi]), non_blocking=True)
            self._record_stage(k)
            if pending is not None:
                pk, plo, phi = pending
                self._wait_stage(pk)
                hp.index_copy_(1, ih[plo:phi], self._stage_view(pk, hp, phi - plo))
            pending = (k, lo, hi)
        pk, plo, phi = pending
        self._wait_stage(pk)
        hp.index_copy_(1, ih[plo:phi], self._stage_view(pk, hp, phi - plo))

    # -- decode-step plumbing -----------------------------------------------

    def _pinned(self, name, shape, dtype, stream=0):
        """A pinned host buffer of the cache, allocated once per (name, shape,
        stream).  One buffer per role and stream is enough: every host
        partial waits for the query copy of its own layer, which its stream
        orders after the previous layer's merge on that stream, the last
        reader of the same buffers.  Layers run on different streams get
        different buffers, since nothing orders one stream's merge before
        another stream's next host partial."""
        bufs = self.__dict__.setdefault("_pin_bufs", {})
        key = (name, tuple(shape), dtype, stream)
        t = bufs.get(key)
        if t is None:
            t = torch.empty(shape, dtype=dtype, pin_memory=True)
            bufs[key] = t
        return t

    def _layer_args(self, layer: int, cls):
        """The layer driver's argument structure of `layer`, one per layer and
        reused step after step: the fields no step changes (the pools, page
        tables and paging of both sides, all allocated once with the cache)
        are set when it is built, and a step writes the others."""
        wl = self.__dict__.setdefault("_wl_args", {})
        a = wl.get(layer)
        if a is None:
            a = wl[layer] = cls()
            data = self.host.data
            if len(data) == 1:  # MLA: one latent pool
                a.host_latent = data[0][layer].data_ptr()
            else:  # GQA: K and V pools
                a.host_k, a.host_v = data[0][layer].data_ptr(), data[1][layer].data_ptr()
            a.host_table = self.host.table_t.data_ptr()
            a.host_lens = self.host.lens_t.data_ptr()
            a.host_page_size = self.page_size
            a.host_max_pages = self.host.table.shape[1]
            a.host_num_pages = self.host.num_pages
            g = self.gpu
            a.page_table = g.page_table.data_ptr()
            a.B, a.page_size = self.batch, g.page_size
            a.max_pages, a.num_pages = g.page_table.shape[1], g.num_pages
            self._gpu_static_args(a, layer)
        if self.controller is not None:
            e0, e1 = self._timing[layer]
            a.ev_step_begin, a.ev_step_end = e0.cuda_event, e1.cuda_event
        elif a.ev_step_begin:
            a.ev_step_begin = a.ev_step_end = None
        return a

    def _gpu_static_args(self, a, layer: int) -> None:
        """The GPU pools of `layer` in its driver structure (per subclass)."""
        raise NotImplementedError

    def _step_args(self, a, layer: int, rows: int, threads: int, max_len: int, nwg: int,
                   ws, out_g, lse_g, q_bufs, out_shape) -> None:
        """The fields of the driver structure a step sets: lengths, plan,
        workspace and split partials, the pinned query copies and the pinned
        bf16 / fp32 host partial (pinned buffers are allocated once per shape)."""
        a.len_in, a.len_out = self.gpu.len_ptrs(layer)
        a.max_len, a.n_splits = max_len, nwg
        a.out_g, a.lse_g = out_g.data_ptr(), lse_g.data_ptr()
        a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
        dev = self.gpu.device
        sk = torch.cuda.current_stream(dev).cuda_stream if dev.type == "cuda" else 0
        for name, shape in q_bufs:
            setattr(a, name, self._pinned(name, shape, torch.bfloat16, sk).data_ptr())
        a.host_threads = int(threads)
        a.out_h = self._pinned("out", out_shape, torch.bfloat16, sk).data_ptr()
        a.lse_h = self._pinned("lse", (rows,), torch.float32, sk).data_ptr()

    def _run_layer(self, layer: int, fn, a, dev) -> None:
        """Runs the layer driver; the device lengths advanced as soon as the
        split step was launched, so the host bookkeeping follows them even
        when a later stage fails."""
        try:
            run_layer(fn, a, ops._stream(dev))
        except WlError as e:
            if e.stage >= 1:
                self.gpu.advance(layer)
            raise
        self.gpu.advance(layer)
        if self.controller is not None:
            self._layer_done(layer, a.host_seconds)

    # -- online share control --------------------------------------------------

    controller = None  # a scheduler.ShareController, or None
    _step_end = None  # perf_counter at the end of the last step's bookkeeping
    _step_t0 = None  # perf_counter at the end of the current step's first layer

    async_moves = False  # controller moves: begin_boundaries (True) or set_boundaries

    def attach(self, controller, async_moves: bool = False) -> None:
        """Let `controller` (scheduler.ShareController) move the boundary after
        every decode step, from the per-layer times this cache measures.
        With async_moves, a move's page copies run under the following decode
        steps (begin_boundaries) and the cache switches to the new boundaries
        after the first step that ends with them done; otherwise the decode
        loop waits for the copies (set_boundaries)."""
        self.controller = controller
        self.async_moves = async_moves
        self._timing = [(torch.cuda.Event(enable_timing=True),
                         torch.cuda.Event(enable_timing=True)) for _ in range(self.num_layers)]
        for e0, e1 in self._timing:  # create the events (the layer driver records them)
            e0.record()
            e1.record()
        self._layer_log = []

    def _layer_done(self, layer: int, host_s: float) -> None:
        """Record a layer's partials for the controller; after the last layer
        of a decode step, fold them into the scheduler and move the boundary
        if it chooses to."""
        g = self.gpu
        if layer == 0:
            self._step_t0 = time.perf_counter()
        self._layer_log.append((layer, float(g.lens[layer].sum()), float(self.host.lens.sum()),
                                host_s))
        if layer != self.num_layers - 1:
            return
        try:
            self._step_done()
        finally:
            self._step_end = time.perf_counter()

    def _step_done(self) -> None:
        """After the last layer of a decode step: the controller's part."""
        ctl = self.controller
        bpt = ctl.bytes_per_token
        for l, g_tok, h_tok, h_s in self._layer_log:
            a, e = self._timing[l]
            e.synchronize()
            ctl.observe_layer(g_tok * bpt, a.elapsed_time(e) * 1e-3, h_tok * bpt, h_s)
        self._layer_log = []
        now = time.perf_counter()
        if self._step_end is not None:
            step_s = now - self._step_end
        elif self._step_t0 is not None and self.num_layers > 1:
            # the first step: from the end of its first layer, scaled to all
            step_s = (now - self._step_t0) * self.num_layers / (self.num_layers - 1)
        else:
            step_s = None
        m = self._move
        if m is not None:
            t0 = now
            done = self.poll_boundaries()
            if not done and step_s is not None:
                # wait for the copies when what is left of them is shorter
                # than what the next step saves at the new boundaries (the
                # scheduler's prediction), or than a small part of a step
                left = m.bytes / self._move_rate - (now - m.t_begin)
                if left < max(self.MOVE_WAIT_FRACTION * step_s, self._switch_gain(m)):
                    self.finish_boundaries()
                    done = True
            if done and m.info is not None:
                step, r0, r1, t_begin, stall = m.info
                t1 = time.perf_counter()
                ctl.record_move(r0, r1, m.pages, t1 - t_begin, stall + t1 - t0, step=step,
                                copy_seconds=self.last_copy_seconds)
        lens = [self.seq_len(b) for b in range(self.batch)]
        host_now = [int(x) for x in self.host.lens]
        targets = ctl.decide(lens, host_now, moving=self._move is not None)
        if targets is None:
            return
        r0, want = ctl.share_of(lens, host_now), ctl.share_of(lens, targets)
        # what the pools and the partition can take now, one GPU page per
        # sequence kept free for the appends of the next steps
        targets = self.feasible_targets(targets, gpu_reserve=self.batch)
        r1 = ctl.share_of(lens, targets)
        if r1 != want:
            ctl.amend_last_share(r1)
        if targets == host_now:
            ctl.record_skip(r0, want, "no free pages for the move")
            return
        # the step's outputs are already queued: a move that cannot start is
        # recorded and skipped, never raised out of the step
        if self.async_moves and self.MOVE_STEP_FRACTION is not None and step_s is not None:
            cap = int(self.MOVE_STEP_FRACTION * step_s * self._move_rate / self._page_bytes())
            targets = self.paced_targets(targets, max(1, cap))
            r1 = ctl.share_of(lens, targets)
            ctl.amend_last_share(r1)
        try:
            if self.async_moves:
                t0 = time.perf_counter()
                if self.begin_boundaries(targets):
                    self._move.info = (ctl.steps, r0, r1, t0, time.perf_counter() - t0)
                return
            if self.gpu.device.type == "cuda":
                torch.cuda.synchronize()
            t0 = time.perf_counter()
            self.set_boundaries(targets)
        except (MemoryError, ValueError) as e:
            ctl.amend_last_share(r0)
            ctl.record_skip(r0, r1, str(e))
            return
        pages = sum(abs(t - h) for t, h in zip(targets, host_now)) // self.page_size
        ctl.record_move(r0, r1, pages, time.perf_counter() - t0)

    def _switch_gain(self, m) -> float:
        """Seconds one decode step is predicted to save at move m's
        boundaries over the current ones (0 when unknown)."""
        if m.info is None or self.controller is None:
            return 0.0
        ctl = self.controller
        _, r0, r1, _, _ = m.info
        layer_bytes = float(sum(self.seq_len(b) for b in range(self.batch))) * ctl.bytes_per_token
        try:
            t0 = ctl.sched.predict(r0, layer_bytes)["layer"]
            t1 = ctl.sched.predict(r1, layer_bytes)["layer"]
        except ValueError:
            return 0.0
        return max(0.0, (t0 - t1) * self.num_layers)

    def _page_bytes(self) -> int:
        """Bytes one page of a sequence moves: all layers, every payload."""
        return sum(p[0, 0].numel() * p.element_size() * p.shape[0] for p in self._gpu_payload())

    def paced_targets(self, targets, max_pages: int) -> list:
        """targets[b] host tokens with the move cut to at most max_pages pages
        in all: every sequence moves the same fraction of its way (rounded
        down to pages), and the pages left by the rounding go to the first
        sequences still short of their targets."""
        ps = self.page_size
        cur = [int(x) for x in self.host.lens]
        want = [abs(int(t) - h) // ps for t, h in zip(targets, cur)]
        total = sum(want)
        if total <= max_pages:
            return [int(t) for t in targets]
        take = [k * max_pages // total for k in want]
        left = max_pages - sum(take)
        for b in range(len(take)):
            if left <= 0:
                break
            if take[b] < want[b]:
                take[b] += 1
                left -= 1
        return [h + (k * ps if int(t) > h else -k * ps)
                for t, h, k in zip(targets, cur, take)]

    def feasible_targets(self, targets, gpu_reserve: int = 0) -> list:
        """targets[b] host tokens, each move cut down to what can start now:
        a move toward the GPU by the free GPU pages (less gpu_reserve) and the
        sequence's partition capacity, a move toward the host by the free host
        pages, sequence by sequence in order.  (Pages a move frees come back
        only at its switch, so they do not count.)"""
        ps = self.page_size
        g = self.gpu
        free_g = g.pool.free - gpu_reserve
        free_h = self.host.pool.free
        out = []
        for b, hn in enumerate(targets):
            h, hn = int(self.host.lens[b]), int(hn)
            if hn < h:
                k = min((h - hn) // ps, max(0, free_g), g.max_pages - int(g._pages_held[b]))
                k = max(0, k)
                free_g -= k
                hn = h - k * ps
            elif hn > h:
                k = min((hn - h) // ps, max(0, free_h))
                free_h -= k
                hn = h + k * ps
            out.append(hn)
        return out


class PagedMlaCache(_PagedTwoSided):
    """Absorbed-MLA latent cache (DeepSeek-V2-Lite: 16 heads, 512 + 64) with a
    paged host segment and an HBM partition."""

    def __init__(self, num_layers, batch, max_tokens, page_size=64, host_pages=None,
                 gpu_pages=None, device="cuda", pin=True):
        self.gpu = MlaGpuPartition(num_layers, batch, max_tokens, page_size, gpu_pages, device)
        super().__init__(num_layers, batch, max_tokens, page_size, host_pages, pin)

    def _page_shapes(self):
        return [(self.page_size, ops.MLA_LATENT)]

    def _gpu_payload(self):
        return [self.gpu.latent]

    def _gpu_static_args(self, a, layer: int) -> None:
        a.latent_pages = self.gpu.latent[layer].data_ptr()

    def load(self, layer: int, b: int, c_kv: torch.Tensor, k_pe: torch.Tensor,
             host_tokens: int) -> None:
        """Prefill sequence b of `layer` with c_kv [L, 512], k_pe [L, 64] (CPU
        bf16): tokens [0, host_tokens) to host pages, the rest to HBM.  Load
        the layers of a sequence with the same split."""
        ps = self.page_size
        L = c_kv.shape[0]
        self._check_no_move("load")
        if host_tokens % ps or not 0 <= host_tokens <= L:
            raise ValueError(f"host_tokens must be a page multiple in [0, {L}]")
        if layer == 0:
            self._host_reserve(b, host_tokens)
            self.host.lens[b] = host_tokens
        elif int(self.host.lens[b]) != host_tokens:
            raise ValueError("every layer of a sequence takes the same split")
        lat = torch.cat([c_kv, k_pe], dim=1)
        pool = self.host.data[0][layer]
        for p in range(host_tokens // ps):
            pool[int(self.host.table[b, p])].copy_(lat[p * ps:(p + 1) * ps])
        if L > host_tokens:
            dev = self.gpu.device
            self.gpu.load_sequence(layer, b, c_kv[host_tokens:].to(dev),
                                   k_pe[host_tokens:].to(dev))

    def step(self, layer: int, q_nope: torch.Tensor, q_pe: torch.Tensor,
             c_new: torch.Tensor, pe_new: torch.Tensor, scale: float, host_threads: int = 0,
             n_workgroups: int = 0, w_uv: torch.Tensor | None = None,
             return_lse: bool = False):
        """One decode step of `layer`: append c_new [B, 1, 512] / pe_new
        [B, 1, 64] to the GPU side and attend over both sides.  q_nope
        [B*16, 512] (W_UK-absorbed), q_pe [B*16, 64] on the GPU.  Returns the
        merged latent [B*16, 512] bf16, or with w_uv [16, Dout, 512] the
        projected attention output [B, 16 * Dout] bf16 (the merge and the
        W_UV epilogue in one launch), ready for o_proj.  With return_lse, a
        pair (that output, merged lse [B*16] fp32)."""
        g = self.gpu
        H = g.check_step_inputs(q_nope, q_pe, c_new, pe_new)
        B = self.batch
        rows = B * H
        dev = q_nope.device
        if w_uv is not None:
            if w_uv.dtype != torch.bfloat16 or w_uv.device != dev or w_uv.dim() != 3 or \
                    w_uv.shape[0] != H or w_uv.shape[2] != ops.MLA_C or \
                    not w_uv.is_contiguous() or w_uv.shape[1] % 32 or w_uv.shape[1] > 512:
                raise ValueError(f"w_uv must be a contiguous bf16 [{H}, Dout, 512] on {dev}, "
                                 "Dout a multiple of 32 up to 512")
        max_len, nwg, ws, out_g, lse_g = g.prepare_split(layer, H, n_workgroups)
        a = self._layer_args(layer, WlMlaLayer)
        a.q_nope, a.q_pe = q_nope.data_ptr(), q_pe.data_ptr()
        a.c_new, a.c_stride = c_new.data_ptr(), c_new.stride(0)
        a.pe_new, a.pe_stride = pe_new.data_ptr(), pe_new.stride(0)
        a.H, a.scale = H, float(scale)
        self._step_args(a, layer, rows, host_threads, max_len, nwg, ws, out_g, lse_g,
                        q_bufs=(("q_nope_h", (rows, ops.MLA_C)), ("q_pe_h", (rows, ops.MLA_PE))),
                        out_shape=(rows, ops.MLA_C))
        lse_out = torch.empty((rows,), dtype=torch.float32, device=dev) if return_lse else None
        a.lse_out = lse_out.data_ptr() if return_lse else None
        if w_uv is None:
            res = torch.empty((rows, ops.MLA_C), dtype=torch.bfloat16, device=dev)
            a.out, a.w_uv, a.Dout, a.out_v = res.data_ptr(), None, 0, None
        else:
            Dout = w_uv.shape[1]
            res = torch.empty((B, H * Dout), dtype=torch.bfloat16, device=dev)
            a.out, a.w_uv, a.Dout, a.out_v = None, w_uv.data_ptr(), Dout, res.data_ptr()
        self._run_layer(layer, layer_lib().wl_mla_layer, a, dev)
        return (res, lse_out) if return_lse else res


class PagedKVCache(_PagedTwoSided):
    """GQA KV cache with a paged host segment and an HBM partition."""

    def __init__(self, num_layers, batch, num_kv_heads, head_dim, max_tokens, page_size=64,
                 host_pages=None, gpu_pages=None, device="cuda", pin=True):
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.gpu = GqaGpuPartition(num_layers, batch, num_kv_heads, head_dim, max_tokens,
                                   page_size, gpu_pages, device)
        super().__init__(num_layers, batch, max_tokens, page_size, host_pages, pin)

    def _page_shapes(self):
        s = (self.num_kv_heads, self.page_size, self.head_dim)
        return [s, s]

    def _gpu_payload(self):
        return [self.gpu.k, self.gpu.v]

    def _gpu_static_args(self, a, layer: int) -> None:
        a.k_pages, a.v_pages = self.gpu.k[layer].data_ptr(), self.gpu.v[layer].data_ptr()
        a.Hkv, a.D = self.num_kv_heads, self.head_dim

    def load(self, layer: int, b: int, k: torch.Tensor, v: torch.Tensor,
             host_tokens: int) -> None:
        """Prefill sequence b of `layer` with k, v [Hkv, L, D] (CPU bf16):
        tokens [0, host_tokens) to host pages, the rest to HBM."""
        ps = self.page_size
        L = k.shape[1]
        self._check_no_move("load")
        if host_tokens % ps or not 0 <= host_tokens <= L:
            raise ValueError(f"host_tokens must be a page multiple in [0, {L}]")
        if layer == 0:
            self._host_reserve(b, host_tokens)
            self.host.lens[b] = host_tokens
        elif int(self.host.lens[b]) != host_tokens:
            raise ValueError("every layer of a sequence takes the same split")
        kp, vp = self.host.data[0][layer], self.host.data[1][layer]
        for p in range(host_tokens // ps):
            pid = int(self.host.table[b, p])
            kp[pid].copy_(k[:, p * ps:(p + 1) * ps])
            vp[pid].copy_(v[:, p * ps:(p + 1) * ps])
        if L > host_tokens:
            dev = self.gpu.device
            self.gpu.load_sequence(layer, b, k[:, host_tokens:].to(dev),
                                   v[:, host_tokens:].to(dev))

    def step(self, layer: int, q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor,
             scale: float, host_threads: int = 0, n_workgroups: int = 0,
             return_lse: bool = False):
        """One decode step of `layer`: append k_new / v_new [B, Hkv, 1, D] to the
        GPU side and attend over both sides.  q [B, Hq, D] on the GPU.
        Returns [B, Hq, D] bf16; with return_lse, a pair (that output,
        merged lse [B, Hq] fp32)."""
        g = self.gpu
        k_new, v_new = g.check_step_inputs(q, k_new, v_new)
        B, Hq, D = q.shape
        dev = q.device
        max_len, nwg, ws, out_g, lse_g = g.prepare_split(layer, Hq, n_workgroups)
        a = self._layer_args(layer, WlGqaLayer)
        a.q, a.k_new, a.v_new = q.data_ptr(), k_new.data_ptr(), v_new.data_ptr()
        a.Hq, a.scale = Hq, float(scale)
        self._step_args(a, layer, B * Hq, host_threads, max_len, nwg, ws, out_g, lse_g,
                        q_bufs=(("q_h", (B, Hq, D)),), out_shape=(B, Hq, D))
        res = torch.empty((B, Hq, D), dtype=torch.bfloat16, device=dev)
        lse_out = torch.empty((B, Hq), dtype=torch.float32, device=dev) if return_lse else None
        a.out, a.lse_out = res.data_ptr(), (lse_out.data_ptr() if return_lse else None)
        self._run_layer(layer, layer_lib().wl_gqa_layer, a, dev)
        return (res, lse_out) if return_lse else res


def absorb_q(q_nope: torch.Tensor, w_uk: torch.Tensor) -> torch.Tensor:
    """The q-side W_UK absorption of the MLA decode (system/deepseek.py:256-263):
    q_nope [B, H, 128] times W_UK[h] [128, 512] per head -> [B*H, 512] bf16,
    the q_nope the MLA step takes.  A plain batched GEMM (torch, per head with
    contiguous operands), not a hand-written kernel."""
    B, H, D = q_nope.shape
    if w_uk.shape[:2] != (H, D):
        raise ValueError(f"w_uk must be [{H}, {D}, latent]")
    q = torch.bmm(q_nope.transpose(0, 1).contiguous(), w_uk.contiguous())  # [H, B, latent]
    return q.transpose(0, 1).reshape(B * H, w_uk.shape[2]).contiguous()
