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

A decode step per layer: q to pinned host memory; the GPU split step
(append + partial over the HBM pages); the native host partial over the host
pages in the calling thread while the GPU runs; its (out, lse) to the GPU;
ws_merge_split.  Lengths are the same in every layer between steps; migrate
only then.
"""
from __future__ import annotations

import numpy as np
import torch

from . import host, ops
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

    # -- filling -------------------------------------------------------------

    def _load_host(self, layer: int, b: int, tensors) -> None:
        """Host tokens [0, n) of sequence b in `layer` from CPU payload rows
        shaped like a page with the token axis holding n (page axis -2 for GQA
        K/V [Hkv, n, D], axis 0 for MLA [n, 576])."""
        raise NotImplementedError

    # -- boundary movement ---------------------------------------------------

    def set_boundary(self, b: int, h_new: int) -> None:
        """Move sequence b's boundary to h_new host tokens (a multiple of the
        page size, at most its length), copying pages between the sides in
        every layer."""
        ps = self.page_size
        L = self.seq_len(b)
        h = int(self.host.lens[b])
        if h_new % ps or not 0 <= h_new <= L:
            raise ValueError(f"boundary {h_new} must be a multiple of {ps} in [0, {L}]")
        if h_new == h:
            return
        g = self.gpu
        k = abs(h_new - h) // ps
        gpu_tok = L - h
        dev = g.device
        if h_new > h:  # GPU's leading k pages -> host
            held_g = int(g._pages_held[b])
            pids_g = g.host_table[b, :k].copy()
            hp0 = int(self.host.held[b])
            self._host_reserve(b, h_new)
            pids_h = self.host.table[b, hp0:hp0 + k].copy()
            ig = torch.from_numpy(pids_g.astype(np.int64)).to(dev)
            ih = torch.from_numpy(pids_h.astype(np.int64))
            for gp, hp in zip(self._gpu_payload(), self.host.data):
                for layer in range(self.num_layers):
                    hp[layer].index_copy_(0, ih, gp[layer].index_select(0, ig).cpu())
            g.host_table[b, :held_g - k] = g.host_table[b, k:held_g]
            g.host_table[b, held_g - k:held_g] = -1
            g._pages_held[b] = held_g - k
            for pid in pids_g:
                g.pool.release(int(pid))
            self._set_gpu_lens(b, gpu_tok - k * ps)
        else:  # host's trailing k pages -> GPU
            held_g = int(g._pages_held[b])
            if held_g + k > g.max_pages:
                raise ValueError(f"sequence {b}: GPU partition capacity exceeded")
            hp1 = h // ps
            pids_h = self.host.table[b, hp1 - k:hp1].copy()
            pids_g = np.array([g.pool.alloc() for _ in range(k)], np.int32)
            ig = torch.from_numpy(pids_g.astype(np.int64)).to(dev)
            ih = torch.from_numpy(pids_h.astype(np.int64))
            for gp, hp in zip(self._gpu_payload(), self.host.data):
                for layer in range(self.num_layers):
                    gp[layer].index_copy_(0, ig, hp[layer].index_select(0, ih).to(dev))
            g.host_table[b, k:held_g + k] = g.host_table[b, :held_g].copy()
            g.host_table[b, :k] = pids_g
            g._pages_held[b] = held_g + k
            for pid in pids_h:
                self.host.pool.release(int(pid))
            self.host.table[b, hp1 - k:hp1] = 0
            self.host.held[b] = hp1 - k
            self._set_gpu_lens(b, gpu_tok + k * ps)
        self.host.lens[b] = h_new
        self._write_gpu_row(b)

    def set_share(self, r: float) -> None:
        """GPU share r for every sequence: host tokens L - floor(r L), rounded
        down to a page multiple (the GPU takes the remainder)."""
        if not 0.0 <= r <= 1.0:
            raise ValueError(f"share {r} outside [0, 1]")
        for b in range(self.batch):
            L = self.seq_len(b)
            h = L - int(np.floor(r * L))
            self.set_boundary(b, (h // self.page_size) * self.page_size)

    # -- decode-step plumbing -----------------------------------------------

    @staticmethod
    def _to_host(*ts):
        out = []
        for t in ts:
            h = torch.empty(t.shape, dtype=t.dtype, pin_memory=True)
            h.copy_(t, non_blocking=True)
            out.append(h)
        ev = torch.cuda.Event()
        ev.record()
        return out, ev

    def _merge(self, step, part, dev):
        if part is None:
            out, _ = ops.merge_split(step, None, want_lse=False)
            return out
        b = tuple(x.to(dev, non_blocking=True) for x in part)
        out, _ = ops.merge_split(step, b, ops.PARTIAL_LSE_F32, want_lse=False)
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

    def load(self, layer: int, b: int, c_kv: torch.Tensor, k_pe: torch.Tensor,
             host_tokens: int) -> None:
        """Prefill sequence b of `layer` with c_kv [L, 512], k_pe [L, 64] (CPU
        bf16): tokens [0, host_tokens) to host pages, the rest to HBM.  Load
        the layers of a sequence with the same split."""
        ps = self.page_size
        L = c_kv.shape[0]
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
             n_workgroups: int = 0) -> torch.Tensor:
        """One decode step of `layer`: append c_new [B, 1, 512] / pe_new
        [B, 1, 64] to the GPU side and attend over both sides.  q_nope
        [B*16, 512], q_pe [B*16, 64] on the GPU.  Returns [B*16, 512] bf16."""
        g = self.gpu
        dev = q_nope.device
        with_host = bool(self.host.lens.any())
        if with_host:
            (qn_h, qp_h), ev = self._to_host(q_nope, q_pe)
        for b in range(self.batch):
            g.reserve(b, int(g.lens[layer, b]) + 1)
        step = ops.mla_append_decode_split(q_nope, q_pe, c_new, pe_new, g.latent[layer],
                                           g.page_table, g.len_dev(layer), g._len_next(layer),
                                           scale, g.max_len(layer) + 1, n_workgroups)
        g._flip(layer)
        g.lens[layer] += 1
        part = None
        if with_host:
            ev.synchronize()
            rows = q_nope.shape[0]
            part = host.mla_partial(
                qn_h, qp_h, self.host.data[0][layer], self.host.table_t, self.host.lens_t,
                scale, host_threads,
                torch.empty((rows, ops.MLA_C), dtype=torch.float32, pin_memory=True),
                torch.empty((rows,), dtype=torch.float32, pin_memory=True))
        return self._merge(step, part, dev)


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

    def load(self, layer: int, b: int, k: torch.Tensor, v: torch.Tensor,
             host_tokens: int) -> None:
        """Prefill sequence b of `layer` with k, v [Hkv, L, D] (CPU bf16):
        tokens [0, host_tokens) to host pages, the rest to HBM."""
        ps = self.page_size
        L = k.shape[1]
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
             scale: float, host_threads: int = 0, n_workgroups: int = 0) -> torch.Tensor:
        """One decode step of `layer`: append k_new / v_new [B, Hkv, 1, D] to the
        GPU side and attend over both sides.  q [B, Hq, D] on the GPU.
        Returns [B, Hq, D] bf16."""
        g = self.gpu
        dev = q.device
        with_host = bool(self.host.lens.any())
        if with_host:
            (q_h,), ev = self._to_host(q)
        for b in range(self.batch):
            g.reserve(b, int(g.lens[layer, b]) + 1)
        step = ops.gqa_append_decode_split(q, k_new.contiguous(), v_new.contiguous(),
                                           g.k[layer], g.v[layer], g.page_table,
                                           g.len_dev(layer), g._len_next(layer), scale,
                                           g.max_len(layer) + 1, n_workgroups)
        g._flip(layer)
        g.lens[layer] += 1
        part = None
        if with_host:
            ev.synchronize()
            B, Hq, D = q.shape
            part = host.gqa_partial(
                q_h, self.host.data[0][layer], self.host.data[1][layer], self.host.table_t,
                self.host.lens_t, scale, host_threads,
                torch.empty((B, Hq, D), dtype=torch.float32, pin_memory=True),
                torch.empty((B, Hq), dtype=torch.float32, pin_memory=True))
        return self._merge(step, part, dev).view(q.shape)
