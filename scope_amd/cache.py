"""Paged HBM partitions of the decode KV cache, and host+GPU partitioned caches.

GqaGpuPartition / MlaGpuPartition hold the GPU-affinity token range of every
sequence in fixed-size HBM pages (default 64 tokens):
  GQA  k, v       [num_layers, num_pages, Hkv, page_size, D] bf16
  MLA  latent     [num_layers, num_pages, page_size, 576]    bf16
  page_table      [B, max_pages] int32 (shared by all layers)
  lengths         two device arrays [2, num_layers, B] int32 + a host mirror:
                  a fused decode step (step()) reads one array and writes the
                  other, then the layer's current array flips
Pages come from a free list and are assigned on the host before an append
needs them; the device page table is updated only when a sequence crosses a
page boundary (once per 64 decode steps).

PartitionedLatentCache mirrors the reference's token-range-partitioned MLA
cache (system/deepseek.py:144-209): the leading `gs` tokens of each sequence
in pinned host memory, the rest in an MlaGpuPartition.
PartitionedKVCache is the GQA analogue (system/mixoffload.py:51-144 holds the
whole cache on the host; here the trailing range lives in HBM).
"""
from __future__ import annotations

import numpy as np
import torch

from . import ops
from .partition import boundary_split, pages_for


class PagePool:
    """Free list of physical page ids."""

    def __init__(self, num_pages: int):
        self.num_pages = num_pages
        self._free = list(range(num_pages - 1, -1, -1))

    def alloc(self) -> int:
        if not self._free:
            raise MemoryError("HBM page pool exhausted")
        return self._free.pop()

    def release(self, pid: int) -> None:
        self._free.append(pid)

    @property
    def free(self) -> int:
        return len(self._free)


class _PagedBase:
    def __init__(self, num_layers, batch, max_tokens, page_size, num_pages, device):
        if page_size <= 0 or page_size % 32:
            raise ValueError("page_size must be a positive multiple of 32")
        self.device = torch.device(device)
        self.num_layers = num_layers
        self.batch = batch
        self.page_size = page_size
        self.max_pages = max(1, pages_for(max_tokens, page_size))
        self.num_pages = num_pages if num_pages is not None else batch * self.max_pages
        self.pool = PagePool(self.num_pages)
        self.host_table = np.full((batch, self.max_pages), -1, np.int32)
        self.page_table = torch.full((batch, self.max_pages), -1, dtype=torch.int32,
                                     device=self.device)
        self.lens = np.zeros((num_layers, batch), np.int64)  # host mirror
        self._len_bufs = torch.zeros((2, num_layers, batch), dtype=torch.int32,
                                     device=self.device)
        self._cur = np.zeros(num_layers, np.int64)
        self._pages_held = np.zeros(batch, np.int64)
        # addresses of the two length arrays of every layer (the step entry
        # points take raw pointers; indexing the tensor would build a view)
        lp = self._len_bufs.data_ptr()
        self._len_ptr = [[lp + 4 * batch * (k * num_layers + l) for l in range(num_layers)]
                         for k in range(2)]
        pd = self.page_table.device  # with its index
        self._dev_index = pd.index if pd.type != "cpu" else -1

    def len_ptrs(self, layer: int):
        """(address of the current device lengths of `layer`, address of the
        other array, which a fused step writes)."""
        c = int(self._cur[layer])
        return self._len_ptr[c][layer], self._len_ptr[1 - c][layer]

    def on_device(self, t: torch.Tensor) -> bool:
        """Whether t is a bf16 tensor on this partition's device."""
        if t.dtype is not torch.bfloat16:
            return False
        if self._dev_index < 0:
            return not t.is_cuda
        return t.is_cuda and t.get_device() == self._dev_index

    def len_dev(self, layer: int) -> torch.Tensor:
        """Device lengths [B] of `layer` (the current one of its two arrays)."""
        return self._len_bufs[int(self._cur[layer]), layer]

    def _len_next(self, layer: int) -> torch.Tensor:
        return self._len_bufs[1 - int(self._cur[layer]), layer]

    def _flip(self, layer: int) -> None:
        self._cur[layer] = 1 - self._cur[layer]

    def reserve(self, b: int, n_tokens: int) -> None:
        """Make sure sequence b owns pages for its first n_tokens positions."""
        need = pages_for(n_tokens, self.page_size)
        if need > self.max_pages:
            raise ValueError(f"sequence {b}: {n_tokens} tokens exceed capacity "
                             f"{self.max_pages * self.page_size}")
        have = int(self._pages_held[b])
        if need <= have:
            return
        for p in range(have, need):
            self.host_table[b, p] = self.pool.alloc()
        self._pages_held[b] = need
        self.page_table[b, have:need].copy_(
            torch.from_numpy(self.host_table[b, have:need].copy()), non_blocking=False)

    def _reserve_next(self, layer: int, n: int) -> None:
        """reserve() for every sequence of `layer` about to grow by n tokens,
        touching only the sequences that need a new page."""
        need = (self.lens[layer] + n + self.page_size - 1) // self.page_size
        for b in np.nonzero(need > self._pages_held)[0]:
            self.reserve(int(b), int(self.lens[layer, b]) + n)

    def _partial_bufs(self, rows: int, Dv: int):
        """The split step's (out fp32 [rows, Dv], lse fp32 [rows]) buffers,
        reused step after step: like the workspace, they belong to the latest
        split step (its merge runs before the next step on the stream, and the
        workspace generation guard refuses an older step's merge)."""
        bufs = getattr(self, "_pbufs", None)
        if bufs is None or bufs[0].shape != (rows, Dv):
            bufs = (torch.empty((rows, Dv), dtype=torch.float32, device=self.device),
                    torch.empty((rows,), dtype=torch.float32, device=self.device))
            self._pbufs = bufs
        return bufs

    def reserve_all(self, n_tokens_per_seq) -> None:
        for b, n in enumerate(n_tokens_per_seq):
            self.reserve(b, int(n))

    def max_len(self, layer: int) -> int:
        return int(self.lens[layer].max()) if self.batch else 0

    def workspace(self, nbytes: int) -> torch.Tensor:
        """The partition's decode workspace, grown on demand.  Calls that
        share it are ordered on the device's stream."""
        ws = getattr(self, "_ws", None)
        if ws is None or ws.numel() < nbytes:
            ws = torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=self.device)
            self._ws = ws
        return ws

    def _split_workspace(self, kind: int, rows_kv: int, heads: int, max_len: int,
                         n_workgroups: int) -> torch.Tensor:
        _, wsb = ops.decode_plan(kind, rows_kv, heads, max_len, n_workgroups)
        return self._split_workspace_bytes(wsb)

    def _split_workspace_bytes(self, wsb: int) -> torch.Tensor:
        """The workspace for a split step of wsb bytes, under a new generation
        (an older split step's merge is refused from now on)."""
        self._ws_gen = getattr(self, "_ws_gen", 0) + 1
        return self.workspace(wsb)

    def _own(self, st: "ops.SplitStep") -> "ops.SplitStep":
        """Tie a split step to the current workspace generation: its merge
        refuses to run once a later step has reused the workspace."""
        st.guard = lambda gen=self._ws_gen: self._ws_gen == gen
        return st

    def reset(self) -> None:
        """Drop all tokens and return every page to the pool."""
        for b in range(self.batch):
            for p in range(int(self._pages_held[b])):
                self.pool.release(int(self.host_table[b, p]))
        self.host_table[:] = -1
        self.page_table.fill_(-1)
        self._pages_held[:] = 0
        self.lens[:] = 0
        self._len_bufs.zero_()
        self._cur[:] = 0


class GqaGpuPartition(_PagedBase):
    """HBM pages of the GPU token range of a GQA KV cache."""

    def __init__(self, num_layers, batch, num_kv_heads, head_dim, max_tokens,
                 page_size=64, num_pages=None, device="cuda"):
        super().__init__(num_layers, batch, max_tokens, page_size, num_pages, device)
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        shape = (num_layers, self.num_pages, num_kv_heads, page_size, head_dim)
        self.k = torch.empty(shape, dtype=torch.bfloat16, device=self.device)
        self.v = torch.empty(shape, dtype=torch.bfloat16, device=self.device)

    def append_4d(self, layer: int, k4d: torch.Tensor, v4d: torch.Tensor) -> None:
        """Append k4d/v4d [B, Hkv, n, D] to every sequence of `layer`
        (InplaceKVCache.append_4d, system/qwenoffload.py:100-118)."""
        n = k4d.shape[2]
        for b in range(self.batch):
            self.reserve(b, int(self.lens[layer, b]) + n)
        ops.kv_append(k4d.contiguous(), v4d.contiguous(), self.k[layer], self.v[layer],
                      self.page_table, self.len_dev(layer))
        self.lens[layer] += n

    def load_sequence(self, layer: int, b: int, k: torch.Tensor, v: torch.Tensor) -> None:
        """Append k, v [Hkv, n, D] to sequence b only (prefill of one row)."""
        n = k.shape[1]
        self.reserve(b, int(self.lens[layer, b]) + n)
        ops.kv_append(k.unsqueeze(0).contiguous(), v.unsqueeze(0).contiguous(),
                      self.k[layer], self.v[layer], self.page_table[b:b + 1],
                      self.len_dev(layer)[b:b + 1])
        self.lens[layer, b] += n

    def attend(self, layer: int, q: torch.Tensor, scale: float, n_workgroups=0):
        """GPU partial over the partition: q [B, Hq, D] -> (out fp32, lse fp32)."""
        return ops.gqa_decode_partial(q, self.k[layer], self.v[layer], self.page_table,
                                      self.len_dev(layer), scale, self.max_len(layer),
                                      n_workgroups)

    def step(self, layer: int, q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor,
             scale: float, n_workgroups=0):
        """One decode step in one launch: append k_new/v_new [B, Hkv, 1, D] and
        attend over the partition including them (the slot copy + attention of
        _resident_layer, roofline/bench_resident_kv.py:261-271).
        Returns (out [B, Hq, D] fp32, lse [B, Hq] fp32)."""
        for b in range(self.batch):
            self.reserve(b, int(self.lens[layer, b]) + 1)
        out = ops.gqa_append_decode_partial(
            q, k_new.contiguous(), v_new.contiguous(), self.k[layer], self.v[layer],
            self.page_table, self.len_dev(layer), self._len_next(layer), scale,
            self.max_len(layer) + 1, n_workgroups)
        self._flip(layer)
        self.lens[layer] += 1
        return out

    def check_step_inputs(self, q: torch.Tensor, k_new: torch.Tensor,
                          v_new: torch.Tensor):
        """The decode step's own inputs, checked (the pools, page table,
        lengths and buffers are the partition's).  Returns contiguous
        (k_new, v_new)."""
        B, Hkv, D = self.batch, self.num_kv_heads, self.head_dim
        k_new, v_new = k_new.contiguous(), v_new.contiguous()
        for t, n in ((q, "q"), (k_new, "k_new"), (v_new, "v_new")):
            if not self.on_device(t):
                raise ValueError(f"{n} must be bf16 on {self.page_table.device}")
        if q.dim() != 3 or q.shape[0] != B or q.shape[2] != D or q.shape[1] % Hkv or \
                not q.is_contiguous():
            raise ValueError(f"q must be a contiguous [{B}, Hq, {D}] with Hq a multiple of {Hkv}")
        if k_new.shape != (B, Hkv, 1, D) or v_new.shape != k_new.shape:
            raise ValueError(f"k_new/v_new must be [B, Hkv, 1, D] = {(B, Hkv, 1, D)}")
        return k_new, v_new

    def prepare_split(self, layer: int, Hq: int, n_workgroups: int = 0):
        """Pages for the step's new token, and (max_len, n_splits, workspace,
        out fp32 [B*Hq, D], lse fp32 [B*Hq]) of a split step of `layer` under
        a new workspace generation."""
        B, Hkv, D = self.batch, self.num_kv_heads, self.head_dim
        self._reserve_next(layer, 1)
        max_len = self.max_len(layer) + 1
        nwg, wsb = ops.gqa_plan(B * Hkv, Hq // Hkv, D, D, max_len, n_workgroups)
        ws = self._split_workspace_bytes(wsb)
        out, lse = self._partial_bufs(B * Hq, D)
        return max_len, nwg, ws, out, lse

    def advance(self, layer: int) -> None:
        """Bookkeeping after a fused step of `layer` was launched: the device
        lengths moved to the other array, one token more."""
        self._flip(layer)
        self.lens[layer] += 1

    def step_split(self, layer: int, q: torch.Tensor, k_new: torch.Tensor,
                   v_new: torch.Tensor, scale: float, n_workgroups=0) -> "ops.SplitStep":
        """step() with the combine of rows shared by several splits (one wave
        each) left to ops.merge_split, which does it in the same launch as the
        merge with the host partial.  Returns the ops.SplitStep to finish."""
        k_new, v_new = self.check_step_inputs(q, k_new, v_new)
        B, Hq, D = q.shape
        max_len, nwg, ws, out, lse = self.prepare_split(layer, Hq, n_workgroups)
        st = ops._gqa_split_launch(q, k_new, v_new, self.k[layer], self.v[layer],
                                   self.page_table, self.len_dev(layer), self._len_next(layer),
                                   scale, max_len, nwg, out.view(B, Hq, D), lse.view(B, Hq), ws)
        self.advance(layer)
        return self._own(st)


class MlaGpuPartition(_PagedBase):
    """HBM pages of the GPU token range of an absorbed-MLA latent cache."""

    def __init__(self, num_layers, batch, max_tokens, page_size=64, num_pages=None,
                 device="cuda"):
        super().__init__(num_layers, batch, max_tokens, page_size, num_pages, device)
        self.latent = torch.empty((num_layers, self.num_pages, page_size, ops.MLA_LATENT),
                                  dtype=torch.bfloat16, device=self.device)

    def append(self, layer: int, c_kv: torch.Tensor, k_pe: torch.Tensor) -> None:
        """Append c_kv [B, n, 512], k_pe [B, n, 64] to every sequence."""
        n = c_kv.shape[1]
        for b in range(self.batch):
            self.reserve(b, int(self.lens[layer, b]) + n)
        ops.latent_append(c_kv, k_pe, self.latent[layer], self.page_table,
                          self.len_dev(layer))
        self.lens[layer] += n

    def load_sequence(self, layer: int, b: int, c_kv: torch.Tensor, k_pe: torch.Tensor) -> None:
        """Append c_kv [n, 512], k_pe [n, 64] to sequence b only."""
        n = c_kv.shape[0]
        self.reserve(b, int(self.lens[layer, b]) + n)
        ops.latent_append(c_kv.unsqueeze(0).contiguous(), k_pe.unsqueeze(0).contiguous(),
                          self.latent[layer], self.page_table[b:b + 1],
                          self.len_dev(layer)[b:b + 1])
        self.lens[layer, b] += n

    def attend(self, layer: int, q_nope: torch.Tensor, q_pe: torch.Tensor, scale: float,
               n_workgroups=0):
        """GPU partial: q_nope [B*H, 512], q_pe [B*H, 64] -> (out, lse)."""
        return ops.mla_decode_partial(q_nope, q_pe, self.latent[layer], self.page_table,
                                      self.len_dev(layer), scale, self.max_len(layer),
                                      n_workgroups)

    def step(self, layer: int, q_nope: torch.Tensor, q_pe: torch.Tensor,
             c_new: torch.Tensor, pe_new: torch.Tensor, scale: float, n_workgroups=0):
        """One decode step in one call: append the new latent (c_new [B, 1, 512],
        pe_new [B, 1, 64]) and attend over the partition including it.
        Returns (out [B*H, 512] fp32, lse [B*H] fp32)."""
        for b in range(self.batch):
            self.reserve(b, int(self.lens[layer, b]) + 1)
        out = ops.mla_append_decode_partial(
            q_nope, q_pe, c_new, pe_new, self.latent[layer], self.page_table,
            self.len_dev(layer), self._len_next(layer), scale, self.max_len(layer) + 1,
            n_workgroups)
        self._flip(layer)
        self.lens[layer] += 1
        return out

    def check_step_inputs(self, q_nope: torch.Tensor, q_pe: torch.Tensor,
                          c_new: torch.Tensor, pe_new: torch.Tensor) -> int:
        """The decode step's own inputs, checked (the pool, page table, lengths
        and buffers are the partition's).  Returns the head count H."""
        B = self.batch
        rows = q_nope.shape[0] if q_nope.dim() == 2 else -1
        for t, n in ((q_nope, "q_nope"), (q_pe, "q_pe"), (c_new, "c_new"), (pe_new, "pe_new")):
            if not self.on_device(t):
                raise ValueError(f"{n} must be bf16 on {self.page_table.device}")
        if rows <= 0 or rows % (16 * B) or q_nope.shape[1] != ops.MLA_C or \
                q_pe.shape != (rows, ops.MLA_PE) or not q_nope.is_contiguous() or \
                not q_pe.is_contiguous():
            raise ValueError(f"q_nope / q_pe must be contiguous [B*H, 512] / [B*H, 64], "
                             f"H a multiple of 16, B = {B}")
        for t, n, w in ((c_new, "c_new", ops.MLA_C), (pe_new, "pe_new", ops.MLA_PE)):
            if t.shape != (B, 1, w) or t.stride(2) != 1:
                raise ValueError(f"{n} must be [B, 1, {w}] with unit last stride")
        return rows // B

    def prepare_split(self, layer: int, H: int, n_workgroups: int = 0):
        """Pages for the step's new token, and (max_len, n_splits, workspace,
        out fp32 [B*H, 512], lse fp32 [B*H]) of a split step of `layer` under
        a new workspace generation."""
        B = self.batch
        self._reserve_next(layer, 1)
        max_len = self.max_len(layer) + 1
        nwg, wsb = ops.decode_plan(1, B, H, max_len, n_workgroups)
        ws = self._split_workspace_bytes(wsb)
        out, lse = self._partial_bufs(B * H, ops.MLA_C)
        return max_len, nwg, ws, out, lse

    def advance(self, layer: int) -> None:
        """Bookkeeping after a fused step of `layer` was launched: the device
        lengths moved to the other array, one token more."""
        self._flip(layer)
        self.lens[layer] += 1

    def step_split(self, layer: int, q_nope: torch.Tensor, q_pe: torch.Tensor,
                   c_new: torch.Tensor, pe_new: torch.Tensor, scale: float,
                   n_workgroups=0) -> "ops.SplitStep":
        """step() with the combine of sequences held by several workgroups left
        to ops.merge_split / ops.merge_split_uv.  Returns the ops.SplitStep."""
        H = self.check_step_inputs(q_nope, q_pe, c_new, pe_new)
        max_len, nwg, ws, out, lse = self.prepare_split(layer, H, n_workgroups)
        st = ops._mla_split_launch(q_nope, q_pe, c_new, pe_new, self.latent[layer],
                                   self.page_table, self.len_dev(layer), self._len_next(layer),
                                   scale, max_len, nwg, out, lse, ws)
        self.advance(layer)
        return self._own(st)


class PartitionedLatentCache:
    """Token-range-partitioned MLA latent cache.

    Same contract as InplaceKVCacheCompressed (system/deepseek.py:144-209):
    the leading `gs` tokens of every sequence are the host segment (pinned
    c [B, gs, 512] and pe [B, gs, 64] per layer), positions >= gs go to the
    GPU partition.  append() splits new tokens at the boundary with the
    reference's arithmetic; get() returns the host views and the GPU partition.
    """

    def __init__(self, num_layers, batch, max_seq, gs, page_size=64, device="cuda"):
        if not 0 <= gs <= max_seq:
            raise ValueError("boundary gs must lie in [0, max_seq]")
        self.num_layers, self.batch, self.max_seq, self.gs = num_layers, batch, max_seq, gs
        pin = torch.cuda.is_available()
        self.host_c = [torch.empty((batch, gs, ops.MLA_C), dtype=torch.bfloat16,
                                   pin_memory=pin) for _ in range(num_layers)]
        self.host_pe = [torch.empty((batch, gs, ops.MLA_PE), dtype=torch.bfloat16,
                                    pin_memory=pin) for _ in range(num_layers)]
        self.gpu = MlaGpuPartition(num_layers, batch, max(max_seq - gs, 1), page_size,
                                   device=device)
        self._filled = [0] * num_layers

    def append(self, layer: int, c_kv: torch.Tensor, k_pe: torch.Tensor) -> None:
        """c_kv [B, n, 512], k_pe [B, n, 64] (host or device)."""
        n = c_kv.shape[1]
        t = self._filled[layer]
        if t + n > self.max_seq:
            raise ValueError("append beyond max_seq")
        (h0, h1, hs), (g0, g1, gsrc) = boundary_split(t, n, self.gs)
        if h1 > h0:
            self.host_c[layer][:, h0:h1].copy_(c_kv[:, hs:hs + h1 - h0])
            self.host_pe[layer][:, h0:h1].copy_(k_pe[:, hs:hs + h1 - h0])
        if g1 > g0:
            dev = self.gpu.device
            c = c_kv[:, gsrc:gsrc + g1 - g0].to(dev).contiguous()
            p = k_pe[:, gsrc:gsrc + g1 - g0].to(dev).contiguous()
            self.gpu.append(layer, c, p)
        self._filled[layer] = t + n

    def get(self, layer: int):
        """((host c, host pe) views of the filled host segment, GPU partition)."""
        t = self._filled[layer]
        n_host = min(t, self.gs)
        return (self.host_c[layer][:, :n_host], self.host_pe[layer][:, :n_host]), self.gpu

    def seq_len(self, layer: int) -> int:
        return self._filled[layer]


class PartitionedKVCache:
    """Token-range-partitioned GQA KV cache: host rows [B*Hkv, S_host, D] for
    the leading tokens of each sequence (pinned), GPU partition for the rest.

    Host lengths may differ per sequence (variable-length batches), so the
    host segment keeps its own per-sequence length.
    """

    def __init__(self, num_layers, batch, num_kv_heads, head_dim, max_host, max_gpu,
                 page_size=64, device="cuda"):
        pin = torch.cuda.is_available()
        self.batch, self.num_kv_heads, self.head_dim = batch, num_kv_heads, head_dim
        self.host_k = [torch.empty((batch * num_kv_heads, max_host, head_dim),
                                   dtype=torch.bfloat16, pin_memory=pin)
                       for _ in range(num_layers)]
        self.host_v = [torch.empty_like(self.host_k[0], pin_memory=pin)
                       for _ in range(num_layers)]
        self.host_len = np.zeros((num_layers, batch), np.int64)
        self.gpu = GqaGpuPartition(num_layers, batch, num_kv_heads, head_dim,
                                   max(max_gpu, 1), page_size, device=device)

    def load_host(self, layer: int, b: int, k: torch.Tensor, v: torch.Tensor) -> None:
        """Set sequence b's host segment to k, v [Hkv, n, D]."""
        n = k.shape[1]
        rows = slice(b * self.num_kv_heads, (b + 1) * self.num_kv_heads)
        self.host_k[layer][rows, :n].copy_(k)
        self.host_v[layer][rows, :n].copy_(v)
        self.host_len[layer, b] = n

    def host_rows(self, layer: int, b: int):
        """(k, v) views [Hkv, n_host, D] of sequence b's host segment."""
        n = int(self.host_len[layer, b])
        rows = slice(b * self.num_kv_heads, (b + 1) * self.num_kv_heads)
        return self.host_k[layer][rows, :n], self.host_v[layer][rows, :n]
