"""Partitioned decode attention: GPU partial over HBM pages, host partial on
the CPU at the same time, LSE merge on the GPU.

partitioned_gqa_decode mirrors the token-split flow of run_kvlen_resident
(roofline/bench_resident_kv.py:314-352) and
_compute_pipelined_attention (system/mixoffload.py:1201-1484);
partitioned_mla_decode mirrors the decode branch of _mla_compressed_forward
(system/deepseek.py:323-403).  The host partial is either
  "native"  this package's AVX-512 BF16 kernels (scope_amd.host): q is copied
            to pinned memory ahead of the GPU launch, the host partial runs in
            the calling thread with the GIL released while the GPU partial
            executes, and its (out, lse) is merged as is; or
  a callable with the contract of the reference CPU kernels
            (kernel/cpu_attn.cpp:1024-1054), which stay usable as they are:
            fused_cpu_attn(q, k, v, scale) / fused_cpu_attn_mla_compressed(
            q_proj, q_pe, c_kv, k_pe, scale) on CPU tensors, run on a worker
            thread.
"""
from __future__ import annotations

import threading

import numpy as np
import torch

from . import host, ops
from .cache import PartitionedKVCache, PartitionedLatentCache

NATIVE = "native"

# Host-partial output conventions -> merge format.
CPU_FORMATS = {
    "fused_cpu_attn_bf16": ops.TRIPLE_NORM_BF16,     # normalised bf16 triple
    "fused_cpu_attn_fp32": ops.TRIPLE_NORM_F32,      # normalised fp32 triple
    "fused_cpu_attn_mla": ops.TRIPLE_UNNORM_F32,     # unnormalised fp32 triple
    "mla_compressed": ops.TRIPLE_UNNORM_F32,
}


class _CpuPartial(threading.Thread):
    def __init__(self, fn):
        super().__init__(daemon=True)
        self._fn = fn
        self.result = None
        self.error = None

    def run(self):
        try:
            self.result = self._fn()
        except BaseException as e:  # surfaced by join_result
            self.error = e

    def join_result(self):
        self.join()
        if self.error is not None:
            raise self.error
        return self.result


def _to_device_pinned(t: torch.Tensor, dev: torch.device) -> torch.Tensor:
    if t.is_cuda:
        return t
    if not t.is_pinned():
        t = t.pin_memory()
    return t.to(dev, non_blocking=True)


def _query_to_host(*qs):
    """Pinned host copies of the GPU queries, enqueued before the GPU partial so
    the host waits only for the copies; returns (*copies, event)."""
    out = []
    for t in qs:
        h = torch.empty(t.shape, dtype=t.dtype, pin_memory=True)
        h.copy_(t, non_blocking=True)
        out.append(h)
    ev = torch.cuda.Event()
    ev.record()
    return (*out, ev)


def _pinned_out(out_shape, lse_shape):
    return (torch.empty(out_shape, dtype=torch.float32, pin_memory=True),
            torch.empty(lse_shape, dtype=torch.float32, pin_memory=True))


def _gqa_gpu(gpu, layer, q, scale, k_new, v_new, n_workgroups):
    """The GPU side: a split step when the call appends (its combine then runs
    inside the merge), else the one-launch partial."""
    if k_new is not None:
        return gpu.step_split(layer, q, k_new, v_new, scale, n_workgroups)
    return gpu.attend(layer, q, scale, n_workgroups)


def _finish(gpu_part, b, fmt):
    """Merge the GPU side (a SplitStep or an (out, lse) partial) with the host
    partial b in format fmt (None: no host partial); bf16 [rows, Dv]."""
    if isinstance(gpu_part, ops.SplitStep):
        out, _ = ops.merge_split(gpu_part, b, fmt, want_lse=False)
        return out
    out_g, lse_g = gpu_part
    if b is None:
        b, fmt = (out_g, torch.full_like(lse_g, float("-inf"))), ops.PARTIAL_LSE_F32
    out, _ = ops.lse_merge(out_g, lse_g, b, fmt, want_lse=False)
    return out


def partitioned_gqa_decode(cache: PartitionedKVCache, layer: int, q: torch.Tensor,
                           scale: float, cpu_attn=None, cpu_format="fused_cpu_attn_bf16",
                           k_new=None, v_new=None, n_workgroups=0, host_threads=0):
    """One decode step of GQA attention over a host/GPU partitioned cache.

    q [B, Hq, D] bf16 on the GPU; k_new/v_new [B, Hkv, 1, D] (optional) are
    appended to the GPU partition in the same launch as its partial.  cpu_attn(q [Hkv, G, D], k [Hkv, S, D],
    v [Hkv, S, D], scale) -> (out, max, sum) is called once per sequence with
    host tokens (the reference kernels take one S per call,
    kernel/cpu_attn.cpp:590).  cpu_attn="native" runs scope_amd.host over the
    whole ragged batch in one call (host_threads, 0 = OpenMP default).
    Returns out [B, Hq, 1, D] bf16.
    """
    gpu = cache.gpu
    B, Hq, D = q.shape
    Hkv = cache.num_kv_heads
    G = Hq // Hkv
    need_cpu = cpu_attn is not None and bool((cache.host_len[layer] > 0).any())
    if need_cpu and cpu_attn == NATIVE:
        q_host, ev = _query_to_host(q)
        g = _gqa_gpu(gpu, layer, q, scale, k_new, v_new, n_workgroups)
        ev.synchronize()
        lens = torch.from_numpy(cache.host_len[layer].astype(np.int32))
        part = host.gqa_partial_dense(q_host, cache.host_k[layer], cache.host_v[layer], lens,
                                      scale, host_threads, *_pinned_out((B, Hq, D), (B, Hq)))
        dev = q.device
        b = tuple(x.to(dev, non_blocking=True) for x in part)
        return _finish(g, b, ops.PARTIAL_LSE_F32).view(B, Hq, 1, D)
    worker = None
    if need_cpu:
        q_host = q.view(B * Hkv, G, D).cpu()

        def host_partial():
            fmt = CPU_FORMATS[cpu_format]
            odt = torch.bfloat16 if fmt == ops.TRIPLE_NORM_BF16 else torch.float32
            o = torch.zeros((B * Hkv, G, D), dtype=odt)
            m = torch.full((B * Hkv, G, 1), float("-inf"), dtype=odt)
            s = torch.zeros((B * Hkv, G, 1), dtype=odt)
            for b in range(B):
                k, v = cache.host_rows(layer, b)
                if k.shape[1] == 0:
                    continue
                rows = slice(b * Hkv, (b + 1) * Hkv)
                ob, mb, sb = cpu_attn(q_host[rows].contiguous(), k, v, scale)
                o[rows], m[rows], s[rows] = ob.to(odt), mb.reshape(Hkv, G, 1).to(odt), \
                    sb.reshape(Hkv, G, 1).to(odt)
            return o, m, s

        worker = _CpuPartial(host_partial)
        worker.start()
    g = _gqa_gpu(gpu, layer, q, scale, k_new, v_new, n_workgroups)
    if worker is None:
        return _finish(g, None, None).view(B, Hq, 1, D)
    o, m, s = worker.join_result()
    dev = q.device
    triple = tuple(_to_device_pinned(x, dev) for x in (o, m, s))
    return _finish(g, triple, CPU_FORMATS[cpu_format]).view(B, Hq, 1, D)


def partitioned_mla_decode(cache: PartitionedLatentCache, layer: int,
                           q_nope: torch.Tensor, q_pe: torch.Tensor, scale: float,
                           cpu_attn_mla_compressed=None, c_new=None, pe_new=None,
                           n_workgroups=0, host_threads=0):
    """One decode step of absorbed-MLA attention over a partitioned latent cache.

    q_nope [B*H, 512] (W_UK-absorbed) and q_pe [B*H, 64] bf16 on the GPU;
    c_new [B, 1, 512] / pe_new [B, 1, 64] are appended first (split at the
    boundary like system/deepseek.py:171-192).  The host partial runs
    cpu_attn_mla_compressed(q_proj, q_pe, c, pe, scale) -> fp32 (o, max, sum)
    over the host segment on a worker thread while the GPU partial runs
    (cpu_attn_mla_compressed="native": scope_amd.host in the calling thread).
    Returns the merged latent output [B*H, 512] bf16 (before W_UV).
    """
    if c_new is not None:
        cache.append(layer, c_new, pe_new)
    (hc, hpe), gpu = cache.get(layer)
    if cpu_attn_mla_compressed == NATIVE and hc.shape[1] > 0:
        B = hc.shape[0]
        qn_host, qp_host, ev = _query_to_host(q_nope, q_pe)
        out_g, lse_g = gpu.attend(layer, q_nope, q_pe, scale, n_workgroups)
        ev.synchronize()
        lens = torch.full((B,), hc.shape[1], dtype=torch.int32)
        rows = q_nope.shape[0]
        part = host.mla_partial_dense(qn_host, qp_host, cache.host_c[layer],
                                      cache.host_pe[layer], lens, scale, host_threads,
                                      *_pinned_out((rows, ops.MLA_C), (rows,)))
        dev = q_nope.device
        b = tuple(x.to(dev, non_blocking=True) for x in part)
        out, _ = ops.lse_merge(out_g, lse_g, b, ops.PARTIAL_LSE_F32, want_lse=False)
        return out
    worker = None
    if cpu_attn_mla_compressed is not None and hc.shape[1] > 0:
        qn_host, qp_host = q_nope.cpu(), q_pe.cpu()
        worker = _CpuPartial(lambda: cpu_attn_mla_compressed(
            qn_host, qp_host, hc.contiguous(), hpe.contiguous(), scale))
        worker.start()
    out_g, lse_g = gpu.attend(layer, q_nope, q_pe, scale, n_workgroups)
    if worker is None:
        empty = torch.full_like(lse_g, float("-inf"))
        out, _ = ops.lse_merge(out_g, lse_g, (out_g, empty), ops.PARTIAL_LSE_F32,
                               want_lse=False)
        return out
    o, m, s = worker.join_result()
    dev = q_nope.device
    triple = tuple(_to_device_pinned(x.float().contiguous(), dev) for x in (o, m, s))
    out, _ = ops.lse_merge(out_g, lse_g, triple, ops.TRIPLE_UNNORM_F32, want_lse=False)
    return out
