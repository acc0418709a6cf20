"""Decode-step benchmark of the GPU KV partition on one MI355X.

Headline workload (one "step" = one decode step of one attention layer):
partitioned GQA decode at the Mixtral-8x7B layer shape: batch 16, 32 query
heads, 8 KV heads, head_dim 128, bf16 N(0,1), per-sequence KV lengths uniform
in [1024, 32768], the trailing floor(r*L) tokens of each sequence in 64-token
HBM pages (r = 0.5 by default).  A step appends one token per sequence to the
GPU partition and runs the load-balanced split-KV GQA partial over the
partition (one launch: ws_gqa_append_decode_split), then combines the split
pieces and LSE-merges them with the host partial (the bf16 (out, max, sum)
triple of the CPU kernel, already resident in HBM) into the final bf16 output
(one launch: ws_merge_split).

Reported on one JSON line (stdout):
  value      algorithmic HBM GB/s of the whole step (bytes below / step time)
  ms_per_step, us_per_layer
  roofline   the fused append + GQA partial kernel: algorithmic bytes per
             launch / its mean duration from timing-only HIP events
             (hipEventDisableSystemFence) around every launch of the timed
             region, against the 8 TB/s HBM peak; traffic from the committed rocprofv3
             FETCH_SIZE / WRITE_SIZE summary when one exists for this workload
  cpu_baseline  the clean-room AVX-512 BF16 host kernel (libwshost.so
             wh_gqa_partial, the reference CPU kernel's contract) over the same
             GPU-share tokens, one call per sequence, on pinned host cores
  by_share, kv_len_sweep, mla, mla_kv_len_sweep, single_partition
             the other shares, the Qwen3 length sweep (batch 4, r = 1), the
             absorbed-MLA layer (DeepSeek-V2-Lite, batch 8, L 16384, r 0.5),
             the MLA length sweep (batch 8, r = 1, 8k..128k tokens) and the
             batch-1 Qwen3 layer with all 4096 tokens on the GPU

Algorithmic bytes of a step (each byte once): KV of every GPU token read,
Q read, GPU partial (out fp32 + lse) written, host partial read, final bf16
output written, appended token written, page-table entries read.

Run: python bench.py [--gpus 1] [--steps K] [--warmup W] [--share r]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import re
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
METRIC = ("GPU-partition decode attn µs/layer + HBM GB/s (% peak) vs KV len; "
          "CPU ref alongside")
PAGE = 64


def log(msg):
    print(msg, file=sys.stderr, flush=True)


# ---------------------------------------------------------------------------
# paged pools


CONTIGUOUS_PAGES = False  # --contiguous-pages: pages in order (locality check)


def _page_table(gpu_tokens, capacity_extra, rng):
    """Fragmented page assignment: every sequence gets the pages for its GPU
    tokens plus room for the appends, page ids drawn from a random permutation
    (in order with --contiguous-pages)."""
    need = [-(-(int(g) + capacity_extra) // PAGE) for g in gpu_tokens]
    max_pages = max(1, max(need))
    num_pages = sum(need)
    perm = rng.permutation(num_pages).astype(np.int32)
    if CONTIGUOUS_PAGES:
        perm = np.arange(num_pages, dtype=np.int32)
    table = np.full((len(need), max_pages), -1, np.int32)
    k = 0
    for b, n in enumerate(need):
        table[b, :n] = perm[k:k + n]
        k += n
    return table, num_pages


def _randn_bf16(shape, gen, sigma, dev):
    import torch

    t = torch.empty(shape, dtype=torch.bfloat16, device=dev)
    # fill in slabs to bound the fp32 temporary
    flat = t.view(-1)
    step = 1 << 27
    for i in range(0, flat.numel(), step):
        n = min(step, flat.numel() - i)
        flat[i:i + n] = (torch.randn(n, generator=gen, device=dev) * sigma).to(torch.bfloat16)
    return t


_HIP_EVENT_DISABLE_SYSTEM_FENCE = 0x20000000  # hip_runtime_api.h
_hip_rt = None


def _hip_runtime():
    """The HIP runtime torch itself loaded (its streams are only valid there),
    found by path in this process's mappings."""
    global _hip_rt
    if _hip_rt is None:
        import torch

        torch.cuda.init()
        with open("/proc/self/maps") as f:
            paths = {ln.split()[-1] for ln in f if "libamdhip64.so" in ln}
        if not paths:
            raise RuntimeError("libamdhip64.so is not loaded")
        L = ctypes.CDLL(sorted(paths)[0])
        vp = ctypes.c_void_p
        L.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(vp), ctypes.c_uint]
        L.hipEventRecord.argtypes = [vp, vp]
        L.hipEventSynchronize.argtypes = [vp]
        L.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), vp, vp]
        L.hipEventDestroy.argtypes = [vp]
        _hip_rt = L
    return _hip_rt


class HipTimingEvent:
    """A timing-only HIP event (hipEventDisableSystemFence) recorded on the
    current torch stream.  A default event's record also performs a
    system-scope release (an L2 writeback so the host could read the results),
    which lands in the launch it brackets: 2-3 us of a 60 us kernel that
    writes 8 MB.  Device work ordered after the kernel on the same stream needs
    no such fence, so the timing events skip it."""

    def __init__(self):
        self._rt = _hip_runtime()
        self.ev = ctypes.c_void_p()
        rc = self._rt.hipEventCreateWithFlags(ctypes.byref(self.ev),
                                              _HIP_EVENT_DISABLE_SYSTEM_FENCE)
        if rc:
            raise RuntimeError(f"hipEventCreateWithFlags failed ({rc})")

    def record(self):
        import torch

        rc = self._rt.hipEventRecord(self.ev,
                                     ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        if rc:
            raise RuntimeError(f"hipEventRecord failed ({rc})")

    def elapsed_time(self, end):
        """Milliseconds from this event to `end` (waits for `end`)."""
        ms = ctypes.c_float()
        rc = (self._rt.hipEventSynchronize(end.ev)
              or self._rt.hipEventElapsedTime(ctypes.byref(ms), self.ev, end.ev))
        if rc:
            raise RuntimeError(f"hipEventElapsedTime failed ({rc})")
        return ms.value

    def __del__(self):
        if self.ev:
            self._rt.hipEventDestroy(self.ev)


class _Timer:
    """Per-launch timing events on the stream the kernels are launched on."""

    def __init__(self, n):
        self.a = [HipTimingEvent() for _ in range(n)]
        self.b = [HipTimingEvent() for _ in range(n)]

    def mean_us(self, n):
        return 1e3 * sum(self.a[i].elapsed_time(self.b[i]) for i in range(n)) / n


# ---------------------------------------------------------------------------
# GQA step


def gqa_step_bench(*, B, Hkv, G, lens, share, steps, warmup, seed, dev, with_host,
                   label, wg=0):
    """Times `steps` decode steps (fused append + GQA partial, then the merge
    with the host partial, or with no host partial when with_host is False)
    and returns a dict of results.  lens: total KV lengths; the GPU holds
    floor(share*L) of each."""
    import torch

    from scope_amd import ops

    D = 128
    Hq = Hkv * G
    L = ops.lib()
    rng = np.random.default_rng(seed)
    gpu_tokens = np.array([int(math.floor(share * int(x))) for x in lens], np.int64)
    extra = warmup + 2 * steps + 1
    table, num_pages = _page_table(gpu_tokens, extra, rng)
    gen = torch.Generator(device=dev).manual_seed(seed)
    k_pages = _randn_bf16((num_pages, Hkv, PAGE, D), gen, 1.0, dev)
    v_pages = _randn_bf16((num_pages, Hkv, PAGE, D), gen, 1.0, dev)
    page_table = torch.from_numpy(table).to(dev)
    # two length arrays, swapped every step (the fused step reads one, writes the other)
    lens2 = torch.zeros((2, B), dtype=torch.int32, device=dev)
    lens2[0] = torch.from_numpy(gpu_tokens.astype(np.int32)).to(dev)
    q = _randn_bf16((B, Hq, D), gen, 1.0, dev)
    k_new = _randn_bf16((B, Hkv, 1, D), gen, 1.0, dev)
    v_new = _randn_bf16((B, Hkv, 1, D), gen, 1.0, dev)
    rows = B * Hq
    # host partial: bf16 (normalised out, max, sum) as fused_cpu_attn returns it
    h_out = _randn_bf16((rows, D), gen, 0.3, dev)
    h_max = (torch.randn(rows, generator=gen, device=dev) + 4).to(torch.bfloat16)
    h_sum = (torch.rand(rows, generator=gen, device=dev) * 50 + 1).to(torch.bfloat16)
    out_g = torch.empty((rows, D), dtype=torch.float32, device=dev)
    lse_g = torch.empty((rows,), dtype=torch.float32, device=dev)
    out = torch.empty((rows, D), dtype=torch.bfloat16, device=dev)

    max_len0 = int(gpu_tokens.max())
    max_len_end = max_len0 + extra
    nwg, wsb = ops.decode_plan(0, B * Hkv, G, max_len_end, wg)
    ws = torch.zeros(max(wsb, 256), dtype=torch.uint8, device=dev)
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    max_pages = table.shape[1]
    scale = ctypes.c_float(D ** -0.5)
    len_ptrs = (p(lens2[0]), p(lens2[1]))
    a_head = (p(q), p(k_new), p(v_new), p(k_pages), p(v_pages), p(page_table))
    a_mid = (B, Hq, Hkv, D, PAGE, max_pages, num_pages)
    a_tail = (nwg, scale, p(out_g), p(lse_g), p(ws), ctypes.c_size_t(wsb), stream)
    cap = PAGE * max_pages
    # the merge reads the lengths the step wrote (its len_out)
    a_merge = [(len_ptrs[k], B, Hkv, G, D, cap, nwg, p(out_g), p(lse_g), p(ws),
                ctypes.c_size_t(wsb), p(h_out), p(h_max), p(h_sum), ops.TRIPLE_NORM_BF16,
                p(out), None, None, stream) for k in (0, 1)]
    if not with_host:  # r = 1: nothing on the host; the merge only combines the pieces
        a_merge = [(len_ptrs[k], B, Hkv, G, D, cap, nwg, p(out_g), p(lse_g), p(ws),
                    ctypes.c_size_t(wsb), None, None, None, 0, p(out), None, None, stream)
                   for k in (0, 1)]
    f_step, f_merge = L.ws_gqa_append_decode_split, L.ws_merge_split

    for i in range(warmup):
        rc = f_step(*a_head, len_ptrs[i % 2], len_ptrs[(i + 1) % 2], *a_mid,
                    max_len0 + i + 1, *a_tail)
        rc |= f_merge(*a_merge[(i + 1) % 2])
        if rc:
            raise RuntimeError(f"{label}: {L.ws_last_error().decode()}")
    # Pass 1, the step time: `steps` steps queued back to back with nothing
    # between them but the two launches (events only around the whole pass).
    # Pass 2, the partial kernel's time: the same steps with a timing-only
    # event pair around every step launch (the events' own cost stays out
    # of pass 1).
    t_ev0 = HipTimingEvent()
    t_ev1 = HipTimingEvent()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    t_ev0.record()
    for i in range(steps):
        a_i = warmup + i
        rc = f_step(*a_head, len_ptrs[a_i % 2], len_ptrs[(a_i + 1) % 2], *a_mid,
                    max_len0 + a_i + 1, *a_tail)
        rc |= f_merge(*a_merge[(a_i + 1) % 2])
        if rc:
            raise RuntimeError(f"{label}: {L.ws_last_error().decode()}")
    t_ev1.record()
    t_host = time.perf_counter() - t0
    torch.cuda.synchronize()
    t_wall = time.perf_counter() - t0
    step_us = 1e3 * t_ev0.elapsed_time(t_ev1) / steps
    timer = _Timer(steps)
    for i in range(steps):
        a_i = warmup + steps + i
        timer.a[i].record()
        rc = f_step(*a_head, len_ptrs[a_i % 2], len_ptrs[(a_i + 1) % 2], *a_mid,
                    max_len0 + a_i + 1, *a_tail)
        timer.b[i].record()
        rc |= f_merge(*a_merge[(a_i + 1) % 2])
        if rc:
            raise RuntimeError(f"{label}: {L.ws_last_error().decode()}")
    torch.cuda.synchronize()
    final_len = lens2[(warmup + 2 * steps) % 2].cpu().numpy()
    if not np.array_equal(final_len, gpu_tokens + warmup + 2 * steps):
        raise RuntimeError(f"{label}: lengths did not advance by one per step")
    part_us = timer.mean_us(steps)
    # tokens attended in pass 1: g + warmup + 1 .. g + warmup + steps (pass 2
    # attends `steps` more per sequence; its partial bytes are the pass-1
    # bytes plus B * steps tokens, which the step figures below leave out)
    mean_tokens = float(gpu_tokens.sum()) + B * (warmup + (steps + 1) / 2.0)
    kv_tok = Hkv * 2 * D * 2
    pages_read = float(sum(-(-(int(g) + warmup + steps // 2) // PAGE) for g in gpu_tokens))
    kernel_bytes = (mean_tokens * kv_tok + rows * D * 2 + rows * (D + 1) * 4
                    + pages_read * 4 + B * kv_tok)
    # the merge: the host triple read (r < 1), the bf16 output written
    step_bytes = kernel_bytes + (rows * (D * 2 + 4) if with_host else 0) + rows * D * 2
    # the partial kernel's bytes in pass 2 (B * steps tokens more per launch)
    part_bytes = kernel_bytes + B * steps * kv_tok
    return {
        "label": label,
        "batch": B, "q_heads": Hq, "kv_heads": Hkv, "head_dim": D,
        "share": share,
        "gpu_tokens": int(gpu_tokens.sum()),
        "max_gpu_tokens": max_len0,
        "workgroups": nwg,
        "us_per_layer": round(step_us, 2),
        "step_gbs": round(step_bytes / step_us / 1e3, 1),
        "partial_us": round(part_us, 2),
        "partial_gbs": round(part_bytes / part_us / 1e3, 1),
        "partial_frac": round(part_bytes / part_us / 1e3 / HBM_PEAK_GBS, 4),
        "step_bytes": int(step_bytes),
        "partial_bytes": int(part_bytes),
        "host_loop_us_per_step": round(1e6 * t_host / steps, 2),
        "wall_us_per_step": round(1e6 * t_wall / steps, 2),
        "_data": (k_pages, v_pages, table, gpu_tokens, q),
    }


# ---------------------------------------------------------------------------
# MLA step


def mla_step_bench(*, B, H, lens, share, steps, warmup, seed, dev, label, wg=0):
    """Times `steps` absorbed-MLA decode steps (fused latent append + partial,
    then the merge with the host partial's fp32 (o, max, sum) triple)."""
    import torch

    from scope_amd import ops

    L = ops.lib()
    rng = np.random.default_rng(seed)
    gpu_tokens = np.array([int(math.floor(share * int(x))) for x in lens], np.int64)
    extra = warmup + 2 * steps + 1
    table, num_pages = _page_table(gpu_tokens, extra, rng)
    gen = torch.Generator(device=dev).manual_seed(seed)
    latent = _randn_bf16((num_pages, PAGE, 576), gen, 0.5, dev)
    page_table = torch.from_numpy(table).to(dev)
    lens2 = torch.zeros((2, B), dtype=torch.int32, device=dev)
    lens2[0] = torch.from_numpy(gpu_tokens.astype(np.int32)).to(dev)
    rows = B * H
    qn = _randn_bf16((rows, 512), gen, 0.5, dev)
    qp = _randn_bf16((rows, 64), gen, 0.5, dev)
    kv_new = _randn_bf16((B, 1, 576), gen, 0.5, dev)
    c_new, pe_new = kv_new[..., :512], kv_new[..., 512:]
    h_out = torch.randn((rows, 512), generator=gen, device=dev) * 5
    h_max = torch.randn(rows, generator=gen, device=dev) + 4
    h_sum = torch.rand(rows, generator=gen, device=dev) * 50 + 1
    out_g = torch.empty((rows, 512), dtype=torch.float32, device=dev)
    lse_g = torch.empty((rows,), dtype=torch.float32, device=dev)
    out = torch.empty((rows, 512), dtype=torch.bfloat16, device=dev)
    max_len0 = int(gpu_tokens.max())
    nwg, wsb = ops.decode_plan(1, B, H, max_len0 + extra, wg)
    ws = torch.zeros(max(wsb, 256), dtype=torch.uint8, device=dev)
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    max_pages = table.shape[1]
    len_ptrs = (p(lens2[0]), p(lens2[1]))
    a_head = (p(qn), p(qp), p(c_new), ctypes.c_int64(576), p(pe_new), ctypes.c_int64(576),
              p(latent), p(page_table))
    a_mid = (B, H, PAGE, max_pages, num_pages)
    a_tail = (nwg, ctypes.c_float(192 ** -0.5), p(out_g), p(lse_g), p(ws),
              ctypes.c_size_t(wsb), stream)
    cap = PAGE * max_pages
    a_merge = [(len_ptrs[k], B, 1, H, 512, cap, nwg, p(out_g), p(lse_g), p(ws),
                ctypes.c_size_t(wsb), p(h_out), p(h_max), p(h_sum), ops.TRIPLE_UNNORM_F32,
                p(out), None, None, stream) for k in (0, 1)]
    f_step, f_merge = L.ws_mla_append_decode_split, L.ws_merge_split
    for i in range(warmup):
        rc = f_step(*a_head, len_ptrs[i % 2], len_ptrs[(i + 1) % 2], *a_mid,
                    max_len0 + i + 1, *a_tail) | f_merge(*a_merge[(i + 1) % 2])
        if rc:
            raise RuntimeError(f"{label}: {L.ws_last_error().decode()}")
    # pass 1: step time with no event between launches; pass 2: per-launch
    # timing events around the step kernel (as gqa_step_bench)
    e0 = HipTimingEvent()
    e1 = HipTimingEvent()
    torch.cuda.synchronize()
    e0.record()
    for i in range(steps):
        a_i = warmup + i
        rc = f_step(*a_head, len_ptrs[a_i % 2], len_ptrs[(a_i + 1) % 2], *a_mid,
                    max_len0 + a_i + 1, *a_tail)
        rc |= f_merge(*a_merge[(a_i + 1) % 2])
        if rc:
            raise RuntimeError(f"{label}: {L.ws_last_error().decode()}")
    e1.record()
    torch.cuda.synchronize()
    step_us = 1e3 * e0.elapsed_time(e1) / steps
    timer = _Timer(steps)
    for i in range(steps):
        a_i = warmup + steps + i
        timer.a[i].record()
        rc = f_step(*a_head, len_ptrs[a_i % 2], len_ptrs[(a_i + 1) % 2], *a_mid,
                    max_len0 + a_i + 1, *a_tail)
        timer.b[i].record()
        rc |= f_merge(*a_merge[(a_i + 1) % 2])
        if rc:
            raise RuntimeError(f"{label}: {L.ws_last_error().decode()}")
    torch.cuda.synchronize()
    part_us = timer.mean_us(steps)
    mean_tokens = float(gpu_tokens.sum()) + B * (warmup + (steps + 1) / 2.0)
    pages_read = float(sum(-(-(int(g) + warmup + steps // 2) // PAGE) for g in gpu_tokens))
    kernel_bytes = (mean_tokens * 1152 + rows * 576 * 2 + rows * 513 * 4 + pages_read * 4
                    + B * 1152)
    step_bytes = kernel_bytes + rows * 514 * 4 + rows * 512 * 2
    # pass 2 attends `steps` more tokens per sequence than pass 1
    kernel_bytes += B * steps * 1152
    flops = (mean_tokens + B * steps) * H * (2 * 576 + 2 * 512)
    return {
        "label": label, "batch": B, "heads": H, "share": share,
        "gpu_tokens": int(gpu_tokens.sum()), "workgroups": nwg,
        "us_per_layer": round(step_us, 2),
        "step_gbs": round(step_bytes / step_us / 1e3, 1),
        "partial_us": round(part_us, 2),
        "partial_gbs": round(kernel_bytes / part_us / 1e3, 1),
        "partial_frac": round(kernel_bytes / part_us / 1e3 / HBM_PEAK_GBS, 4),
        "partial_tflops": round(flops / part_us / 1e6, 2),
        # algorithmic flops / event time against the 2.5 PFLOP/s dense bf16
        # peak; the counter-based figures are in "counters" when committed
        "flops_frac_bf16_dense": round(flops / part_us / 1e6 / 2500.0, 4),
        "partial_bytes": int(kernel_bytes),
        "partial_flops": int(flops),
        "step_bytes": int(step_bytes),
    }


# ---------------------------------------------------------------------------
# Host partial (libwshost.so) and the multi-layer MLA decode with both partitions


def _host_pages(tokens, rng):
    """Exact page assignment of a host segment (no room for appends: decode
    appends go to the GPU partition), page ids from a random permutation."""
    need = [-(-int(t) // PAGE) for t in tokens]
    max_pages = max(1, max(need))
    num_pages = max(1, sum(need))
    perm = rng.permutation(num_pages).astype(np.int32)
    table = np.zeros((len(need), max_pages), np.int32)
    k = 0
    for b, n in enumerate(need):
        table[b, :n] = perm[k:k + n]
        k += n
    return table, num_pages


def _host_threads():
    n = len(os.sched_getaffinity(0))
    omp = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    return min(n, omp) if omp > 0 else n


def host_gqa_bench(*, Hkv, G, host_tokens, reps, seed, dev, threads, label):
    """Native host partial (wh_gqa_partial) over a paged host segment holding
    host_tokens[b] tokens per sequence; median of `reps` calls."""
    import torch

    from scope_amd import host

    D = 128
    rng = np.random.default_rng(seed)
    table, num_pages = _host_pages(host_tokens, rng)
    gen = torch.Generator(device=dev).manual_seed(seed)
    kp = _randn_bf16((num_pages, Hkv, PAGE, D), gen, 1.0, dev).cpu()
    vp = _randn_bf16((num_pages, Hkv, PAGE, D), gen, 1.0, dev).cpu()
    B = len(host_tokens)
    q = _randn_bf16((B, Hkv * G, D), gen, 1.0, dev).cpu()
    lens = torch.from_numpy(np.asarray(host_tokens, np.int32))
    tab = torch.from_numpy(table)
    out = torch.empty((B, Hkv * G, D), dtype=torch.float32)
    lse = torch.empty((B, Hkv * G), dtype=torch.float32)
    host.gqa_partial(q, kp, vp, tab, lens, D ** -0.5, threads, out, lse)
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        host.gqa_partial(q, kp, vp, tab, lens, D ** -0.5, threads, out, lse)
        times.append(time.perf_counter() - t0)
    t = float(np.median(times))
    nbytes = float(np.sum(host_tokens)) * Hkv * 2 * D * 2
    return {"label": label, "threads": threads, "host_tokens": int(np.sum(host_tokens)),
            "us": round(t * 1e6, 1), "gbs": round(nbytes / t / 1e9, 2)}


def host_mla_bench(*, host_tokens, reps, seed, dev, threads, label):
    """Native host partial (wh_mla_partial) over a paged host latent pool."""
    import torch

    from scope_amd import host

    rng = np.random.default_rng(seed)
    table, num_pages = _host_pages(host_tokens, rng)
    gen = torch.Generator(device=dev).manual_seed(seed)
    pool = _randn_bf16((num_pages, PAGE, 576), gen, 0.5, dev).cpu()
    B = len(host_tokens)
    qn = _randn_bf16((B * 16, 512), gen, 0.5, dev).cpu()
    qp = _randn_bf16((B * 16, 64), gen, 0.5, dev).cpu()
    lens = torch.from_numpy(np.asarray(host_tokens, np.int32))
    tab = torch.from_numpy(table)
    out = torch.empty((B * 16, 512), dtype=torch.float32)
    lse = torch.empty((B * 16,), dtype=torch.float32)
    host.mla_partial(qn, qp, pool, tab, lens, 192 ** -0.5, threads, out, lse)
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        host.mla_partial(qn, qp, pool, tab, lens, 192 ** -0.5, threads, out, lse)
        times.append(time.perf_counter() - t0)
    t = float(np.median(times))
    tok = float(np.sum(host_tokens))
    return {"label": label, "threads": threads, "host_tokens": int(tok),
            "us": round(t * 1e6, 1), "gbs": round(tok * 1152 / t / 1e9, 2),
            "tflops": round(tok * 16 * (2 * 576 + 2 * 512) / t / 1e12, 3)}


def migration_bench(*, B, layers, lens, seed, dev, label):
    """Boundary movement of a two-sided paged MLA cache (scope_amd.paged):
    share 0.5 -> 0.75 moves host pages to HBM, 0.75 -> 0.5 moves them back,
    every layer; wall time of each set_share, in GB/s of pages moved."""
    import torch

    from scope_amd.paged import PagedMlaCache

    lens = np.asarray(lens, np.int64)
    pages = int(sum(-(-int(L) // PAGE) for L in lens)) + B
    cache = PagedMlaCache(layers, B, max_tokens=int(lens.max()) + PAGE, page_size=PAGE,
                          host_pages=pages, gpu_pages=pages, device=dev)
    gen = torch.Generator(device=dev).manual_seed(seed)
    src = _randn_bf16((int(lens.max()), 576), gen, 0.5, dev).cpu()
    c, pe = src[:, :512].contiguous(), src[:, 512:].contiguous()
    for layer in range(layers):
        for b, L in enumerate(lens):
            L = int(L)
            h = L - int(math.floor(0.5 * L))
            cache.load(layer, b, c[:L], pe[:L], (h // PAGE) * PAGE)
    torch.cuda.synchronize()
    page_bytes = PAGE * 576 * 2 * layers
    res = {"label": label, "batch": B, "layers": layers, "page_size": PAGE}
    for name, r in (("host_to_hbm", 0.75), ("hbm_to_host", 0.5), ("host_to_hbm_2", 0.75),
                    ("hbm_to_host_2", 0.5)):
        before = int(cache.host.held.sum())
        t0 = time.perf_counter()
        cache.set_share(r)
        torch.cuda.synchronize()
        dt = time.perf_counter() - t0
        moved = abs(before - int(cache.host.held.sum()))
        res[name] = {"pages": moved, "bytes": moved * page_bytes, "ms": round(dt * 1e3, 2),
                     "gbs": round(moved * page_bytes / dt / 1e9, 2)}
    return res


def epilogue_bench(*, B, L, steps, seed, dev, label):
    """The MLA step's finish with and without the fused W_UV epilogue: (a)
    ws_merge_split to the bf16 latent, then the reference's per-head bmm with
    W_UV^T (system/deepseek.py:405) through torch; (b) ws_mla_merge_split_uv.
    Both after the same split step; event time per finish."""
    import torch

    from scope_amd import ops

    H, Dout = 16, 128
    rng = np.random.default_rng(seed)
    lens = np.full(B, L, np.int64)
    table, num_pages = _page_table(lens, 2, rng)
    gen = torch.Generator(device=dev).manual_seed(seed)
    latent = _randn_bf16((num_pages, PAGE, 576), gen, 0.5, dev)
    pt = torch.from_numpy(table).to(dev)
    lens2 = torch.zeros((2, B), dtype=torch.int32, device=dev)
    lens2[0] = torch.from_numpy(lens.astype(np.int32)).to(dev)
    qn = _randn_bf16((B * H, 512), gen, 0.5, dev)
    qp = _randn_bf16((B * H, 64), gen, 0.5, dev)
    kv = _randn_bf16((B, 1, 576), gen, 0.5, dev)
    w_uv = _randn_bf16((H, Dout, 512), gen, 0.05, dev)
    w_uv_t = w_uv.transpose(1, 2).contiguous()  # [H, 512, Dout]
    step = ops.mla_append_decode_split(qn, qp, kv[..., :512], kv[..., 512:], latent, pt,
                                       lens2[0], lens2[1], 192 ** -0.5, L + 1)

    def unfused():
        lat, _ = ops.merge_split(step, None, want_lse=False)
        o_v = torch.bmm(lat.view(B, H, 512).transpose(0, 1).contiguous(), w_uv_t)
        return o_v.transpose(0, 1).reshape(B, H * Dout)  # the layout o_proj takes

    def fused():
        return ops.merge_split_uv(step, w_uv)[0]

    res = {"label": label, "batch": B, "tokens": L}
    for name, fn in (("merge_then_bmm_us", unfused), ("fused_uv_us", fused)):
        for _ in range(5):
            fn()
        e0 = HipTimingEvent()
        e1 = HipTimingEvent()
        torch.cuda.synchronize()
        e0.record()
        for _ in range(steps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        res[name] = round(1e3 * e0.elapsed_time(e1) / steps, 2)
    return res


_HOST_BW = {}


def host_read_gbs(threads, nbytes=1 << 30, reps=3, probes=5):
    """Host DRAM streaming read bandwidth (wh_host_read_gbs: `threads` OpenMP
    threads summing a buffer they first touched with 512-bit loads): the
    median of `probes` probes, each the best of `reps` passes, measured once
    per thread count in a run so that every figure of the run is compared
    with the same number (single probes on these virtual hosts have ranged
    over 2x within one run)."""
    from scope_amd import host

    if threads not in _HOST_BW:
        vals = sorted(round(host.host_read_gbs(nbytes, threads, reps), 1)
                      for _ in range(probes))
        _HOST_BW[threads] = (float(np.median(vals)), vals)
    return _HOST_BW[threads][0]


def host_read_probes(threads):
    """The probes behind host_read_gbs(threads) (after it has run)."""
    return _HOST_BW.get(threads, (None, []))[1]


def share_model(rows, host_bw_gbs=None):
    """Calibrates the share scheduler's roofline model from a share sweep of
    the multi-layer MLA run and compares its per-layer predictions with the
    measured ones.  Each side is fitted from its own partial's times,
    bounded by its physical rate (the HBM peak; the host read bandwidth of
    the run) and with single outlying points left out (a point more than 15%
    off the fit of the others, e.g. a GPU partial slowed by clocks that
    dropped while the GPU waited milliseconds for the host side); the
    residuals and the points left out are reported."""
    from scope_amd.scheduler import ShareScheduler, fit_side_report

    gpts = [(r["gpu_tokens"] * 1152.0, r["gpu_partial_us_per_layer"] * 1e-6) for r in rows]
    hpts = [(r["host_tokens"] * 1152.0, r["host_partial_us_per_layer"] * 1e-6) for r in rows
            if r["host_tokens"] > 0]
    gfit = fit_side_report(gpts, max_rate_bps=HBM_PEAK_GBS * 1e9, reject_rel=0.15)
    hfit = fit_side_report(hpts, max_rate_bps=host_bw_gbs * 1e9 if host_bw_gbs else None,
                           reject_rel=0.15)
    gpu, hst = gfit.side, hfit.side
    mixed = [r for r in rows if r["host_tokens"] > 0]
    resid = [r["us_per_layer"] - max(r["gpu_partial_us_per_layer"],
                                     r["host_partial_us_per_layer"]) for r in mixed]
    only = [r for r in rows if r["host_tokens"] == 0]
    gpu_only_resid = [r["us_per_layer"] - r["gpu_partial_us_per_layer"] for r in only]
    sched = ShareScheduler(gpu=gpu, host=hst, xfer_s=float(np.median(resid)) * 1e-6,
                           merge_s=0.0,
                           merge_gpu_only_s=(float(np.median(gpu_only_resid)) * 1e-6
                                             if only else 0.0))
    W = rows[0]["layer_bytes"]
    pred = [sched.predict(r["share"], W)["layer"] * 1e6 for r in rows]
    share_of = {r["gpu_tokens"] * 1152.0: r["share"] for r in rows}
    share_of_h = {r["host_tokens"] * 1152.0: r["share"] for r in rows}
    return {
        "gpu_fit": {"fixed_us": round(gpu.fixed_s * 1e6, 1),
                    "gbs": round(gpu.rate_bps / 1e9, 1),
                    "bound_gbs": HBM_PEAK_GBS, "rate_capped": gfit.rate_capped,
                    "shares_left_out": [share_of[b] for b, _ in gfit.rejected]},
        "host_fit": {"fixed_us": round(hst.fixed_s * 1e6, 1),
                     "gbs": round(hst.rate_bps / 1e9, 1),
                     "bound_gbs": host_bw_gbs, "rate_capped": hfit.rate_capped,
                     "shares_left_out": [share_of_h[b] for b, _ in hfit.rejected]},
        "xfer_merge_us": round(sched.xfer_s * 1e6, 1),
        "r_balance": round(sched.balance_share(W), 4),
        "r_choice_unbounded": sched.choose(W),
        "shares": [r["share"] for r in rows],
        "predicted_us": [round(x, 1) for x in pred],
        "measured_us": [r["us_per_layer"] for r in rows],
        "rel_error": [round(x / r["us_per_layer"] - 1.0, 3) for x, r in zip(pred, rows)],
    }


def lognormal_lens(B, seed, median=4096, sigma=1.0, lo=256, hi=65536):
    """Sequence lengths ~ lognormal(ln median, sigma) clipped to [lo, hi]."""
    rng = np.random.default_rng(seed)
    x = rng.lognormal(mean=math.log(median), sigma=sigma, size=B)
    return np.clip(np.floor(x), lo, hi).astype(np.int64)


def mla_model_bench(*, B, layers, lens, share, steps, warmup, seed, dev, threads, label):
    """One decode step of a `layers`-layer absorbed-MLA model over a
    token-range-partitioned latent cache, per layer in dependency order:
    q -> host (pinned, ws_copy), GPU split step (append + partial over the
    HBM pages) while the host partial (wh_mla_partial) attends the host
    pages, merge (reading the host partial from pinned memory in place).  The q copy of layer l+1 is ordered after layer l's
    merge on the stream, as the real model's next query would be.  Returns
    the per-layer critical path and its parts."""
    import torch

    from scope_amd import host, ops

    L = ops.lib()
    H = 16
    rows = B * H
    lens = np.asarray(lens, np.int64)
    g_tok = np.floor(share * lens).astype(np.int64)
    h_tok = lens - g_tok
    rng = np.random.default_rng(seed)
    extra = warmup + steps + 1
    g_table, g_pages = _page_table(g_tok, extra, rng)
    h_table, h_pages = _host_pages(h_tok, rng)
    gen = torch.Generator(device=dev).manual_seed(seed)
    g_pools = [_randn_bf16((g_pages, PAGE, 576), gen, 0.5, dev) for _ in range(layers)]
    h_pools = [_randn_bf16((h_pages, PAGE, 576), gen, 0.5, dev).cpu() for _ in range(layers)]
    page_table = torch.from_numpy(g_table).to(dev)
    lens_d = torch.zeros((layers, 2, B), dtype=torch.int32, device=dev)
    lens_d[:, 0] = torch.from_numpy(g_tok.astype(np.int32)).to(dev)
    # q_nope and q_pe of a layer are adjacent (one copy to the host); the host
    # partial's out and lse are adjacent (one copy back)
    qbuf = _randn_bf16((layers, rows * 576), gen, 0.5, dev)
    qn = [qbuf[l, :rows * 512].view(rows, 512) for l in range(layers)]
    qp = [qbuf[l, rows * 512:].view(rows, 64) for l in range(layers)]
    kv_new = _randn_bf16((layers, B, 1, 576), gen, 0.5, dev)
    out_g = torch.empty((rows, 512), dtype=torch.float32, device=dev)
    lse_g = torch.empty((rows,), dtype=torch.float32, device=dev)
    out = torch.empty((rows, 512), dtype=torch.bfloat16, device=dev)
    q_h = torch.empty((rows * 576,), dtype=torch.bfloat16, pin_memory=True)
    qn_h, qp_h = q_h[:rows * 512].view(rows, 512), q_h[rows * 512:].view(rows, 64)
    # the host partial: bf16 out (wh_mla_partial_bf16) and fp32 lse, pinned
    oc_h = torch.empty((rows, 512), dtype=torch.bfloat16, pin_memory=True)
    lc_h = torch.empty((rows,), dtype=torch.float32, pin_memory=True)
    h_lens = torch.from_numpy(h_tok.astype(np.int32))
    h_tab = torch.from_numpy(h_table)
    with_host = bool(h_tok.sum() > 0)
    scale = 192 ** -0.5
    h_calls = [host.mla_partial(qn_h, qp_h, h_pools[l], h_tab, h_lens, scale, threads, oc_h,
                                lc_h, prepare=True) for l in range(layers)]
    max_len0 = int(g_tok.max())
    nwg, wsb = ops.decode_plan(1, B, H, max_len0 + extra, 0)
    ws = torch.zeros(max(wsb, 256), dtype=torch.uint8, device=dev)
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    cap = PAGE * g_table.shape[1]
    ev_q = torch.cuda.Event()
    e_a = [HipTimingEvent() for _ in range(layers)]
    e_b = [HipTimingEvent() for _ in range(layers)]
    f_step, f_merge = L.ws_mla_append_decode_split, L.ws_merge_split

    def one_step(i, timed):
        cpu_s = 0.0
        for l in range(layers):
            if with_host:  # the query to the host by the library's copy kernel
                ops.copy_(q_h, qbuf[l])
                ev_q.record()
            li, lo = p(lens_d[l, i % 2]), p(lens_d[l, (i + 1) % 2])
            if timed:
                e_a[l].record()
            rc = f_step(p(qn[l]), p(qp[l]), p(kv_new[l]), ctypes.c_int64(576),
                        ctypes.c_void_p(kv_new[l].data_ptr() + 1024), ctypes.c_int64(576),
                        p(g_pools[l]), p(page_table), li, lo, B, H, PAGE, g_table.shape[1],
                        g_pages, max_len0 + i + 1, nwg, ctypes.c_float(scale), p(out_g),
                        p(lse_g), p(ws), ctypes.c_size_t(wsb), stream)
            if timed:
                e_b[l].record()
            if with_host:
                ev_q.synchronize()
                t0 = time.perf_counter()
                h_calls[l]()
                cpu_s += time.perf_counter() - t0
                # the merge reads the host partial in place (pinned memory)
                rc |= f_merge(lo, B, 1, H, 512, cap, nwg, p(out_g), p(lse_g), p(ws),
                              ctypes.c_size_t(wsb), p(oc_h), p(lc_h), None,
                              ops.PARTIAL_LSE_BF16, p(out), None, None, stream)
            else:
                rc |= f_merge(lo, B, 1, H, 512, cap, nwg, p(out_g), p(lse_g), p(ws),
                              ctypes.c_size_t(wsb), None, None, None, 0, p(out), None, None,
                              stream)
            if rc:
                raise RuntimeError(f"{label}: {L.ws_last_error().decode()}")
        return cpu_s

    for i in range(warmup):
        one_step(i, False)
    torch.cuda.synchronize()
    walls, cpus, gpus = [], [], []
    for k in range(steps):
        i = warmup + k
        t0 = time.perf_counter()
        cpus.append(one_step(i, True))
        torch.cuda.synchronize()
        walls.append(time.perf_counter() - t0)
        gpus.append(sum(e_a[l].elapsed_time(e_b[l]) for l in range(layers)) * 1e-3)
    wall = float(np.median(walls))
    cpu = float(np.median(cpus))
    gpu = float(np.median(gpus))
    g_bytes = float(g_tok.sum()) * 1152
    h_bytes = float(h_tok.sum()) * 1152
    return {
        "label": label, "batch": B, "layers": layers, "share": share,
        "gpu_tokens": int(g_tok.sum()), "host_tokens": int(h_tok.sum()),
        "host_threads": threads, "workgroups": nwg,
        "us_per_layer": round(wall / layers * 1e6, 1),
        "ms_per_step": round(wall * 1e3, 3),
        "gpu_partial_us_per_layer": round(gpu / layers * 1e6, 1),
        "gpu_partial_gbs": round(g_bytes / (gpu / layers) / 1e9, 1) if gpu > 0 else None,
        "host_partial_us_per_layer": round(cpu / layers * 1e6, 1) if with_host else 0.0,
        "host_partial_gbs": round(h_bytes / (cpu / layers) / 1e9, 2) if with_host else None,
        "layer_bytes": int(g_bytes + h_bytes),
    }


def share_control_bench(*, B, layers, lens, start_share, budget_frac, steps, seed, dev, threads,
                        label, async_moves=False):
    """The share controller driving a two-sided paged MLA cache
    (scope_amd.paged.PagedMlaCache + scheduler.ShareController) through
    `steps` decode steps of a `layers`-layer model, with an HBM budget of
    budget_frac of the cache's bytes, starting from share start_share.
    With async_moves the page copies of a move run under the following
    steps (side stream) instead of between them.  Returns the per-step
    share, wall time per layer and the moves."""
    import torch

    from scope_amd.paged import PagedMlaCache
    from scope_amd.scheduler import ShareController, ShareScheduler, Side

    H = 16
    lens = [int(x) for x in lens]
    bpt = 1152
    total = sum(lens) * bpt * layers
    sched = ShareScheduler(gpu=Side(15e-6, 5e12, max_rate_bps=HBM_PEAK_GBS * 1e9),
                           host=Side(40e-6, 50e9, max_rate_bps=host_read_gbs(threads) * 1e9),
                           xfer_s=60e-6, hbm_budget_bytes=budget_frac * total)
    ctl = ShareController(sched, bpt, layers, PAGE)
    host0 = ctl.targets_for(start_share, lens)
    need_h = sum(-(-L // PAGE) for L in lens) + B  # host pages for any share
    need_g = int(budget_frac * sum(lens) / PAGE) + 2 * B + (steps + PAGE) * B // PAGE
    cache = PagedMlaCache(layers, B, max_tokens=max(lens) + steps + 1, page_size=PAGE,
                          host_pages=need_h, gpu_pages=need_g, device=dev)
    cache.reserve_layout(lens, host0)
    gen = torch.Generator(device=dev).manual_seed(seed)
    cache.gpu.latent.normal_(0.0, 0.5, generator=gen)
    rnd = _randn_bf16((need_h, PAGE, 576), gen, 0.5, dev).cpu()
    for l in range(layers):
        cache.host.data[0][l].copy_(rnd)
    del rnd
    rows = B * H
    qn = [_randn_bf16((rows, 512), gen, 0.5, dev) for _ in range(layers)]
    qp = [_randn_bf16((rows, 64), gen, 0.5, dev) for _ in range(layers)]
    kv_new = _randn_bf16((layers, B, 1, 576), gen, 0.5, dev)
    cache.attach(ctl, async_moves=async_moves)
    scale = 192 ** -0.5
    per_step = []
    cur = torch.cuda.current_stream(dev)
    torch.cuda.synchronize()
    for i in range(steps):
        # a decode loop waits for its own stream (the step's outputs), not for
        # the side stream of a move's copies
        cur.synchronize()
        t0 = time.perf_counter()
        for l in range(layers):
            cache.step(l, qn[l], qp[l], kv_new[l, :, :, :512], kv_new[l, :, :, 512:], scale,
                       host_threads=threads)
        cur.synchronize()
        dt = time.perf_counter() - t0
        per_step.append({"step": i, "share_after": round(ctl.shares[-1], 4),
                         "moving": cache.moving, "ms": round(dt * 1e3, 2)})
        log(f"share control step {i}: share {per_step[-1]['share_after']}, "
            f"{per_step[-1]['ms']} ms" + (", a move in flight" if cache.moving else ""))
    cache.finish_boundaries()
    # a move's stall (the copies when waited for; else only their issue and
    # the switch) is counted at the step that started it
    for i, st in enumerate(per_step):
        moved = [m for m in ctl.moves if m.step == i + 1]
        stall = sum(m.stall_seconds for m in moved)
        st["us_per_layer_excl_move"] = round((st["ms"] * 1e-3 - stall) / layers * 1e6, 1)
        st["move_stall_ms"] = round(stall * 1e3, 2)
        st["move_pages_per_layer"] = sum(m.pages for m in moved)
    moves = [{"step": m.step, "from": round(m.share_from, 4), "to": round(m.share_to, 4),
              "pages_per_layer": m.pages, "ms": round(m.seconds * 1e3, 1),
              "stall_ms": round(m.stall_seconds * 1e3, 2),
              "copy_ms": round(m.copy_seconds * 1e3, 1),
              "gbs": round(m.pages * PAGE * bpt * layers / m.copy_seconds / 1e9, 1)}
             for m in ctl.moves]
    return {"label": label, "batch": B, "layers": layers, "start_share": start_share,
            "async_moves": async_moves,
            "total_ms": round(sum(p["ms"] for p in per_step), 1),
            "hbm_budget_frac": budget_frac, "host_threads": threads,
            "capacity_share_start": round(sched.capacity_share(sum(lens) * bpt, layers), 4),
            "chosen": [round(r, 4) for r in ctl.chosen], "steps": per_step, "moves": moves,
            "gpu_rate_gbs": round(sched.gpu.rate_bps / 1e9, 1),
            "host_rate_gbs": round(sched.host.rate_bps / 1e9, 1)}


# ---------------------------------------------------------------------------
# CPU baseline: the clean-room AVX-512 BF16 host kernel (libwshost.so), with
# the oracle's scalar C restatement of the reference CPU kernel beside it


def _host_info():
    info = {"affinity_cores": len(os.sched_getaffinity(0))}
    try:
        txt = open("/proc/cpuinfo").read()
        m = re.search(r"model name\s*:\s*(.*)", txt)
        info["cpu_model"] = m.group(1).strip() if m else "?"
        fam = re.search(r"cpu family\s*:\s*(\d+)", txt)
        mod = re.search(r"model\s*:\s*(\d+)", txt)
        if fam and mod:  # e.g. family 25 = Zen 3/4, 26 = Zen 5 on AMD
            info["cpu_family_model"] = f"{fam.group(1)}/{mod.group(1)}"
        flags = set(re.search(r"flags\s*:\s*(.*)", txt).group(1).split())
        info["isa"] = [f for f in ("avx2", "avx512f", "avx512bw", "avx512_bf16",
                                   "amx_bf16") if f in flags]
    except Exception:  # pragma: no cover - informational only
        pass
    return info


def _pin_threads(n):
    """Pins this process to its first n allowed cores (the CPU column's stated
    core set); returns the previous affinity for _unpin."""
    old = os.sched_getaffinity(0)
    cores = sorted(old)[:max(1, n)]
    os.sched_setaffinity(0, cores)
    return old, cores


def cpu_baseline(data, Hkv, G, budget_s, threads):
    """The CPU column: the clean-room AVX-512 BF16 host kernel (wh_gqa_partial,
    the production counterpart of the reference's fused_cpu_attn) over the
    same GPU-share tokens as the step, called once per sequence as the
    reference contract requires (one length per call, kernel/cpu_attn.cpp:590),
    on `threads` pinned cores; median of >= 10 passes over all sequences
    after 3 warm-up passes.  Beside it, the oracle's scalar C restatement of
    the reference kernel over a bounded sample (the checker's speed, context
    only)."""
    import torch

    from oracle import port
    from scope_amd import host

    k_pages, v_pages, table, gpu_tokens, q = data
    D = 128
    B = len(gpu_tokens)
    scale = D ** -0.5
    # host copies of every sequence's GPU share, dense [Hkv, g, D] (the layout
    # the reference CPU kernel takes)
    seqs = []
    for b in range(B):
        g = int(gpu_tokens[b])
        if g <= 0:
            continue
        n_pages = -(-g // PAGE)
        pids = torch.from_numpy(table[b, :n_pages].astype(np.int64)).to(k_pages.device)
        k = k_pages[pids].permute(1, 0, 2, 3).reshape(Hkv, n_pages * PAGE, D)[:, :g]
        v = v_pages[pids].permute(1, 0, 2, 3).reshape(Hkv, n_pages * PAGE, D)[:, :g]
        seqs.append((b, g, k.contiguous().cpu(), v.contiguous().cpu()))
    if not seqs:
        return None
    q_h = q.cpu()
    outs = [(torch.empty((1, Hkv * G, D), dtype=torch.float32),
             torch.empty((1, Hkv * G), dtype=torch.float32)) for _ in seqs]
    # dense rows are the one-page-per-sequence case of the paged call
    calls = [host.gqa_partial(q_h[b:b + 1], k.view(1, Hkv, g, D), v.view(1, Hkv, g, D),
                              torch.zeros((1, 1), dtype=torch.int32), [g], scale, threads, o,
                              l, prepare=True)
             for (b, g, k, v), (o, l) in zip(seqs, outs)]
    old_aff, cores = _pin_threads(threads)
    try:
        for _ in range(3):
            for c in calls:
                c()
        passes = []
        spent = 0.0
        while len(passes) < 10 or (spent < budget_s and len(passes) < 200):
            t0 = time.perf_counter()
            for c in calls:
                c()
            dt = time.perf_counter() - t0
            passes.append(dt)
            spent += dt
        bw = host_read_gbs(threads)
    finally:
        os.sched_setaffinity(0, old_aff)
    t = float(np.median(passes))
    nbytes = sum(g for _, g, _, _ in seqs) * Hkv * 2 * D * 2
    gbs = nbytes / t / 1e9

    # the oracle's scalar C restatement, bounded sample (context only)
    port.lib()
    qh = q_h.view(torch.int16).numpy().view(np.uint16).reshape(B, Hkv, G, D)
    port_bytes, port_s, n_port = 0.0, 0.0, 0
    while port_s < min(2.0, budget_s):
        b, g, k, v = seqs[n_port % len(seqs)]
        kh = k.view(torch.int16).numpy().view(np.uint16)
        vh = v.view(torch.int16).numpy().view(np.uint16)
        t0 = time.perf_counter()
        port.cpu_attn(qh[b], kh, vh, scale, normalize=True, n_threads=threads)
        port_s += time.perf_counter() - t0
        port_bytes += g * Hkv * 2 * D * 2
        n_port += 1
    return {
        "value": round(gbs, 2),
        "unit": "GB/s",
        "cores": threads,
        "kind": "clean-room",
        "kernel": ("wh_gqa_partial: clean-room AVX-512 BF16 / OpenMP implementation of the "
                   "reference CPU kernel's contract (fused_cpu_attn, kernel/cpu_attn.cpp:"
                   "572-636), libwshost.so"),
        "pinned_cores": f"{cores[0]}-{cores[-1]}" if len(cores) > 1 else str(cores[0]),
        "sample": (f"the whole GPU share of the step ({sum(g for _, g, _, _ in seqs)} tokens "
                   f"of {len(seqs)} sequences, {nbytes / 1e6:.0f} MB of bf16 K/V), one call "
                   f"per sequence ({Hkv} KV rows x {G} heads, one length per call); median "
                   f"of {len(passes)} passes after 3 warm-up passes"),
        "us_per_layer_equiv": round(t * 1e6, 1),
        "host_read_gbs": bw,
        "host_read_probes_gbs": host_read_probes(threads),
        "frac_of_host_read": round(gbs / bw, 3) if bw else None,
        "oracle_port_gbs": round(port_bytes / port_s / 1e9, 2) if port_s > 0 else None,
        "oracle_port_sample": f"{n_port} calls of the oracle's scalar C restatement, "
                              f"{port_s:.1f} s",
    }


# ---------------------------------------------------------------------------
# traffic from the committed rocprofv3 PMC summary


# Workloads timed beside the headline (all by default; --workloads picks some):
#   shares     headline shape at r = 0.25, 0.75
#   qwen3      Qwen3 B4 length sweep 8k..128k, r = 1
#   single     Qwen3 B1 L4096 in one partition
#   mla        DeepSeek-V2-Lite B8 L16384 r 0.5
#   mla_sweep  DeepSeek-V2-Lite B8 length sweep 8k..128k
#   host       native host partial rates and the host read bandwidth
#   model      27-layer DeepSeek-V2-Lite decode, B32 lognormal, every share
#   migrate    boundary movement of a paged two-sided MLA cache (4 layers, B32)
#   epilogue   MLA merge + W_UV: fused kernel against merge then bmm
#   mla128     DeepSeek-V2 (128 heads) B4 L32768, r = 1
WORKLOADS = ("shares", "qwen3", "single", "mla", "mla_sweep", "mla128", "host", "model",
             "migrate", "epilogue")
# Extra workloads for profiling runs (not in the default set): the MLA layer at
# B8 L32768, r = 1, on its own.
EXTRA_WORKLOADS = ("mla32k",)

# The kernel the headline roofline is measured on (its rocprofv3 name).
HEAD_KERNEL = "ws::gqa_decode_kernel<4, 128, 128, true>"


MLA_KERNEL = "ws::mla_decode_kernel<true>"


def committed_counters(workload_key, kernel):
    """The committed rocprofv3 counter summary of a workload's kernel from
    profiles/traffic.json (HBM traffic over algorithmic bytes, MFMA
    utilisation, LDS bank-conflict share), or None when none is committed for
    this kernel."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            ent = json.load(f).get(workload_key)
    except (OSError, ValueError):
        return None
    if ent is None or ent.get("kernel") != kernel:
        return None
    keep = ("traffic_over_algorithmic", "traffic_bytes_per_launch", "mfma_util",
            "mfma_busy_cycles_per_dispatch", "lds_bank_conflict_frac", "kernel_trace_mean_us")
    out = {k: ent[k] for k in keep if k in ent}
    out["source"] = f"profiles/traffic.json[{workload_key}] ({kernel})"
    return out


def committed_traffic(workload_key, kernel=HEAD_KERNEL):
    """HBM bytes per launch of the GQA partial kernel from profiles/, if a
    FETCH_SIZE/WRITE_SIZE summary for this workload and this kernel is
    committed (a summary of another kernel is not reported)."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(path):
        return None
    try:
        with open(path) as f:
            doc = json.load(f)
        ent = doc.get(workload_key)
        if ent is None or ent.get("kernel") != kernel:
            return None
        return ent.get("traffic_bytes_per_launch")
    except (OSError, ValueError):
        return None


# ---------------------------------------------------------------------------


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--share", type=float, default=0.5)
    ap.add_argument("--seed", type=int, default=2000)
    ap.add_argument("--cpu-budget", type=float, default=10.0,
                    help="seconds of CPU time for the CPU baseline (0 = skip)")
    ap.add_argument("--headline-only", action="store_true",
                    help="only the headline workload (no sweep, MLA, other shares)")
    ap.add_argument("--wg", type=int, default=0,
                    help="workgroups of the headline GQA call (0 = library choice)")
    ap.add_argument("--wg-sweep", type=str, default="",
                    help="comma list of workgroup counts to time on the headline")
    ap.add_argument("--mla-wg-sweep", type=str, default="",
                    help="comma list of workgroup counts to time on the MLA layer")
    ap.add_argument("--page-size", type=int, default=64,
                    help="tokens per HBM page (a multiple of 32)")
    ap.add_argument("--contiguous-pages", action="store_true",
                    help="assign each sequence's pages in order instead of shuffled")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run a plain 256 MiB device copy (PMC scale factor)")
    ap.add_argument("--workloads", type=str, default=",".join(WORKLOADS),
                    help="comma list of the workloads beside the headline: "
                         + ", ".join(WORKLOADS + EXTRA_WORKLOADS))
    ap.add_argument("--model-layers", type=int, default=27,
                    help="layers of the multi-layer MLA decode with host partials (0 = skip)")
    ap.add_argument("--model-steps", type=int, default=5,
                    help="timed decode steps of the multi-layer MLA run")
    ap.add_argument("--skip-headline", action="store_true",
                    help="run only the --workloads (profiling runs of one workload); "
                         "prints their results without the headline line")
    args = ap.parse_args()
    global CONTIGUOUS_PAGES, PAGE
    CONTIGUOUS_PAGES = args.contiguous_pages
    if args.page_size <= 0 or args.page_size % 32:
        ap.error("--page-size must be a positive multiple of 32")
    PAGE = args.page_size

    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}): the GPU "
              "partition shards by (sequence, KV head) rows with no exchange, and no "
              "multi-GPU figure is produced", file=sys.stderr)
        sys.exit(2)

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    from scope_amd import ops

    ops.lib()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    # headline: Mixtral shape, B 16, L ~ U[1024, 32768], trailing floor(r L) on the GPU
    B, Hkv, G = 16, 8, 4
    lens = np.random.default_rng(args.seed).integers(1024, 32769, B)
    head = data = None
    if not args.skip_headline:
        log(f"headline: mixtral gqa B={B} share={args.share} lens={lens.tolist()}")
        head = gqa_step_bench(B=B, Hkv=Hkv, G=G, lens=lens, share=args.share,
                              steps=args.steps, warmup=args.warmup, seed=args.seed, dev=dev,
                              with_host=args.share < 1.0, label="mixtral_b16", wg=args.wg)
        data = head.pop("_data")
        log(f"headline: {head['us_per_layer']} us/layer, partial {head['partial_us']} us "
            f"= {head['partial_gbs']} GB/s")

    extra = {}
    if args.wg_sweep:
        sw = []
        for w in [int(x) for x in args.wg_sweep.split(",")]:
            res = gqa_step_bench(B=B, Hkv=Hkv, G=G, lens=lens, share=args.share,
                                 steps=args.steps, warmup=args.warmup, seed=args.seed,
                                 dev=dev, with_host=True, label=f"mixtral_b16_wg{w}", wg=w)
            res.pop("_data")
            sw.append({k: res[k] for k in ("workgroups", "us_per_layer", "partial_us",
                                           "partial_gbs")})
            log(f"wg {w}: {res['us_per_layer']} us/layer, partial {res['partial_us']} us "
                f"= {res['partial_gbs']} GB/s")
        extra["wg_sweep"] = sw
    if args.mla_wg_sweep:
        sw = []
        for w in [int(x) for x in args.mla_wg_sweep.split(",")]:
            res = mla_step_bench(B=8, H=16, lens=[16384] * 8, share=0.5, steps=args.steps,
                                 warmup=args.warmup, seed=args.seed + 3, dev=dev,
                                 label=f"mla_wg{w}", wg=w)
            sw.append({k: res[k] for k in ("workgroups", "us_per_layer", "partial_us",
                                           "partial_gbs")})
            log(f"mla wg {w}: {res['us_per_layer']} us/layer, partial {res['partial_us']} "
                f"us = {res['partial_gbs']} GB/s")
        extra["mla_wg_sweep"] = sw
    W = set() if args.headline_only else set(args.workloads.split(","))
    unknown = W - set(WORKLOADS) - set(EXTRA_WORKLOADS)
    if unknown:
        ap.error(f"unknown workloads {sorted(unknown)}; choose from {WORKLOADS}")
    if "shares" in W:
        by_share = []
        for r in (0.25, 0.75):
            res = gqa_step_bench(B=B, Hkv=Hkv, G=G, lens=lens, share=r, steps=args.steps,
                                 warmup=args.warmup, seed=args.seed, dev=dev,
                                 with_host=True, label=f"mixtral_b16_r{r}")
            res.pop("_data")
            by_share.append(res)
            log(f"share {r}: {res['us_per_layer']} us/layer, partial {res['partial_gbs']} GB/s")
        extra["by_share"] = by_share
    if "qwen3" in W:
        sweep = []
        for Lq in (8192, 32768, 65536, 131072):
            res = gqa_step_bench(B=4, Hkv=4, G=8, lens=[Lq] * 4, share=1.0,
                                 steps=max(10, args.steps // 2), warmup=args.warmup,
                                 seed=args.seed + Lq, dev=dev, with_host=False,
                                 label=f"qwen3_b4_L{Lq}")
            res.pop("_data")
            sweep.append(res)
            log(f"qwen3 B4 L={Lq}: {res['us_per_layer']} us/layer, partial "
                f"{res['partial_us']} us = {res['partial_gbs']} GB/s")
        extra["kv_len_sweep"] = sweep
    if "single" in W:
        one = gqa_step_bench(B=1, Hkv=4, G=8, lens=[4096], share=1.0, steps=args.steps,
                             warmup=args.warmup, seed=args.seed + 1, dev=dev,
                             with_host=False, label="qwen3_b1_L4096")
        one.pop("_data")
        extra["single_partition"] = one
    if "mla" in W:
        mla = mla_step_bench(B=8, H=16, lens=[16384] * 8, share=0.5, steps=args.steps,
                             warmup=args.warmup, seed=args.seed + 3, dev=dev,
                             label="dsv2lite_mla_b8_L16384")
        mla["counters"] = committed_counters("dsv2lite_mla_b8_L16384_r0.5", MLA_KERNEL)
        extra["mla"] = mla
        log(f"mla: {mla['us_per_layer']} us/layer, partial {mla['partial_us']} us = "
            f"{mla['partial_gbs']} GB/s, {mla['partial_tflops']} TFLOP/s")
    if "mla32k" in W:
        res = mla_step_bench(B=8, H=16, lens=[32768] * 8, share=1.0,
                             steps=max(10, args.steps // 2), warmup=args.warmup,
                             seed=args.seed + 7 + 32768, dev=dev, label="dsv2lite_mla_b8_L32768")
        res["counters"] = committed_counters("dsv2lite_mla_b8_L32768_r1", MLA_KERNEL)
        extra["mla32k"] = res
        log(f"mla B8 L=32768: {res['us_per_layer']} us/layer, partial {res['partial_us']} us "
            f"= {res['partial_gbs']} GB/s")
    if "mla_sweep" in W:
        msweep = []
        for Lm in (8192, 32768, 65536, 131072):
            res = mla_step_bench(B=8, H=16, lens=[Lm] * 8, share=1.0,
                                 steps=max(10, args.steps // 2), warmup=args.warmup,
                                 seed=args.seed + 7 + Lm, dev=dev, label=f"dsv2lite_mla_b8_L{Lm}")
            if Lm == 32768:
                res["counters"] = committed_counters("dsv2lite_mla_b8_L32768_r1", MLA_KERNEL)
            msweep.append(res)
            log(f"mla B8 L={Lm}: {res['us_per_layer']} us/layer, partial {res['partial_us']} us "
                f"= {res['partial_gbs']} GB/s")
        extra["mla_kv_len_sweep"] = msweep

    if "mla128" in W:
        # DeepSeek-V2 absorbed MLA, 128 heads over the shared latent: the
        # one-pass HBM time of the latent is the bound the step is compared to
        res = mla_step_bench(B=4, H=128, lens=[32768] * 4, share=1.0,
                             steps=max(10, args.steps // 2), warmup=args.warmup,
                             seed=args.seed + 128, dev=dev, label="dsv2_mla_h128_b4_L32768")
        one_pass = 4 * 32768 * 1152 / (HBM_PEAK_GBS * 1e3)
        res["one_pass_hbm_us"] = round(one_pass, 2)
        res["partial_over_one_pass"] = round(res["partial_us"] / one_pass, 2)
        extra["mla128"] = res
        log(f"mla H128 B4 L=32768: {res['us_per_layer']} us/layer, partial {res['partial_us']} "
            f"us = {res['partial_over_one_pass']}x the one-pass HBM time, "
            f"{res.get('partial_tflops')} TFLOP/s")

    th = _host_threads()
    if "host" in W:
        # native host partial rates (the other half of the partitioned step)
        h_mix = lens - np.floor(args.share * lens).astype(np.int64)
        hp = [host_gqa_bench(Hkv=Hkv, G=G, host_tokens=h_mix, reps=5, seed=args.seed + 11,
                             dev=dev, threads=th, label=f"mixtral_b16_r{args.share}_host"),
              host_mla_bench(host_tokens=[8192] * 8, reps=5, seed=args.seed + 12, dev=dev,
                             threads=th, label="dsv2lite_mla_b8_L16384_r0.5_host")]
        bw = host_read_gbs(th)
        hinfo = _host_info()
        for r in hp:
            r.update(hinfo)
            r["host_read_gbs"] = bw
            r["host_read_probes_gbs"] = host_read_probes(th)
            r["frac_of_host_read"] = round(r["gbs"] / bw, 3)
            log(f"host partial {r['label']}: {r['us']} us = {r['gbs']} GB/s on {th} threads "
                f"({r['frac_of_host_read']:.0%} of the {bw} GB/s host read bandwidth)")
        extra["host_partial"] = hp
    if "model" in W and args.model_layers > 0:
        # DeepSeek-V2-Lite decode step: B 32, lognormal lengths, every share
        m_lens = lognormal_lens(32, args.seed + 5)
        log(f"mla model: B=32 layers={args.model_layers} lens median "
            f"{int(np.median(m_lens))} max {int(m_lens.max())} total {int(m_lens.sum())}")
        rows = []
        for r in (0.1, 0.3, 0.5, 0.7, 0.9, 1.0):
            res = mla_model_bench(B=32, layers=args.model_layers, lens=m_lens, share=r,
                                  steps=args.model_steps, warmup=2, seed=args.seed + 13,
                                  dev=dev, threads=th, label=f"dsv2lite_mla_b32_r{r}")
            rows.append(res)
            log(f"mla model r={r}: {res['us_per_layer']} us/layer (gpu partial "
                f"{res['gpu_partial_us_per_layer']} us, host partial "
                f"{res['host_partial_us_per_layer']} us)")
            torch.cuda.empty_cache()
        extra["mla_model"] = {"lens_seed": args.seed + 5, "lens": m_lens.tolist(),
                              "length_model": "lognormal(ln 4096, 1.0) clipped [256, 65536]",
                              "by_share": rows,
                              "scheduler": share_model(rows, host_read_gbs(th))}
        sc = share_control_bench(B=32, layers=args.model_layers, lens=m_lens, start_share=0.1,
                                 budget_frac=0.5, steps=10, seed=args.seed + 23, dev=dev,
                                 threads=th, label="dsv2lite_mla_b32_share_control")
        extra["mla_model"]["share_control"] = sc
        torch.cuda.empty_cache()
        sa = share_control_bench(B=32, layers=args.model_layers, lens=m_lens, start_share=0.1,
                                 budget_frac=0.5, steps=10, seed=args.seed + 23, dev=dev,
                                 threads=th, label="dsv2lite_mla_b32_share_control_async",
                                 async_moves=True)
        extra["mla_model"]["share_control_async"] = sa
        log(f"share control: {sc['total_ms']} ms over 10 steps waiting for the moves, "
            f"{sa['total_ms']} ms with the copies under the steps")
        torch.cuda.empty_cache()
        sm = extra["mla_model"]["scheduler"]
        log(f"share model: gpu {sm['gpu_fit']}, host {sm['host_fit']}, r_balance "
            f"{sm['r_balance']}, predicted/measured us per layer "
            f"{list(zip(sm['predicted_us'], sm['measured_us']))}, relative error "
            f"{sm['rel_error']}")

    if "epilogue" in W:
        ep = [epilogue_bench(B=8, L=8192, steps=args.steps, seed=args.seed + 19, dev=dev,
                             label="dsv2lite_mla_b8_L8192"),
              epilogue_bench(B=32, L=4096, steps=args.steps, seed=args.seed + 20, dev=dev,
                             label="dsv2lite_mla_b32_L4096")]
        for r in ep:
            log(f"epilogue {r['label']}: merge + bmm {r['merge_then_bmm_us']} us, fused "
                f"{r['fused_uv_us']} us")
        extra["epilogue"] = ep

    if "migrate" in W:
        mig = migration_bench(B=32, layers=4, lens=lognormal_lens(32, args.seed + 5),
                              seed=args.seed + 17, dev=dev, label="dsv2lite_mla_b32_4layers")
        extra["migration"] = mig
        log(f"migration: {mig}")
        torch.cuda.empty_cache()

    if args.copy_calibration:
        n = 256 << 20
        src = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"copy calibration: 5 x {n} bytes read + written")

    if head is None:  # a profiling run of the chosen workloads only
        print(json.dumps({"skip_headline": True, **extra}), flush=True)
        return

    cpu = None
    if args.cpu_budget > 0:
        threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or len(os.sched_getaffinity(0))
        cpu = cpu_baseline(data, Hkv, G, args.cpu_budget, threads)
        cpu.update(_host_info())
        log(f"cpu baseline: {cpu['value']} GB/s on {threads} threads")

    wk = f"mixtral_b16_r{args.share}"
    roofline = {
        "bound": "hbm",
        "achieved": head["partial_gbs"],
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(head["partial_gbs"] / HBM_PEAK_GBS, 4),
        "traffic": committed_traffic(wk),
        "kernel": f"{HEAD_KERNEL} (ws_gqa_append_decode_split: append + load-balanced "
                  "split-KV partial, one launch; combine in the merge launch)",
        "algorithmic_bytes_per_launch": head["partial_bytes"],
        "mean_launch_us": head["partial_us"],
    }
    line = {
        "metric": METRIC,
        "value": round(head["step_gbs"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["us_per_layer"] / 1e3, 5),
        "us_per_layer": head["us_per_layer"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": (f"partitioned GQA decode step (append + split-KV partial + LSE "
                         f"merge), Mixtral-8x7B layer: batch {B}, 32 q / 8 KV heads, "
                         f"head_dim 128, L ~ U[1024, 32768], GPU share r={args.share} "
                         f"in 64-token pages"),
            "batch": B, "q_heads": 32, "kv_heads": 8, "head_dim": 128,
            "share": args.share, "page_size": PAGE,
            "gpu_tokens": head["gpu_tokens"], "seed": args.seed,
        },
        "roofline": roofline,
        "cpu_baseline": cpu,
        "headline": head,
    }
    line.update(extra)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
