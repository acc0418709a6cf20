"""Partition arithmetic of the token-range-split KV cache (host-side integers).

A sequence of L tokens is split at a boundary: the leading tokens stay in
host memory (the CPU partial attends over them) and the trailing tokens live
in HBM pages (the GPU partial).  New decode tokens always land above the
boundary, i.e. in the GPU partition.
"""
from __future__ import annotations

import math

# CPU token count at the measured KV lengths of the reference's DeepSeek-V2
# runtime (system/deepseek.py:127-130).  Kept identical: it is the calibrated
# policy that the drop-in must reproduce.
KV_LEN_GS_TABLE = {
    2048: 1280, 4096: 2560, 8192: 4096, 16384: 6144,
    32768: 12288, 65536: 32768, 131072: 65536,
}


def lookup_gs(total_kv: int) -> int:
    """Host (CPU) token count for a sequence of total_kv tokens: clamp to the
    table ends, else linear interpolation truncated to int
    (system/deepseek.py:132-142)."""
    keys = sorted(KV_LEN_GS_TABLE)
    if total_kv <= keys[0]:
        return KV_LEN_GS_TABLE[keys[0]]
    if total_kv >= keys[-1]:
        return KV_LEN_GS_TABLE[keys[-1]]
    lo = max(k for k in keys if k <= total_kv)
    hi = min(k for k in keys if k >= total_kv)
    if lo == hi:
        return KV_LEN_GS_TABLE[lo]
    g0, g1 = KV_LEN_GS_TABLE[lo], KV_LEN_GS_TABLE[hi]
    return int(g0 + (g1 - g0) * (total_kv - lo) / (hi - lo))


def clamp_gs(gs: int, total_kv: int, cache_gs: int | None = None) -> int:
    """Boundary actually used at decode time: never above the cache's fixed
    host capacity, within [0, total_kv] (system/deepseek.py:327-335)."""
    if cache_gs is not None:
        gs = min(gs, cache_gs)
    return max(0, min(gs, total_kv))


def gpu_share(total_kv: int, r: float) -> int:
    """GPU tokens at share r: the trailing floor(r * L) tokens."""
    if not 0.0 <= r <= 1.0:
        raise ValueError(f"share r={r} outside [0, 1]")
    return int(math.floor(r * total_kv))


def round_gs_to(gs: int, multiple: int = 64) -> int:
    """Round a CPU token count up to the page granularity
    (system/qwenoffload.py:1284-1286 rounds the chunk to 64)."""
    return ((gs + multiple - 1) // multiple) * multiple


def boundary_split(t: int, n_new: int, gs: int):
    """Place new tokens [t, t + n_new) on either side of boundary gs.

    Returns (host_slots, gpu_slots); each is (dst0, dst1, src0): destination
    slots [dst0, dst1) of that partition (GPU slots relative to gs) filled
    from source offset src0 of the new tokens.  Same arithmetic as
    InplaceKVCacheCompressed.append (system/deepseek.py:181-188).
    """
    if t < 0 or n_new < 0 or gs < 0:
        raise ValueError("negative position")
    h0, h1 = min(t, gs), min(t + n_new, gs)
    g0, g1 = max(t, gs) - gs, max(t + n_new, gs) - gs
    return (h0, h1, h0 - t), (g0, g1, g0 + gs - t)


def pages_for(n_tokens: int, page_size: int) -> int:
    return (n_tokens + page_size - 1) // page_size
