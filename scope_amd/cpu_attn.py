"""The reference CPU extension's Python surface on libwshost.so.

kernel/cpu_attn.cpp:1024-1054 binds fused_cpu_attn, fused_cpu_attn_fp32,
fused_cpu_attn_mla, fused_cpu_attn_mla_compressed, set_num_threads and
get_num_threads; the runtimes call them through an extension handle
(system/mixoffload.py:1333, system/qwenoffload.py:1085,1412,
system/deepseek.py:355, roofline/bench_resident_kv.py:129-133).  This module
has the same names, arguments and output shapes, so it can stand in for that
handle (`self._cpu_attn_ext = scope_amd.cpu_attn`), and runs this package's
host kernels (AVX-512 BF16, or fp32 FMAs for float32 inputs).

Outputs are the reference's own triples: max is the row's largest scaled
score q.k * scale, sum the sum of exp(q.k * scale - max), both fp32 and rounded
to bf16 only where the reference rounds them (fused_cpu_attn on bf16 inputs,
kernel/cpu_attn.cpp:631-634); out is normalised (fused_cpu_attn,
fused_cpu_attn_fp32) or not (fused_cpu_attn_mla, _mla_compressed) as there.
The host kernels carry exactly this running max and sum (log2-domain scores,
so sum is the same number), and return them through wh_attn_triple /
wh_mla_triple.

Differences from the reference: an empty sequence (S == 0) gives out = 0,
max = -inf, sum = 0 (the merge identity) where the reference divides by zero;
head widths are multiples of 16 up to 256, or 192 / 128, where the reference
takes any multiple of 16; at most 16 query heads share a KV row (G <= 16), and
absorbed MLA takes H a multiple of 16.
"""
from __future__ import annotations

import os

import torch

from . import host

_threads = 0  # 0: the OpenMP default


def set_num_threads(n: int) -> None:
    """Threads of the following calls (kernel/cpu_attn.cpp:1046-1050)."""
    global _threads
    _threads = max(1, int(n))


def get_num_threads() -> int:
    """Threads a call uses (kernel/cpu_attn.cpp:1051-1053)."""
    if _threads > 0:
        return _threads
    omp = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    return omp if omp > 0 else len(os.sched_getaffinity(0))


def _rows(t: torch.Tensor, name: str, width: int):
    """A [N, S, width] K or V view as paged-pool arguments: (tensor whose
    data_ptr is row 0, token stride of a row in tokens).  Rows may be strided
    (dims 0-1, as the reference honours them, kernel/cpu_attn.cpp:598-601);
    a layout a page cannot express is copied first."""
    if t.dim() != 3 or t.shape[2] != width:
        raise ValueError(f"{name} must be [N, S, {width}], got {tuple(t.shape)}")
    N, S, _ = t.shape
    if t.stride(2) != 1 or t.stride(1) != width or (N > 1 and t.stride(0) % width) or \
            (N > 1 and t.stride(0) < S * width):
        t = t.contiguous()
    row = t.stride(0) // width if N > 1 else max(S, 1)
    return t, max(row, 1)


def _triple(q, k, v, scale, normalize, threads):
    """fp32 (out [N, G, Dv], max [N, G], sum [N, G]) over dense rows k, v
    [N, S, D], out normalised when `normalize`."""
    if not q.is_contiguous():
        raise ValueError("q must be contiguous")
    N, G, Dk = q.shape
    Dv = v.shape[2]
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("k and v must have q's dtype")
    if k.shape[:2] != v.shape[:2] or k.shape[0] != N:
        raise ValueError(f"k {tuple(k.shape)} / v {tuple(v.shape)} do not match q "
                         f"{tuple(q.shape)}")
    S = k.shape[1]
    if N == 0 or S == 0:  # nothing to attend: the merge identity
        return (torch.zeros((N, G, Dv), dtype=torch.float32),
                torch.full((N, G), float("-inf"), dtype=torch.float32),
                torch.zeros((N, G), dtype=torch.float32))
    k, pk = _rows(k, "k", Dk)
    v, pv = _rows(v, "v", Dv)
    if pk != pv:  # one page size for both pools
        k, v = k.contiguous(), v.contiguous()
        pk = pv = max(S, 1)
    table = torch.arange(N, dtype=torch.int32).view(N, 1)
    lens = torch.full((N,), S, dtype=torch.int32)
    # row n of k / v is page n of a pool with one KV head and pk tokens per page
    try:
        kp = torch.as_strided(k, (N, 1, pk, Dk), (pk * Dk, pk * Dk, Dk, 1))
        vp = torch.as_strided(v, (N, 1, pk, Dv), (pk * Dv, pk * Dv, Dv, 1))
    except RuntimeError:  # the last row's page would run past the storage
        kp = k.contiguous().view(N, 1, S, Dk)
        vp = v.contiguous().view(N, 1, S, Dv)
    return host.attn_triple(q, kp, vp, table, lens, scale, normalize, threads)


def fused_cpu_attn(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float):
    """kernel/cpu_attn.cpp:572-636: q [B_kv, G, D], k / v [B_kv, S, D], bf16 or
    float32.  Returns the normalised out and (max, sum) [B_kv, G, 1], all bf16
    for bf16 inputs (each rounded from its fp32 value), float32 for float32
    inputs."""
    if q.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError("q must be float32 or bfloat16")
    out, m, s = _triple(q, k, v, scale, True, get_num_threads())
    m, s = m.unsqueeze(-1), s.unsqueeze(-1)
    if q.dtype == torch.bfloat16:
        return out.to(torch.bfloat16), m.to(torch.bfloat16), s.to(torch.bfloat16)
    return out, m, s


def fused_cpu_attn_fp32(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float):
    """kernel/cpu_attn.cpp:817-848: float32 inputs; normalised out, max, sum
    (float32)."""
    if q.dtype != torch.float32 or k.dtype != torch.float32 or v.dtype != torch.float32:
        raise ValueError("fused_cpu_attn_fp32 requires float32 inputs")
    out, m, s = _triple(q, k, v, scale, True, get_num_threads())
    return out, m.unsqueeze(-1), s.unsqueeze(-1)


def fused_cpu_attn_mla(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float):
    """kernel/cpu_attn.cpp:638-672: bf16 q [B_kv, G, Dk], k [B_kv, S, Dk],
    v [B_kv, S, Dv] (Dk may differ from Dv); unnormalised float32 out and
    float32 (max, sum)."""
    if q.dtype != torch.bfloat16:
        raise ValueError("fused_cpu_attn_mla requires bf16 inputs")
    out, m, s = _triple(q, k, v, scale, False, get_num_threads())
    return out, m.unsqueeze(-1), s.unsqueeze(-1)


def fused_cpu_attn_mla_compressed(q_proj: torch.Tensor, q_pe: torch.Tensor,
                                  c_kv: torch.Tensor, k_pe: torch.Tensor, scale: float):
    """kernel/cpu_attn.cpp:852-1022: q_proj [B*H, 512], q_pe [B*H, 64],
    c_kv [B, S, 512], k_pe [B, S, 64] bf16 (H = q rows / B, a multiple of 16
    here); unnormalised float32 out [B*H, 512], max [B*H], sum [B*H]."""
    if not (q_proj.is_contiguous() and c_kv.is_contiguous()):
        raise ValueError("q_proj and c_kv must be contiguous")
    B, S = c_kv.shape[0], c_kv.shape[1]
    if B == 0 or c_kv.dim() != 3 or c_kv.shape[2] != host.MLA_C or \
            tuple(k_pe.shape) != (B, S, host.MLA_PE):
        raise ValueError(f"c_kv must be [B, S, 512] and k_pe [B, S, 64], got "
                         f"{tuple(c_kv.shape)} / {tuple(k_pe.shape)}")
    if S == 0:  # nothing to attend: the merge identity
        rows = q_proj.shape[0]
        return (torch.zeros((rows, host.MLA_C), dtype=torch.float32),
                torch.full((rows,), float("-inf"), dtype=torch.float32),
                torch.zeros((rows,), dtype=torch.float32))
    return host.mla_triple_dense(q_proj.contiguous(), q_pe.contiguous(), c_kv,
                                 k_pe.contiguous(), [S] * B, scale, False, get_num_threads())
