"""Drop-in replacements with the reference's GPU-side function signatures.

The reference's GPU partial helpers work on contiguous [N, S, D] K/V and the
(o, max, sum) triple.  These wrappers keep the signatures and run the gfx950
kernels.  A contiguous [N, S, D] buffer is the paged layout with Hkv = 1,
page_size = S and page n = row n, so no copy is made.

The triples returned here are the *equivalent* triple (o = normalised output,
max = lse, sum = 1): _pairwise_merge and the final o / sum give the same
results as with the reference's (unnormalised o, max, sum), because the merge
only uses max and sum through exp(max - M) * sum.
"""
from __future__ import annotations

import torch

from . import ops


def _dense_paging(n: int, s: int, device):
    page_table = torch.arange(n, dtype=torch.int32, device=device).view(n, 1)
    gpu_len = torch.full((n,), s, dtype=torch.int32, device=device)
    return page_table, gpu_len


def local_bmm_softmax(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float,
                      n_workgroups: int = 0):
    """_local_bmm_softmax (roofline/bench_resident_kv.py:150-157).

    q [N, G, Dk], k [N, S, Dk], v [N, S, Dv] bf16 contiguous on the GPU ->
    (o [N, G, Dv] fp32, max [N, G, 1] fp32, sum [N, G, 1] fp32), equivalent
    triple.  Dk == Dv == 128 for the GQA model entries (any multiple of 16 up
    to 256 has a kernel); Dk 192 / Dv 128 with G = 1 for the ds2 entry
    (roofline/bench_resident_kv.py:10).
    """
    N, G, Dk = q.shape
    S = k.shape[1]
    Dv = v.shape[2]
    if S == 0:
        return (torch.zeros((N, G, Dv), dtype=torch.float32, device=q.device),
                torch.full((N, G, 1), float("-inf"), dtype=torch.float32, device=q.device),
                torch.zeros((N, G, 1), dtype=torch.float32, device=q.device))
    pt, ln = _dense_paging(N, S, q.device)
    out, lse = ops.attn_decode_partial(q.contiguous(), k.contiguous().view(N, 1, S, Dk),
                                       v.contiguous().view(N, 1, S, Dv), pt, ln, scale, S,
                                       n_workgroups)
    return out, lse.unsqueeze(-1), torch.ones_like(lse).unsqueeze(-1)


def pairwise_merge(o1, m1, s1, o2, m2, s2):
    """_pairwise_merge (roofline/bench_resident_kv.py:141-148) on the GPU.

    Both triples unnormalised fp32 (o [..., Dv], m/s [..., 1]); returns the
    equivalent merged triple (o normalised, lse, 1)."""
    lse1 = torch.where(s1 > 0, m1 + torch.log(s1.clamp(min=1e-30)),
                       torch.full_like(m1, float("-inf")))
    o1n = torch.where(s1 > 0, o1 / s1.clamp(min=1e-30), torch.zeros_like(o1))
    out, lse = ops.lse_merge(o1n.contiguous(), lse1.contiguous(),
                             (o2.contiguous(), m2.contiguous(), s2.contiguous()),
                             ops.TRIPLE_UNNORM_F32, out_dtype=torch.float32)
    return out, lse.view(m1.shape), torch.ones_like(s1)


def resident_layer(q, k_buf, v_buf, new_k, new_v, scale):
    """_resident_layer (roofline/bench_resident_kv.py:261-271): write the new
    token into the last slot of the resident buffers and attend over all of
    them, in one launch.  k_buf [N, cap, Dk], v_buf [N, cap, Dv], new_k
    [N, 1, Dk], new_v [N, 1, Dv], q [N, G, Dk]; returns the equivalent triple
    like local_bmm_softmax."""
    N, cap, Dk = k_buf.shape
    Dv = v_buf.shape[2]
    if N <= 0 or cap <= 0:
        G = q.shape[1]
        return (torch.zeros((max(N, 0), G, Dv), dtype=torch.float32, device=q.device),
                torch.full((max(N, 0), G, 1), float("-inf"), dtype=torch.float32,
                           device=q.device),
                torch.zeros((max(N, 0), G, 1), dtype=torch.float32, device=q.device))
    pt, ln = _dense_paging(N, cap - 1, q.device)
    out, lse = ops.attn_decode_partial(
        q.contiguous(), k_buf.view(N, 1, cap, Dk), v_buf.view(N, 1, cap, Dv), pt, ln, scale,
        cap, k_new=new_k.contiguous().view(N, 1, 1, Dk),
        v_new=new_v.contiguous().view(N, 1, 1, Dv))
    return out, lse.unsqueeze(-1), torch.ones_like(lse).unsqueeze(-1)
