"""Builders of seeded paged pools for the GPU tests (written with plain torch
indexing, independent of the append kernel)."""
from __future__ import annotations

import numpy as np
import torch

from tests.helpers import bf16_randn


def page_layout(lens, page_size, seed, spare=2):
    """Random physical page ids for sequences of the given lengths.
    Returns (page_table np [B, max_pages] int32, num_pages)."""
    rng = np.random.default_rng(seed)
    need = [(int(L) + page_size - 1) // page_size for L in lens]
    max_pages = max(1, max(need) if need else 1)
    num_pages = sum(need) + spare
    perm = rng.permutation(num_pages)
    table = np.full((len(lens), max_pages), -1, np.int32)
    k = 0
    for b, n in enumerate(need):
        table[b, :n] = perm[k:k + n]
        k += n
    return table, num_pages


def scatter_tokens(pages, table_dev, b, x, page_size, head_axis=True):
    """pages[page_table[b, t // PS], (:), t % PS] = x[(:), t] for all t."""
    L = x.shape[1] if head_axis else x.shape[0]
    if L == 0:
        return
    t = torch.arange(L, device=pages.device)
    pid = table_dev[b, (t // page_size)].long()
    off = t % page_size
    if head_axis:  # x [Hkv, L, D] -> pages [P, Hkv, PS, D]
        pages[pid, :, off, :] = x.to(pages.device).permute(1, 0, 2)
    else:  # x [L, W] -> pages [P, PS, W]
        pages[pid, off, :] = x.to(pages.device)


def gqa_pool(lens, Hkv, D, page_size, seed, device="cuda", sigma=1.0):
    """Paged GQA K/V for sequences of `lens` tokens; returns
    (k_pages, v_pages, page_table, gpu_len, ks, vs) with ks[b], vs[b] the CPU
    bf16 tensors [Hkv, L_b, D]."""
    table, num_pages = page_layout(lens, page_size, seed)
    k_pages = torch.zeros((num_pages, Hkv, page_size, D), dtype=torch.bfloat16, device=device)
    v_pages = torch.zeros_like(k_pages)
    tdev = torch.from_numpy(table).to(device)
    ks, vs = [], []
    for b, L in enumerate(lens):
        k = bf16_randn((Hkv, int(L), D), seed * 1000 + 2 * b + 1, sigma)
        v = bf16_randn((Hkv, int(L), D), seed * 1000 + 2 * b + 2, sigma)
        scatter_tokens(k_pages, tdev, b, k, page_size)
        scatter_tokens(v_pages, tdev, b, v, page_size)
        ks.append(k)
        vs.append(v)
    gpu_len = torch.tensor([int(L) for L in lens], dtype=torch.int32, device=device)
    return k_pages, v_pages, tdev, gpu_len, ks, vs


def mla_pool(lens, page_size, seed, device="cuda", sigma=0.5):
    """Paged 576-wide latents; returns (latent_pages, page_table, gpu_len,
    cs [L,512], pes [L,64]) per sequence."""
    table, num_pages = page_layout(lens, page_size, seed)
    lat = torch.zeros((num_pages, page_size, 576), dtype=torch.bfloat16, device=device)
    tdev = torch.from_numpy(table).to(device)
    cs, pes = [], []
    for b, L in enumerate(lens):
        c = bf16_randn((int(L), 512), seed * 1000 + 2 * b + 1, sigma)
        pe = bf16_randn((int(L), 64), seed * 1000 + 2 * b + 2, sigma)
        scatter_tokens(lat, tdev, b, torch.cat([c, pe], 1), page_size, head_axis=False)
        cs.append(c)
        pes.append(pe)
    gpu_len = torch.tensor([int(L) for L in lens], dtype=torch.int32, device=device)
    return lat, tdev, gpu_len, cs, pes
