"""Decode steps of the two-sided paged caches (scope_amd/paged.py) on the
GPU, with the native host partial, before and after moving the boundary in
both directions, against fp64 attention over the whole sequence."""
import numpy as np
import pytest
import torch

from helpers import OUT_ATOL, OUT_RTOL, assert_close, bf16_randn, bits
from oracle import attn_np as O
from scope_amd.paged import PagedKVCache, PagedMlaCache

pytestmark = pytest.mark.gpu
DEV = "cuda"
PS = 64


def _say(msg):
    print(msg, flush=True)


def test_paged_mla_steps_across_boundary_moves():
    B, H, layers = 3, 16, 2
    lens = [700, 130, 64]
    hosts = [256, 64, 0]
    scale = 192 ** -0.5
    steps = 3
    total = max(lens) + steps
    cache = PagedMlaCache(layers, B, max_tokens=total + PS, page_size=PS, device=DEV)
    lat = {}
    for layer in range(layers):
        for b, (L, h) in enumerate(zip(lens, hosts)):
            lat[layer, b] = torch.cat([bf16_randn((L + steps, 512), 10 * layer + b, 0.5),
                                       bf16_randn((L + steps, 64), 10 * layer + b + 5, 0.5)],
                                      dim=1)
            x = lat[layer, b]
            cache.load(layer, b, x[:L, :512].contiguous(), x[:L, 512:].contiguous(), h)
    shares = [None, 0.2, 0.9]   # start, share down (GPU -> host), share up
    for s, share in enumerate(shares):
        if share is not None:
            cache.set_share(share)
        _say(f"paged mla step {s} share={share} host={[cache.host_tokens(b) for b in range(B)]}")
        for layer in range(layers):
            pos = [lens[b] + s for b in range(B)]
            new = torch.stack([lat[layer, b][pos[b]] for b in range(B)]).view(B, 1, 576)
            qn = bf16_randn((B * H, 512), 900 + 10 * s + layer, 0.5)
            qp = bf16_randn((B * H, 64), 950 + 10 * s + layer, 0.5)
            out = cache.step(layer, qn.to(DEV), qp.to(DEV), new[..., :512].contiguous().to(DEV),
                             new[..., 512:].contiguous().to(DEV), scale, host_threads=3)
            torch.cuda.synchronize()
            got = out.float().cpu().numpy()
            for b in range(B):
                full = bits(lat[layer, b][:pos[b] + 1])
                hh = slice(b * H, (b + 1) * H)
                want, _ = O.mla_attention_fp64(bits(qn[hh]), bits(qp[hh]), full[None, :, :512],
                                               full[None, :, 512:], scale)
                assert_close(got[hh], want, OUT_ATOL, OUT_RTOL, f"step {s} layer {layer} b={b}")
    for b in range(B):
        assert cache.seq_len(b) == lens[b] + steps


def test_paged_gqa_steps_across_boundary_moves():
    B, Hkv, G, D, layers = 2, 8, 4, 128, 1
    lens = [900, 200]
    hosts = [448, 128]
    scale = D ** -0.5
    steps = 3
    cache = PagedKVCache(layers, B, Hkv, D, max_tokens=max(lens) + steps + PS, page_size=PS,
                         device=DEV)
    ks = [bf16_randn((Hkv, L + steps, D), 300 + b) for b, L in enumerate(lens)]
    vs = [bf16_randn((Hkv, L + steps, D), 400 + b) for b, L in enumerate(lens)]
    for b, (L, h) in enumerate(zip(lens, hosts)):
        cache.load(0, b, ks[b][:, :L].contiguous(), vs[b][:, :L].contiguous(), h)
    for s, share in enumerate([None, 0.1, 0.95]):
        if share is not None:
            cache.set_share(share)
        _say(f"paged gqa step {s} share={share} host={[cache.host_tokens(b) for b in range(B)]}")
        pos = [lens[b] + s for b in range(B)]
        k_new = torch.stack([ks[b][:, pos[b]:pos[b] + 1] for b in range(B)]).to(DEV)
        v_new = torch.stack([vs[b][:, pos[b]:pos[b] + 1] for b in range(B)]).to(DEV)
        q = bf16_randn((B, Hkv * G, D), 500 + s)
        out = cache.step(0, q.to(DEV), k_new, v_new, scale, host_threads=3)
        torch.cuda.synchronize()
        got = out.float().cpu().numpy()
        qb = bits(q).reshape(B, Hkv, G, D)
        for b in range(B):
            want, _ = O.gqa_attention_fp64(qb[b], bits(ks[b][:, :pos[b] + 1]),
                                           bits(vs[b][:, :pos[b] + 1]), scale)
            assert_close(got[b].reshape(Hkv, G, D), want, OUT_ATOL, OUT_RTOL, f"step {s} b={b}")
