"""Parity at the benchmark configurations that the other GPU tests cover only
at smaller sizes.

Qwen3-30B-A3B large-KV sweep: batch 4, 32 q / 4 KV heads, head_dim 128,
r = 1, 8k..128k tokens per sequence, through the split step (fused append +
partial) and the split merge with no host partial.  Every (sequence, q head)
row is checked against the oracle's C restatement of the reference CPU kernel
(pinned to fp64 in tests/test_oracle.py), two rows against fp64 attention, and
the appended token bit for bit in its page.

DeepSeek-V2-Lite 27-layer decode loop, reduced to 3 layers x 2 steps: batch
32 with lognormal lengths (median 4096, sigma 1, clipped to [256, 65536],
seed 2005, the benchmark's batch, whose longest sequence has 65536 tokens),
through PagedMlaCache with the native host partial over the host pages, at
GPU shares 0.1, 0.5 and 0.9.  Every sequence of every layer and step is
checked against fp64 attention over all of its tokens, and the appended
latents bit for bit in their pages.
"""
import math

import numpy as np
import pytest
import torch

from helpers import LSE_ATOL, LSE_RTOL, OUT_ATOL, OUT_RTOL, assert_close, bits
from oracle import attn_np as O
from oracle import port
from scope_amd import ops
from scope_amd.cache import GqaGpuPartition
from scope_amd.paged import PagedMlaCache
from bench import lognormal_lens  # the benchmark's own batch

pytestmark = pytest.mark.gpu
DEV = "cuda"
PS = 64
THREADS = 16


def _say(msg):
    print(msg, flush=True)


def _randn_bf16(shape, gen, sigma=1.0):
    return (torch.randn(shape, generator=gen, device=DEV) * sigma).to(torch.bfloat16)


@pytest.mark.parametrize("L", [8192, 32768, 65536, 131072])
def test_qwen3_b4_full_gpu_share(L):
    B, Hkv, G, D = 4, 4, 8, 128
    scale = D ** -0.5
    _say(f"qwen3 B{B} r=1 L={L}: split step + merge, all rows vs the C port")
    gen = torch.Generator(device=DEV).manual_seed(4000 + L // 1024)
    k = _randn_bf16((B, Hkv, L + 1, D), gen)  # token L is the step's appended one
    v = _randn_bf16((B, Hkv, L + 1, D), gen)
    q = _randn_bf16((B, Hkv * G, D), gen)
    part = GqaGpuPartition(1, B, Hkv, D, max_tokens=L + 1, device=DEV)
    for b in range(B):
        part.load_sequence(0, b, k[b, :, :L], v[b, :, :L])
    st = part.step_split(0, q, k[:, :, L:L + 1].contiguous(), v[:, :, L:L + 1].contiguous(),
                         scale)
    out, lse = ops.merge_split(st, None, out_dtype=torch.float32)
    out16, _ = ops.merge_split(st, None, out_dtype=torch.bfloat16, want_lse=False)
    torch.cuda.synchronize()
    assert part.lens[0].tolist() == [L + 1] * B
    assert part.len_dev(0).cpu().tolist() == [L + 1] * B

    # the appended token, bit for bit, in its page slot
    pid = [int(part.host_table[b, L // PS]) for b in range(B)]
    off = L % PS
    for b in range(B):
        assert np.array_equal(bits(part.k[0][pid[b], :, off]), bits(k[b, :, L])), b
        assert np.array_equal(bits(part.v[0][pid[b], :, off]), bits(v[b, :, L])), b

    got = out.cpu().numpy().reshape(B, Hkv, G, D)
    got_l = lse.cpu().numpy().reshape(B, Hkv, G)
    got16 = out16.float().cpu().numpy().reshape(B, Hkv, G, D)
    qb = bits(q).reshape(B, Hkv, G, D)
    kb, vb = bits(k), bits(v)
    for b in range(B):
        po, pm, psum = port.cpu_attn(qb[b], kb[b], vb[b], scale, normalize=True,
                                     n_threads=THREADS)
        assert_close(got[b], po, OUT_ATOL, OUT_RTOL, f"L={L} b={b} out vs C port")
        assert_close(got16[b], po, OUT_ATOL, OUT_RTOL, f"L={L} b={b} bf16 out vs C port")
        assert_close(got_l[b], (pm + np.log(psum))[..., 0], LSE_ATOL, LSE_RTOL,
                     f"L={L} b={b} lse vs C port")
    for b, kvh in ((0, 0), (B - 1, Hkv - 1)):
        want, wl = O.gqa_attention_fp64(qb[b, kvh][None], kb[b, kvh][None], vb[b, kvh][None],
                                        scale)
        assert_close(got[b, kvh], want[0], OUT_ATOL, OUT_RTOL, f"L={L} b={b} kvh={kvh} fp64")
        assert_close(got_l[b, kvh], wl[0], LSE_ATOL, LSE_RTOL, f"L={L} b={b} kvh={kvh} lse")


# ---------------------------------------------------------------------------
# DeepSeek-V2-Lite decode loop over a two-sided paged latent cache

MLA_LAYERS, MLA_STEPS, MLA_H = 3, 2, 16
MLA_SCALE = 192 ** -0.5


@pytest.fixture(scope="module")
def dsv2_batch():
    """Latents of every layer (tokens L_b + 2: two decode steps), queries of
    every (step, layer), and the fp64 attention of every (step, layer) over
    each sequence's tokens so far (it does not depend on the share)."""
    B, H = 32, MLA_H
    lens = [int(x) for x in lognormal_lens(B, 2005)]
    assert max(lens) == 65536
    gen = torch.Generator(device=DEV).manual_seed(5005)
    lat = [[_randn_bf16((L + MLA_STEPS, 576), gen, 0.5).cpu() for L in lens]
           for _ in range(MLA_LAYERS)]
    qs = [[(_randn_bf16((B * H, 512), gen, 0.5), _randn_bf16((B * H, 64), gen, 0.5))
           for _ in range(MLA_LAYERS)] for _ in range(MLA_STEPS)]
    _say(f"dsv2-lite B{B}: {sum(lens)} tokens, fp64 references of "
         f"{MLA_STEPS} steps x {MLA_LAYERS} layers")
    ref = {}
    for l in range(MLA_LAYERS):
        lat_bits = [bits(x) for x in lat[l]]
        for s in range(MLA_STEPS):
            qn, qp = bits(qs[s][l][0]), bits(qs[s][l][1])
            o_all = np.empty((B * H, 512))
            l_all = np.empty((B * H,))
            for b, L in enumerate(lens):
                full = lat_bits[b][:L + 1 + s]
                rows = slice(b * H, (b + 1) * H)
                o_all[rows], l_all[rows] = O.mla_attention_fp64(
                    qn[rows], qp[rows], full[None, :, :512], full[None, :, 512:], MLA_SCALE)
            ref[(s, l)] = (o_all, l_all)
    return lens, lat, qs, ref


@pytest.mark.parametrize("r", [0.1, 0.3, 0.5, 0.7, 0.9])
def test_dsv2lite_b32_lognormal_decode_loop(dsv2_batch, r):
    lens, lat, qs, ref = dsv2_batch
    B, H = len(lens), MLA_H
    host_tok = [((L - int(math.floor(r * L))) // PS) * PS for L in lens]
    gpu_pages = sum(-(-(L + MLA_STEPS - h) // PS) for L, h in zip(lens, host_tok)) + 4
    host_pages = sum(h // PS for h in host_tok) + 4
    _say(f"dsv2-lite B{B} r={r}: {sum(L - h for L, h in zip(lens, host_tok))} GPU tokens, "
         f"{sum(host_tok)} host tokens, {MLA_LAYERS} layers x {MLA_STEPS} steps")
    cache = PagedMlaCache(MLA_LAYERS, B, max_tokens=max(lens) + MLA_STEPS, page_size=PS,
                          host_pages=host_pages, gpu_pages=gpu_pages, device=DEV)
    for l in range(MLA_LAYERS):
        for b, L in enumerate(lens):
            x = lat[l][b]
            cache.load(l, b, x[:L, :512], x[:L, 512:], host_tok[b])
    for s in range(MLA_STEPS):
        for l in range(MLA_LAYERS):
            new = torch.stack([lat[l][b][L + s] for b, L in enumerate(lens)]).to(DEV)
            qn, qp = qs[s][l]
            out, lse = cache.step(l, qn, qp, new[:, None, :512], new[:, None, 512:], MLA_SCALE,
                                  host_threads=THREADS, return_lse=True)
            torch.cuda.synchronize()
            want, wl = ref[(s, l)]
            got = out.float().cpu().numpy()
            got_l = lse.cpu().numpy()
            for b in range(B):
                rows = slice(b * H, (b + 1) * H)
                what = f"r={r} step={s} layer={l} b={b} (L={lens[b]}, host {host_tok[b]})"
                assert_close(got[rows], want[rows], OUT_ATOL, OUT_RTOL, what)
                assert_close(got_l[rows], wl[rows], LSE_ATOL, LSE_RTOL, what + " lse")
    # the appended latents, bit for bit, in their GPU pages
    g = cache.gpu
    for l in range(MLA_LAYERS):
        for b, L in enumerate(lens):
            for s in range(MLA_STEPS):
                t = L + s - host_tok[b]  # position inside the GPU side
                pid = int(g.host_table[b, t // PS])
                assert np.array_equal(bits(g.latent[l][pid, t % PS]), bits(lat[l][b][L + s])), \
                    (r, l, b, s)
    assert [cache.seq_len(b) for b in range(B)] == [L + MLA_STEPS for L in lens]
