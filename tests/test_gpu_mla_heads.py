"""Absorbed MLA with more than 16 heads on the GPU (DeepSeek-V2: 128 heads
over one shared 576-wide latent; the reference takes nH = q rows / B,
kernel/cpu_attn.cpp:860, system/deepseek.py:256-260): each 16-head group is a
plan sequence of its own over the same latent.  Against fp64, through the
one-launch partial, the split step with the native host partial and the
merge, the merge with the W_UV epilogue, and the paged two-sided cache.
"""
import numpy as np
import pytest
import torch

from oracle import attn_np as O
from scope_amd import host, ops
from scope_amd.paged import PagedMlaCache
from tests.gpu_pool import mla_pool
from tests.helpers import (LSE_ATOL, LSE_RTOL, OUT_ATOL, OUT_RTOL, assert_close, bf16_randn,
                           bits)

pytestmark = pytest.mark.gpu
DEV = "cuda"
PS = 64
SCALE = 192 ** -0.5


def _say(msg):
    print(msg, flush=True)


def _want(qn, qp, cs, pes, H):
    outs, lses = [], []
    for b in range(len(cs)):
        rows = slice(b * H, (b + 1) * H)
        o, l = O.mla_attention_fp64(bits(qn[rows]), bits(qp[rows]), bits(cs[b])[None],
                                    bits(pes[b])[None], SCALE)
        outs.append(o)
        lses.append(l)
    return np.concatenate(outs), np.concatenate(lses)


@pytest.mark.parametrize("H,wg", [(32, 0), (128, 0), (128, 5)])
def test_mla_partial_many_heads(H, wg):
    lens = [0, 70, 1500, 4097]
    _say(f"mla H={H} wg={wg} lens={lens}")
    lat, pt, gl, cs, pes = mla_pool(lens, PS, seed=81)
    B = len(lens)
    qn = bf16_randn((B * H, 512), 82, 0.5).to(DEV)
    qp = bf16_randn((B * H, 64), 83, 0.5).to(DEV)
    out, lse = ops.mla_decode_partial(qn, qp, lat, pt, gl, SCALE, max(lens), n_workgroups=wg)
    torch.cuda.synchronize()
    want, wl = _want(qn, qp, cs, pes, H)
    assert_close(out.cpu().numpy(), want, OUT_ATOL, OUT_RTOL, f"H={H} out")
    assert_close(lse.cpu().numpy(), wl, LSE_ATOL, LSE_RTOL, f"H={H} lse")


@pytest.mark.parametrize("scale", [-SCALE, 0.0])
def test_mla_128_heads_non_positive_scale(scale):
    """A negative scale (the kernel negates the queries and uses |scale|) and
    a zero scale (every score equal: uniform weights, lse = ln n), partial
    blocks and an empty sequence included, against fp64 at that scale."""
    H = 128
    lens = [0, 70, 1500, 4097]
    _say(f"mla H=128 scale={scale} lens={lens}")
    lat, pt, gl, cs, pes = mla_pool(lens, PS, seed=141)
    B = len(lens)
    qn = bf16_randn((B * H, 512), 142, 0.5).to(DEV)
    qp = bf16_randn((B * H, 64), 143, 0.5).to(DEV)
    out, lse = ops.mla_decode_partial(qn, qp, lat, pt, gl, scale, max(lens))
    torch.cuda.synchronize()
    outs, lses = [], []
    for b in range(B):
        rows = slice(b * H, (b + 1) * H)
        o, l = O.mla_attention_fp64(bits(qn[rows]), bits(qp[rows]), bits(cs[b])[None],
                                    bits(pes[b])[None], scale)
        outs.append(o)
        lses.append(l)
    want, wl = np.concatenate(outs), np.concatenate(lses)
    assert_close(out.cpu().numpy(), want, OUT_ATOL, OUT_RTOL, f"scale={scale} out")
    assert_close(lse.cpu().numpy(), wl, LSE_ATOL, LSE_RTOL, f"scale={scale} lse")
    if scale == 0.0:
        assert np.allclose(lse.cpu().numpy()[H:2 * H], np.log(70), atol=1e-5)


@pytest.mark.parametrize("wg", [3, 7])
def test_mla_128_heads_append_in_long_segments(wg):
    """Fused append with few workgroups: segments of hundreds of blocks, so
    the block holding the appended token (written into its page before the
    segment's loads) goes out late in the load ring, and each sequence's last
    block is partial.  Against fp64 over the old tokens plus the new one, and
    the appended latents bit-exact in their pages."""
    H = 128
    lens = [3000, 1500, 64]
    B = len(lens)
    _say(f"mla H=128 append, {wg} workgroups, lens={lens}")
    lat_all = [bf16_randn((L + 1, 576), 160 + b, 0.5) for b, L in enumerate(lens)]
    lat, pt, gl, _, _ = mla_pool([L + 1 for L in lens], PS, seed=170)
    for b, L in enumerate(lens):
        t = torch.arange(L, device=DEV)
        lat[pt[b, t // PS].long(), t % PS] = lat_all[b][:L].to(DEV)
    gl.copy_(torch.tensor(lens, dtype=torch.int32, device=DEV))
    qn = bf16_randn((B * H, 512), 171, 0.5).to(DEV)
    qp = bf16_randn((B * H, 64), 172, 0.5).to(DEV)
    new = torch.stack([x[-1] for x in lat_all]).to(DEV)[:, None]
    len_out = torch.zeros_like(gl)
    out, lse = ops.mla_append_decode_partial(qn, qp, new[..., :512], new[..., 512:], lat, pt, gl,
                                             len_out, SCALE, max(lens) + 1, n_workgroups=wg)
    torch.cuda.synchronize()
    want, wl = _want(qn, qp, [x[:, :512] for x in lat_all], [x[:, 512:] for x in lat_all], H)
    assert_close(out.cpu().numpy(), want, OUT_ATOL, OUT_RTOL, f"wg={wg} out")
    assert_close(lse.cpu().numpy(), wl, LSE_ATOL, LSE_RTOL, f"wg={wg} lse")
    assert len_out.cpu().tolist() == [L + 1 for L in lens]
    lb = bits(lat)
    for b, L in enumerate(lens):
        assert np.array_equal(lb[int(pt[b, L // PS]), L % PS], bits(lat_all[b][-1])), b


def test_mla_split_step_128_heads_with_host_partial_and_uv():
    H, Dout = 128, 128
    lens = [333, 2000, 64]
    host_lens = [128, 1000, 0]
    _say("mla H=128 split step + host partial + merge / merge with W_UV")
    B = len(lens)
    # GPU side holds tokens [host_len, L) of each sequence plus the new token
    lat_all = [bf16_randn((L + 1, 576), 90 + b, 0.5) for b, L in enumerate(lens)]
    gpu_parts = [x[h:L] for x, h, L in zip(lat_all, host_lens, lens)]
    lat, pt, gl, _, _ = mla_pool([x.shape[0] + 1 for x in gpu_parts], PS, seed=84)
    # overwrite the pool rows with the GPU tokens (mla_pool drew its own data)
    for b, x in enumerate(gpu_parts):
        n = x.shape[0]
        t = torch.arange(n, device=DEV)
        lat[pt[b, t // PS].long(), t % PS] = x.to(DEV)
    gl.copy_(torch.tensor([x.shape[0] for x in gpu_parts], dtype=torch.int32, device=DEV))
    qn = bf16_randn((B * H, 512), 85, 0.5).to(DEV)
    qp = bf16_randn((B * H, 64), 86, 0.5).to(DEV)
    new = torch.stack([x[-1] for x in lat_all]).to(DEV)[:, None]
    len_out = torch.zeros_like(gl)
    st = ops.mla_append_decode_split(qn, qp, new[..., :512], new[..., 512:], lat, pt, gl, len_out,
                                     SCALE, int(gl.max()) + 1)
    hc = torch.zeros((B, max(host_lens), 512), dtype=torch.bfloat16)
    hpe = torch.zeros((B, max(host_lens), 64), dtype=torch.bfloat16)
    for b, h in enumerate(host_lens):
        hc[b, :h] = lat_all[b][:h, :512]
        hpe[b, :h] = lat_all[b][:h, 512:]
    ho, hl = host.mla_partial_dense(qn.cpu(), qp.cpu(), hc, hpe, host_lens, SCALE, 8)
    hb = (ho.to(DEV), hl.to(DEV))
    out, lse = ops.merge_split(st, hb, ops.PARTIAL_LSE_F32, out_dtype=torch.float32)
    w_uv = bf16_randn((H, Dout, 512), 87, 0.05).to(DEV)
    out_v, latent, lse2 = ops.merge_split_uv(st, w_uv, hb, ops.PARTIAL_LSE_F32,
                                             want_latent=True, want_lse=True)
    torch.cuda.synchronize()
    cs = [x[:, :512] for x in lat_all]
    pes = [x[:, 512:] for x in lat_all]
    want, wl = _want(qn, qp, cs, pes, H)
    assert_close(out.cpu().numpy(), want, OUT_ATOL, OUT_RTOL, "merged out")
    assert_close(lse.cpu().numpy(), wl, LSE_ATOL, LSE_RTOL, "merged lse")
    assert_close(latent.float().cpu().numpy(), want, OUT_ATOL, OUT_RTOL, "uv latent")
    assert_close(lse2.cpu().numpy(), wl, LSE_ATOL, LSE_RTOL, "uv lse")
    w = O.as_f64(bits(w_uv))
    want_v = np.einsum("bhk,hvk->bhv", want.reshape(B, H, 512), w).reshape(B, H * Dout)
    assert_close(out_v.float().cpu().numpy(), want_v, OUT_ATOL, OUT_RTOL, "out_v")
    # the new latent was written once, bit-exact
    assert len_out.cpu().tolist() == [x.shape[0] + 1 for x in gpu_parts]
    lb = bits(lat)
    for b, x in enumerate(gpu_parts):
        n = x.shape[0]
        assert np.array_equal(lb[int(pt[b, n // PS]), n % PS], bits(lat_all[b][-1])), b


def test_paged_mla_cache_128_heads():
    H, layers = 128, 2
    lens = [700, 129]
    B = len(lens)
    _say("paged mla cache H=128")
    cache = PagedMlaCache(layers, B, max_tokens=1024, page_size=PS, device=DEV)
    lat = [[bf16_randn((L + 1, 576), 100 + 10 * l + b, 0.5) for b, L in enumerate(lens)]
           for l in range(layers)]
    for l in range(layers):
        for b, L in enumerate(lens):
            cache.load(l, b, lat[l][b][:L, :512], lat[l][b][:L, 512:], 128 if b == 0 else 64)
    for l in range(layers):
        qn = bf16_randn((B * H, 512), 120 + l, 0.5).to(DEV)
        qp = bf16_randn((B * H, 64), 130 + l, 0.5).to(DEV)
        new = torch.stack([x[-1] for x in lat[l]]).to(DEV)[:, None]
        out, lse = cache.step(l, qn, qp, new[..., :512], new[..., 512:], SCALE, host_threads=8,
                              return_lse=True)
        torch.cuda.synchronize()
        want, wl = _want(qn, qp, [x[:, :512] for x in lat[l]], [x[:, 512:] for x in lat[l]], H)
        assert_close(out.float().cpu().numpy(), want, OUT_ATOL, OUT_RTOL, f"layer {l}")
        assert_close(lse.cpu().numpy(), wl, LSE_ATOL, LSE_RTOL, f"layer {l} lse")


@pytest.mark.parametrize("append", [False, True])
def test_mla_128_heads_scores_climbing_past_the_first_block(append):
    """128 heads: the rope keys (k_pe, the 64 score-only columns) of every
    token after each sequence's first 32 are scaled up 1024-fold, so scores
    climb far above the first block's maximum (by a few hundred in log2
    units, where probabilities against that maximum would overflow fp32):
    the segment must run again against its true maximum.  The values (c_kv)
    keep their N(0, 0.5) scale.  Outputs and LSE against fp64, and the same
    run unscaled (no climb) alongside."""
    H = 128
    lens = [40, 700, 97]
    B = len(lens)
    _say(f"mla H=128 climbing scores append={append}")
    for factor in (1.0, 1024.0):
        lat_all = []
        for b, L in enumerate(lens):
            x = bf16_randn((L + 1, 576), 140 + b, 0.5).float()
            x[32:, 512:] *= factor
            lat_all.append(x.to(torch.bfloat16))
        n_gpu = [L + 1 if append else L for L in lens]
        lat, pt, gl, _, _ = mla_pool([n + 1 for n in n_gpu], PS, seed=145)
        for b, L in enumerate(lens):
            t = torch.arange(L, device=DEV)
            lat[pt[b, t // PS].long(), t % PS] = lat_all[b][:L].to(DEV)
        gl.copy_(torch.tensor(lens, dtype=torch.int32, device=DEV))
        qn = bf16_randn((B * H, 512), 146, 0.5).to(DEV)
        qp = bf16_randn((B * H, 64), 147, 0.5).to(DEV)
        if append:
            new = torch.stack([x[-1] for x in lat_all]).to(DEV)[:, None]
            len_out = torch.zeros_like(gl)
            out, lse = ops.mla_append_decode_partial(qn, qp, new[..., :512], new[..., 512:], lat,
                                                     pt, gl, len_out, SCALE, max(lens) + 1)
            cs = [x[:, :512] for x in lat_all]
            pes = [x[:, 512:] for x in lat_all]
        else:
            out, lse = ops.mla_decode_partial(qn, qp, lat, pt, gl, SCALE, max(lens))
            cs = [x[:L, :512] for x, L in zip(lat_all, lens)]
            pes = [x[:L, 512:] for x, L in zip(lat_all, lens)]
        torch.cuda.synchronize()
        want, wl = _want(qn, qp, cs, pes, H)
        assert np.isfinite(out.cpu().numpy()).all()
        assert_close(out.cpu().numpy(), want, OUT_ATOL, OUT_RTOL, f"factor {factor} out")
        assert_close(lse.cpu().numpy(), wl, LSE_ATOL, LSE_RTOL, f"factor {factor} lse")


def test_mla_128_heads_b4_every_row_against_the_c_restatement():
    """DeepSeek-V2 shape, 128 heads, B 4 at 8192 tokens per sequence plus the
    appended one, split step + merge: every row's output and LSE against
    the oracle's C restatement of fused_cpu_attn_mla_compressed over all
    tokens, and the appended latents bit-exact in their pages."""
    from oracle import port
    H, B, L = 128, 4, 8192
    _say("mla H=128 B4 L8192 against the C restatement")
    gen = torch.Generator(device=DEV).manual_seed(150)
    lat_all = [(torch.randn((L + 1, 576), generator=gen, device=DEV) * 0.5).to(torch.bfloat16)
               for _ in range(B)]
    lat, pt, gl, _, _ = mla_pool([L + 1] * B, PS, seed=151)
    for b in range(B):
        t = torch.arange(L, device=DEV)
        lat[pt[b, t // PS].long(), t % PS] = lat_all[b][:L]
    gl.fill_(L)
    qn = (torch.randn((B * H, 512), generator=gen, device=DEV) * 0.5).to(torch.bfloat16)
    qp = (torch.randn((B * H, 64), generator=gen, device=DEV) * 0.5).to(torch.bfloat16)
    new = torch.stack([x[-1] for x in lat_all])[:, None]
    len_out = torch.zeros_like(gl)
    st = ops.mla_append_decode_split(qn, qp, new[..., :512], new[..., 512:], lat, pt, gl, len_out,
                                     SCALE, L + 1)
    out, lse = ops.merge_split(st, None, out_dtype=torch.float32)
    torch.cuda.synchronize()
    full = np.stack([bits(x) for x in lat_all])
    po, pm, ps = port.cpu_attn_mla_compressed(bits(qn), bits(qp), full[:, :, :512],
                                              full[:, :, 512:], SCALE, n_threads=16)
    assert_close(out.cpu().numpy(), po / ps[:, None], OUT_ATOL, OUT_RTOL, "out vs C port")
    assert_close(lse.cpu().numpy(), pm + np.log(ps), LSE_ATOL, LSE_RTOL, "lse vs C port")
    assert len_out.cpu().tolist() == [L + 1] * B
    lb = bits(lat)
    for b in range(B):
        assert np.array_equal(lb[int(pt[b, L // PS]), L % PS], bits(lat_all[b][-1])), b


def test_mla_128_heads_b4_full_size_against_the_c_restatement():
    """DeepSeek-V2 shape at the size the step is timed on: 128 heads, B 4 at
    32768 tokens per sequence plus the appended one, split step + merge.
    Sequences 0 and 3 (every head) against the oracle's C restatement over
    all their tokens; all four appended latents bit-exact in their pages."""
    from oracle import port
    H, B, L = 128, 4, 32768
    _say("mla H=128 B4 L32768 against the C restatement (sequences 0, 3)")
    gen = torch.Generator(device=DEV).manual_seed(160)
    lat_all = [(torch.randn((L + 1, 576), generator=gen, device=DEV) * 0.5).to(torch.bfloat16)
               for _ in range(B)]
    lat, pt, gl, _, _ = mla_pool([L + 1] * B, PS, seed=161)
    for b in range(B):
        t = torch.arange(L, device=DEV)
        lat[pt[b, t // PS].long(), t % PS] = lat_all[b][:L]
    gl.fill_(L)
    qn = (torch.randn((B * H, 512), generator=gen, device=DEV) * 0.5).to(torch.bfloat16)
    qp = (torch.randn((B * H, 64), generator=gen, device=DEV) * 0.5).to(torch.bfloat16)
    new = torch.stack([x[-1] for x in lat_all])[:, None]
    len_out = torch.zeros_like(gl)
    st = ops.mla_append_decode_split(qn, qp, new[..., :512], new[..., 512:], lat, pt, gl, len_out,
                                     SCALE, L + 1)
    out, lse = ops.merge_split(st, None, out_dtype=torch.float32)
    torch.cuda.synchronize()
    out, lse = out.cpu().numpy(), lse.cpu().numpy()
    assert len_out.cpu().tolist() == [L + 1] * B
    lb = bits(lat)
    for b in range(B):
        assert np.array_equal(lb[int(pt[b, L // PS]), L % PS], bits(lat_all[b][-1])), b
    for b in (0, 3):
        rows = slice(b * H, (b + 1) * H)
        full = bits(lat_all[b])[None]
        po, pm, ps = port.cpu_attn_mla_compressed(bits(qn[rows]), bits(qp[rows]),
                                                  full[:, :, :512], full[:, :, 512:], SCALE,
                                                  n_threads=16)
        assert_close(out[rows], po / ps[:, None], OUT_ATOL, OUT_RTOL, f"out b={b} vs C port")
        assert_close(lse[rows], pm + np.log(ps), LSE_ATOL, LSE_RTOL, f"lse b={b} vs C port")
