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
