"""Full-size parity through properties that hold at any size.

At the benchmark shapes the merged attention must not depend on where the
partition boundary lies: the GPU partial over the trailing floor(r L) tokens
merged with the host partial over the rest is the same softmax for every r.
Each case builds the partitioned cache at three shares (data drawn on the
GPU for speed), runs the fused append + split step, the native host partial
and the merge, and checks (a) the shares agree with each other, outputs and
merged LSE, (b) every row's output and LSE against the oracle's C restatement
of the reference CPU kernel over the whole sequence, and sampled rows against
fp64 attention.
"""
import numpy as np
import pytest
import torch

from helpers import LSE_ATOL, LSE_RTOL, OUT_ATOL, OUT_RTOL, assert_close, bits
from oracle import attn_np as O
from oracle import port
from scope_amd import host, ops
from scope_amd.cache import GqaGpuPartition, MlaGpuPartition

pytestmark = pytest.mark.gpu
DEV = "cuda"
PS = 64


def _say(msg):
    print(msg, flush=True)


def _randn_bf16(shape, gen, sigma=1.0):
    return (torch.randn(shape, generator=gen, device=DEV) * sigma).to(torch.bfloat16)


def test_mixtral_b16_full_size_share_invariance():
    """Mixtral layer, B 16, 32 q / 8 KV heads, L ~ U[1024, 32768] (seed 2000)."""
    B, Hkv, G, D = 16, 8, 4, 128
    lens = np.random.default_rng(2000).integers(1024, 32769, B)
    scale = D ** -0.5
    gen = torch.Generator(device=DEV).manual_seed(11)
    # token L of each sequence is the step's appended token
    k = [_randn_bf16((Hkv, int(L) + 1, D), gen) for L in lens]
    v = [_randn_bf16((Hkv, int(L) + 1, D), gen) for L in lens]
    q = _randn_bf16((B, Hkv * G, D), gen)
    k_new = torch.stack([x[:, -1:] for x in k])
    v_new = torch.stack([x[:, -1:] for x in v])
    outs, lses = {}, {}
    for r in (0.25, 0.5, 0.75):
        g = [int(np.floor(r * int(L))) for L in lens]
        h = [int(L) - gg for L, gg in zip(lens, g)]
        _say(f"full-size mixtral r={r}: {sum(g)} GPU tokens, {sum(h)} host tokens")
        part = GqaGpuPartition(1, B, Hkv, D, max_tokens=max(g) + PS + 1, device=DEV)
        for b in range(B):
            part.load_sequence(0, b, k[b][:, h[b]:int(lens[b])], v[b][:, h[b]:int(lens[b])])
        hk = torch.zeros((B * Hkv, max(h), D), dtype=torch.bfloat16)
        hv = torch.zeros_like(hk)
        for b in range(B):
            hk[b * Hkv:(b + 1) * Hkv, :h[b]] = k[b][:, :h[b]].cpu()
            hv[b * Hkv:(b + 1) * Hkv, :h[b]] = v[b][:, :h[b]].cpu()
        st = part.step_split(0, q, k_new, v_new, scale)
        ho, hl = host.gqa_partial_dense(q.cpu(), hk, hv, h, scale, 16)
        out, lse = ops.merge_split(st, (ho.to(DEV), hl.to(DEV)), ops.PARTIAL_LSE_F32,
                                   out_dtype=torch.float32)
        torch.cuda.synchronize()
        outs[r] = out.cpu().numpy().reshape(B, Hkv, G, D)
        lses[r] = lse.cpu().numpy().reshape(B, Hkv, G)
        assert part.lens[0].tolist() == [gg + 1 for gg in g]
    # (a) the boundary does not change the attention
    for r in (0.5, 0.75):
        assert_close(outs[r], outs[0.25], 5e-3, 5e-3, f"share {r} vs 0.25")
        assert_close(lses[r], lses[0.25], LSE_ATOL, LSE_RTOL, f"share {r} vs 0.25 lse")
    # (b) every row against the oracle's C restatement of the reference CPU
    # kernel (pinned to fp64), sampled rows against fp64, over the whole
    # sequence
    qb = bits(q).reshape(B, Hkv, G, D)
    for b in range(B):
        po, pm, ps = port.cpu_attn(qb[b], bits(k[b]), bits(v[b]), scale, normalize=True,
                                   n_threads=16)
        pl = (pm + np.log(ps))[..., 0]
        for r in outs:
            assert_close(outs[r][b], po, OUT_ATOL, OUT_RTOL, f"r={r} b={b} vs C port")
            assert_close(lses[r][b], pl, LSE_ATOL, LSE_RTOL, f"r={r} b={b} lse vs C port")
    for b in (0, 5, 13):
        for kvh in (0, 7):
            want, wl = O.gqa_attention_fp64(qb[b, kvh][None], bits(k[b][kvh:kvh + 1]),
                                            bits(v[b][kvh:kvh + 1]), scale)
            for r in outs:
                what = f"r={r} b={b} kvh={kvh}"
                assert_close(outs[r][b, kvh], want[0], OUT_ATOL, OUT_RTOL, what)
                assert_close(lses[r][b, kvh], wl[0], LSE_ATOL, LSE_RTOL, what + " lse")


def test_dsv2lite_mla_b8_full_size_share_invariance():
    """DeepSeek-V2-Lite absorbed MLA, B 8, 16 heads, L 16384."""
    B, H, L = 8, 16, 16384
    scale = 192 ** -0.5
    gen = torch.Generator(device=DEV).manual_seed(12)
    lat = [_randn_bf16((L + 1, 576), gen, 0.5) for _ in range(B)]
    qn = _randn_bf16((B * H, 512), gen, 0.5)
    qp = _randn_bf16((B * H, 64), gen, 0.5)
    new = torch.stack([x[-1:] for x in lat])
    outs, lses = {}, {}
    for r in (0.25, 0.5, 1.0):
        g = int(np.floor(r * L))
        h = L - g
        _say(f"full-size mla r={r}: {B * g} GPU tokens, {B * h} host tokens")
        part = MlaGpuPartition(1, B, max_tokens=g + PS + 1, device=DEV)
        for b in range(B):
            if g:
                part.load_sequence(0, b, lat[b][h:L, :512].contiguous(),
                                   lat[b][h:L, 512:].contiguous())
        st = part.step_split(0, qn, qp, new[..., :512], new[..., 512:], scale)
        if h:
            hc = torch.stack([x[:h, :512].cpu() for x in lat]).contiguous()
            hpe = torch.stack([x[:h, 512:].cpu() for x in lat]).contiguous()
            ho, hl = host.mla_partial_dense(qn.cpu(), qp.cpu(), hc, hpe, [h] * B, scale, 16)
            out, lse = ops.merge_split(st, (ho.to(DEV), hl.to(DEV)), ops.PARTIAL_LSE_F32,
                                       out_dtype=torch.float32)
        else:
            out, lse = ops.merge_split(st, None, out_dtype=torch.float32)
        torch.cuda.synchronize()
        outs[r] = out.cpu().numpy()
        lses[r] = lse.cpu().numpy()
    for r in (0.5, 1.0):
        assert_close(outs[r], outs[0.25], 5e-3, 5e-3, f"share {r} vs 0.25")
        assert_close(lses[r], lses[0.25], LSE_ATOL, LSE_RTOL, f"share {r} vs 0.25 lse")
    # every sequence against the C restatement of fused_cpu_attn_mla_compressed
    # over all L + 1 tokens (unnormalised out, max, sum -> out / sum, lse)
    full = np.stack([bits(x) for x in lat])
    po, pm, ps = port.cpu_attn_mla_compressed(bits(qn), bits(qp), full[:, :, :512],
                                              full[:, :, 512:], scale, n_threads=16)
    pl = pm + np.log(ps)
    po = po / ps[:, None]
    for r in outs:
        for b in range(B):
            rows = slice(b * H, (b + 1) * H)
            assert_close(outs[r][rows], po[rows], OUT_ATOL, OUT_RTOL, f"r={r} b={b} vs C port")
            assert_close(lses[r][rows], pl[rows], LSE_ATOL, LSE_RTOL,
                         f"r={r} b={b} lse vs C port")
    for b in (0, 7):
        rows = slice(b * H, (b + 1) * H)
        want, wl = O.mla_attention_fp64(bits(qn[rows]), bits(qp[rows]), full[b:b + 1, :, :512],
                                        full[b:b + 1, :, 512:], scale)
        for r in outs:
            assert_close(outs[r][rows], want, OUT_ATOL, OUT_RTOL, f"r={r} b={b}")
            assert_close(lses[r][rows], wl, LSE_ATOL, LSE_RTOL, f"r={r} b={b} lse")


@pytest.mark.parametrize("L", [32768, 131072])
def test_dsv2lite_mla_b8_length_sweep_all_in_hbm(L):
    """The MLA length sweep's shapes (16 heads, B=8, r = 1): the fused append
    + split step + merge over L tokens per sequence plus the appended one.
    Every head of sequences 0 and 7 against the C restatement over all their
    tokens; every appended latent bit-exact in its page."""
    from gpu_pool import page_layout
    H, B = 16, 8
    _say(f"mla B8 H16 L={L} r=1 against the C restatement (sequences 0, 7)")
    gen = torch.Generator(device=DEV).manual_seed(170 + L % 97)
    table, num_pages = page_layout([L + 1] * B, PS, seed=171)
    pt = torch.from_numpy(table).to(DEV)
    lat = torch.zeros((num_pages, PS, 576), dtype=torch.bfloat16, device=DEV)
    t = torch.arange(L, device=DEV)
    keep, new = {}, []
    for b in range(B):
        x = _randn_bf16((L + 1, 576), gen, 0.5)
        lat[pt[b, t // PS].long(), t % PS] = x[:L]
        new.append(x[-1])
        if b in (0, 7):
            keep[b] = bits(x)
        del x
    gl = torch.full((B,), L, dtype=torch.int32, device=DEV)
    qn = _randn_bf16((B * H, 512), gen, 0.5)
    qp = _randn_bf16((B * H, 64), gen, 0.5)
    new = torch.stack(new)[:, None]
    len_out = torch.zeros_like(gl)
    scale = 192 ** -0.5
    st = ops.mla_append_decode_split(qn, qp, new[..., :512], new[..., 512:], lat, pt, gl,
                                     len_out, scale, L + 1)
    out, lse = ops.merge_split(st, None, out_dtype=torch.float32)
    torch.cuda.synchronize()
    out, lse = out.cpu().numpy(), lse.cpu().numpy()
    assert len_out.cpu().tolist() == [L + 1] * B
    slots = lat[pt[:, L // PS].long(), L % PS]
    assert torch.equal(slots, new[:, 0]), "appended latents"
    for b, full in keep.items():
        rows = slice(b * H, (b + 1) * H)
        po, pm, ps = port.cpu_attn_mla_compressed(bits(qn[rows]), bits(qp[rows]),
                                                  full[None, :, :512], full[None, :, 512:],
                                                  scale, n_threads=16)
        assert_close(out[rows], po / ps[:, None], OUT_ATOL, OUT_RTOL, f"L={L} out b={b}")
        assert_close(lse[rows], pm + np.log(ps), LSE_ATOL, LSE_RTOL, f"L={L} lse b={b}")
