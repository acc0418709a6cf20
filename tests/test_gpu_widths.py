"""GPU parity of the GQA decode path at head widths other than 128 (every
multiple of 16 up to 256; the reference's GPU partial is a torch bmm of any
width, roofline/bench_resident_kv.py:150-157, and its CPU kernel takes any
multiple of 16, kernel/cpu_attn.cpp:583), through the C-ABI, against fp64
attention and the oracle's C restatement of the reference CPU kernel.

Bar: appends bit-exact; outputs within 2e-2 abs/rel; fp32 LSE within 1e-3.
"""
import numpy as np
import pytest
import torch

from oracle import attn_np as O
from oracle import port
from scope_amd import ops
from scope_amd.cache import PartitionedKVCache
from scope_amd.decode import NATIVE, partitioned_gqa_decode
from scope_amd.partition import gpu_share
from tests.gpu_pool import gqa_pool
from tests.helpers import (LSE_ATOL, LSE_RTOL, OUT_ATOL, OUT_RTOL, assert_close,
                           bf16_randn, bits)

pytestmark = pytest.mark.gpu
DEV = "cuda"
WIDTHS = [64, 256]
# widths whose kernels take the group size at run time; 16-column key tails
# (48, 80, 112, ...) and value rows split over fewer than 16 lanes (80: 10
# lanes of 8 columns, 176: 11 of 16)
OTHER_WIDTHS = [16, 32, 48, 80, 96, 112, 144, 160, 176, 192, 208, 224, 240]


def _say(msg):
    print(msg, flush=True)


def _check_rows(out, lse, q, ks, vs, lens, Hkv, G, D, scale, what, port_check=False):
    B = len(lens)
    o = out.cpu().numpy().reshape(B, Hkv, G, D)
    l = lse.cpu().numpy().reshape(B, Hkv, G)
    qb = bits(q).reshape(B, Hkv, G, D)
    for b, n in enumerate(lens):
        want, wl = O.gqa_attention_fp64(qb[b], bits(ks[b][:, :n]), bits(vs[b][:, :n]), scale)
        assert_close(o[b], want, OUT_ATOL, OUT_RTOL, f"{what} b={b}")
        assert_close(l[b], wl, LSE_ATOL, LSE_RTOL, f"{what} lse b={b}")
        if port_check and n > 0:
            po, pm, ps = port.cpu_attn(qb[b], bits(ks[b][:, :n]), bits(vs[b][:, :n]), scale,
                                       normalize=True, n_threads=8)
            assert_close(o[b], po, OUT_ATOL, OUT_RTOL, f"{what} port b={b}")
            assert_close(l[b], (pm + np.log(ps))[..., 0], LSE_ATOL, LSE_RTOL,
                         f"{what} port lse b={b}")


@pytest.mark.parametrize("D", WIDTHS)
@pytest.mark.parametrize("G,wg", [(1, 0), (4, 3), (8, 0), (16, 7)])
def test_gqa_width_partial(D, G, wg):
    """Ragged lengths (empty, one token, block and page edges, rows over many
    splits), every group size class, against fp64 and the C port."""
    lens = [0, 1, 31, 33, 64, 300, 1500]
    Hkv = 2
    _say(f"gqa width D={D} G={G} wg={wg}")
    k_pages, v_pages, pt, gl, ks, vs = gqa_pool(lens, Hkv, D, 64, seed=D + G, device=DEV)
    q = bf16_randn((len(lens), Hkv * G, D), 5 * D + G)
    scale = D ** -0.5
    out, lse = ops.gqa_decode_partial(q.to(DEV), k_pages, v_pages, pt, gl, scale, max(lens),
                                      n_workgroups=wg)
    torch.cuda.synchronize()
    _check_rows(out, lse, q, ks, vs, lens, Hkv, G, D, scale, f"D={D}", port_check=True)
    # the separate-width entry point runs the same kernel: the same bits
    o2, l2 = ops.attn_decode_partial(q.to(DEV), k_pages, v_pages, pt, gl, scale, max(lens),
                                     n_workgroups=wg)
    torch.cuda.synchronize()
    assert torch.equal(o2.cpu(), out.cpu()) and torch.equal(l2.cpu(), lse.cpu())


@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("G", [3, 7, 12])
def test_gqa_group_sizes_without_a_kernel_of_their_own(D, G):
    """Group sizes that are not powers of two (Qwen2-7B: 28 query heads over
    4 KV heads) run the width's kernel with the group size read at run time;
    the fused append step over the same inputs agrees bit for bit with the
    unfused call."""
    lens = [0, 5, 64, 700]
    Hkv = 2
    _say(f"gqa group size G={G} D={D}")
    total = [L + 1 for L in lens]
    k_pages, v_pages, pt, gl, ks, vs = gqa_pool(total, Hkv, D, 64, seed=G + D, device=DEV)
    q = bf16_randn((len(lens), Hkv * G, D), 3 * G + D).to(DEV)
    scale = D ** -0.5
    k_new = torch.stack([k[:, L:L + 1] for k, L in zip(ks, lens)]).to(DEV).contiguous()
    v_new = torch.stack([v[:, L:L + 1] for v, L in zip(vs, lens)]).to(DEV).contiguous()
    len_in = torch.tensor(lens, dtype=torch.int32, device=DEV)
    len_out = torch.zeros_like(len_in)
    out, lse = ops.gqa_append_decode_partial(q, k_new, v_new, k_pages, v_pages, pt, len_in,
                                             len_out, scale, max(total), 5)
    o2, l2 = ops.gqa_decode_partial(q, k_pages, v_pages, pt, len_out, scale, max(total), 5)
    torch.cuda.synchronize()
    assert torch.equal(o2.cpu(), out.cpu()) and torch.equal(l2.cpu(), lse.cpu())
    _check_rows(out, lse, q.cpu(), ks, vs, total, Hkv, G, D, scale, f"G={G} D={D}",
                port_check=True)


@pytest.mark.parametrize("D", OTHER_WIDTHS)
@pytest.mark.parametrize("G,wg", [(1, 0), (6, 5)])
def test_gqa_other_widths_partial(D, G, wg):
    """Every other multiple of 16, group sizes 1 and 6 (a size without a
    kernel of its own), against fp64 and the C port."""
    lens = [0, 1, 33, 300, 1100]
    Hkv = 2
    _say(f"gqa width D={D} G={G} wg={wg}")
    k_pages, v_pages, pt, gl, ks, vs = gqa_pool(lens, Hkv, D, 64, seed=D + 3 * G, device=DEV)
    q = bf16_randn((len(lens), Hkv * G, D), 7 * D + G)
    scale = D ** -0.5
    out, lse = ops.attn_decode_partial(q.to(DEV), k_pages, v_pages, pt, gl, scale, max(lens),
                                       n_workgroups=wg)
    torch.cuda.synchronize()
    _check_rows(out, lse, q, ks, vs, lens, Hkv, G, D, scale, f"D={D}", port_check=True)


@pytest.mark.parametrize("D", WIDTHS + [48, 80, 96, 176, 240])
def test_gqa_width_fused_steps_append_bit_exact(D):
    """Three fused append + attend steps with page size 32: outputs against
    fp64, the unfused call over the written pages bit-identical, and every
    appended K/V row in its page slot bit for bit."""
    Hkv, G, PS, steps = 4, 4, 32, 3
    lens = [0, 1, 31, 32, 95, 400]
    B = len(lens)
    total = [L + steps for L in lens]
    _say(f"gqa width fused steps D={D}")
    k_pages, v_pages, pt, gl, ks, vs = gqa_pool(total, Hkv, D, PS, seed=3 * D, device=DEV)
    for b, L in enumerate(lens):
        for t in range(L, L + steps):
            k_pages[pt[b, t // PS].long(), :, t % PS] = 0
            v_pages[pt[b, t // PS].long(), :, t % PS] = 0
    lens2 = torch.zeros((2, B), dtype=torch.int32, device=DEV)
    lens2[0] = torch.tensor(lens, dtype=torch.int32)
    scale = D ** -0.5
    for i in range(steps):
        q = bf16_randn((B, Hkv * G, D), 40 + i)
        k_new = torch.stack([k[:, L + i:L + i + 1] for k, L in zip(ks, lens)]).to(DEV)
        v_new = torch.stack([v[:, L + i:L + i + 1] for v, L in zip(vs, lens)]).to(DEV)
        len_in, len_out = lens2[i % 2], lens2[(i + 1) % 2]
        out, lse = ops.gqa_append_decode_partial(q.to(DEV), k_new.contiguous(),
                                                 v_new.contiguous(), k_pages, v_pages, pt,
                                                 len_in, len_out, scale, max(lens) + i + 1, 5)
        torch.cuda.synchronize()
        assert len_out.cpu().tolist() == [L + i + 1 for L in lens]
        _check_rows(out, lse, q, ks, vs, [L + i + 1 for L in lens], Hkv, G, D, scale,
                    f"D={D} step {i}")
        o2, l2 = ops.gqa_decode_partial(q.to(DEV), k_pages, v_pages, pt, len_out, scale,
                                        max(lens) + i + 1, 5)
        torch.cuda.synchronize()
        assert torch.equal(o2.cpu(), out.cpu()) and torch.equal(l2.cpu(), lse.cpu())
    kp, vp = bits(k_pages), bits(v_pages)
    tab = pt.cpu().numpy()
    for h in range(Hkv):
        gk = O.gather_paged(kp, tab, total, head=h)
        gv = O.gather_paged(vp, tab, total, head=h)
        for b in range(B):
            assert np.array_equal(gk[b], bits(ks[b][h])), (b, h)
            assert np.array_equal(gv[b], bits(vs[b][h])), (b, h)


@pytest.mark.parametrize("D", WIDTHS + [80, 144])
def test_gqa_width_full_step_bf16(D):
    """The whole-step entry point: bf16 output is the fp32 output rounded to
    nearest even, the fp32 output bit-identical to the partial step's."""
    Hkv, G, PS = 2, 8, 64
    lens = [0, 7, 64, 1000]
    B = len(lens)
    total = [L + 1 for L in lens]
    _say(f"gqa width full step D={D}")
    k_pages, v_pages, pt, gl, ks, vs = gqa_pool(total, Hkv, D, PS, seed=7 * D, device=DEV)
    q = bf16_randn((B, Hkv * G, D), 8).to(DEV)
    k_new = torch.stack([k[:, L:L + 1] for k, L in zip(ks, lens)]).to(DEV).contiguous()
    v_new = torch.stack([v[:, L:L + 1] for v, L in zip(vs, lens)]).to(DEV).contiguous()
    len_in = torch.tensor(lens, dtype=torch.int32, device=DEV)
    scale = D ** -0.5
    ob, of, lse = ops.gqa_append_decode_full(q, k_new, v_new, k_pages, v_pages, pt, len_in,
                                             None, scale, max(total), 0, want_fp32=True)
    o1, l1 = ops.gqa_append_decode_partial(q, k_new, v_new, k_pages, v_pages, pt, len_in,
                                           None, scale, max(total), 0)
    torch.cuda.synchronize()
    assert torch.equal(of.cpu(), o1.cpu()) and torch.equal(lse.cpu(), l1.cpu())
    assert np.array_equal(bits(ob), bits(of.to(torch.bfloat16)))
    _check_rows(ob.float(), lse, q.cpu(), ks, vs, total, Hkv, G, D, scale, f"full D={D}")


@pytest.mark.parametrize("D", WIDTHS + [112, 208])
@pytest.mark.parametrize("fmt", [ops.PARTIAL_LSE_F32, ops.TRIPLE_NORM_BF16])
def test_gqa_width_split_step_and_host_merge(D, fmt):
    """Deferred-combine step + merge with a host partial in two of the
    reference CPU kernel's output conventions, against the fp64 merge."""
    from tests.test_gpu_kernels import _host_partial

    Hkv, G, PS = 4, 4, 64
    lens = [1, 40, 700, 2500]
    B = len(lens)
    total = [L + 1 for L in lens]
    _say(f"gqa width split + merge D={D} fmt={fmt}")
    k_pages, v_pages, pt, gl, ks, vs = gqa_pool(total, Hkv, D, PS, seed=11 * D, device=DEV)
    lens2 = torch.zeros((2, B), dtype=torch.int32, device=DEV)
    lens2[0] = torch.tensor(lens, dtype=torch.int32)
    q = bf16_randn((B, Hkv * G, D), 12)
    k_new = torch.stack([k[:, L:L + 1] for k, L in zip(ks, lens)]).to(DEV).contiguous()
    v_new = torch.stack([v[:, L:L + 1] for v, L in zip(vs, lens)]).to(DEV).contiguous()
    scale = D ** -0.5
    step = ops.gqa_append_decode_split(q.to(DEV), k_new, v_new, k_pages, v_pages, pt,
                                       lens2[0], lens2[1], scale, max(lens) + 1, 0)
    rows = B * Hkv * G
    hb, host_o, host_l = _host_partial(fmt, rows, D, 13)
    out, lse = ops.merge_split(step, hb, fmt, out_dtype=torch.float32)
    torch.cuda.synchronize()
    got = out.cpu().numpy().reshape(B, Hkv, G, D)
    gls = lse.cpu().numpy().reshape(B, Hkv, G)
    qb = bits(q).reshape(B, Hkv, G, D)
    ho, hl = host_o.reshape(B, Hkv, G, D), host_l.reshape(B, Hkv, G)
    for b in range(B):
        g_o, g_l = O.gqa_attention_fp64(qb[b], bits(ks[b]), bits(vs[b]), scale)
        want, wl = O.merge_fp64(g_o, g_l, ho[b], hl[b])
        assert_close(got[b], want, OUT_ATOL, OUT_RTOL, f"merged D={D} b={b}")
        assert_close(gls[b], wl, LSE_ATOL, LSE_RTOL, f"merged lse D={D} b={b}")


@pytest.mark.parametrize("D", WIDTHS + [80])
def test_gqa_width_noalloc_matches_workspace_call(D):
    """The no-allocation entry point at another width: bit-identical to the
    workspace entry point, on two calls in a row, the second smaller."""
    Hkv, G, PS = 2, 4, 64
    scale = D ** -0.5
    for lens, seed in (([5, 300, 1200], 1), ([2, 70], 2)):
        B = len(lens)
        total = [L + 1 for L in lens]
        _say(f"gqa width noalloc D={D} lens={lens}")
        kp, vp, pt, gl, ks, vs = gqa_pool(total, Hkv, D, PS, seed=D + seed, device=DEV)
        kp2, vp2 = kp.clone(), vp.clone()
        q = bf16_randn((B, Hkv * G, D), 90 + seed).to(DEV)
        k_new = torch.stack([k[:, L:L + 1] for k, L in zip(ks, lens)]).to(DEV).contiguous()
        v_new = torch.stack([v[:, L:L + 1] for v, L in zip(vs, lens)]).to(DEV).contiguous()
        len_in = torch.tensor(lens, dtype=torch.int32, device=DEV)
        o1, l1 = ops.gqa_append_decode_partial(q, k_new, v_new, kp, vp, pt, len_in, None,
                                               scale, max(total), 6)
        o2 = torch.empty_like(o1)
        l2 = torch.empty_like(l1)
        ops.gqa_append_decode_partial_noalloc(q, k_new, v_new, kp2, vp2, pt, len_in, None,
                                              scale, max(total), o2, l2, 6)
        torch.cuda.synchronize()
        assert torch.equal(o1.cpu(), o2.cpu()) and torch.equal(l1.cpu(), l2.cpu())
        assert torch.equal(kp.cpu(), kp2.cpu()) and torch.equal(vp.cpu(), vp2.cpu())


@pytest.mark.parametrize("D", WIDTHS + [80, 112])
def test_partitioned_gqa_step_with_native_host_partial(D):
    """One two-sided decode step through the partitioned cache: GPU split
    step with the append, this package's host partial over the host tokens
    (bf16, any multiple of 16 up to 256), merge; against fp64 attention over
    the whole sequence."""
    B, Hkv, G = 3, 4, 4
    rng = np.random.default_rng(D)
    lens = rng.integers(100, 1500, B)
    _say(f"partitioned gqa D={D} lens={lens.tolist()}")
    scale = D ** -0.5
    k_all = [bf16_randn((Hkv, int(L) + 1, D), 50 + b) for b, L in enumerate(lens)]
    v_all = [bf16_randn((Hkv, int(L) + 1, D), 60 + b) for b, L in enumerate(lens)]
    g = [gpu_share(int(L), 0.5) for L in lens]
    cache = PartitionedKVCache(1, B, Hkv, D, max_host=int(lens.max()),
                               max_gpu=max(g) + 64, device=DEV)
    for b, L in enumerate(lens):
        h = int(L) - g[b]
        cache.load_host(0, b, k_all[b][:, :h], v_all[b][:, :h])
        cache.gpu.load_sequence(0, b, k_all[b][:, h:L].to(DEV), v_all[b][:, h:L].to(DEV))
    k_new = torch.stack([k[:, -1:] for k in k_all]).to(DEV)
    v_new = torch.stack([v[:, -1:] for v in v_all]).to(DEV)
    q = bf16_randn((B, Hkv * G, D), 70)
    out = partitioned_gqa_decode(cache, 0, q.to(DEV), scale, NATIVE,
                                 cpu_format="fused_cpu_attn_bf16", k_new=k_new, v_new=v_new,
                                 host_threads=3)
    torch.cuda.synchronize()
    assert out.shape == (B, Hkv * G, 1, D)
    got = out.float().cpu().numpy()[:, :, 0]
    qb = bits(q).reshape(B, Hkv, G, D)
    for b in range(B):
        want, _ = O.gqa_attention_fp64(qb[b], bits(k_all[b]), bits(v_all[b]), scale)
        assert_close(got[b].reshape(Hkv, G, D), want, OUT_ATOL, OUT_RTOL, f"D={D} b={b}")
    assert cache.gpu.lens[0].tolist() == [gg + 1 for gg in g]


@pytest.mark.parametrize("D", [64, 80, 96, 256])
def test_reference_api_local_bmm_softmax_widths(D):
    """The reference-signature GPU partial (_local_bmm_softmax,
    roofline/bench_resident_kv.py:150-157) at other head widths: its
    (o, max, sum) triple against fp64 attention."""
    from scope_amd import reference_api
    N, G, S = 6, 4, 700
    q, k, v = (bf16_randn((N, G, D), 20 + D), bf16_randn((N, S, D), 21 + D),
               bf16_randn((N, S, D), 22 + D))
    scale = D ** -0.5
    o, m, s = reference_api.local_bmm_softmax(q.to(DEV), k.to(DEV), v.to(DEV), scale)
    torch.cuda.synchronize()
    ow, lw = O.gqa_attention_fp64(bits(q), bits(k), bits(v), scale)
    assert_close(o.cpu().numpy(), ow, OUT_ATOL, OUT_RTOL, f"o D={D}")
    lse = (m + torch.log(s)).cpu().numpy()[..., 0]
    assert_close(lse, lw, LSE_ATOL, LSE_RTOL, f"max + log(sum) D={D}")


@pytest.mark.parametrize("Dk,Dv", [(40, 40), (8, 8), (272, 272), (128, 64), (256, 128)])
def test_unsupported_widths_are_rejected(Dk, Dv):
    B, Hkv, PS = 1, 1, 64
    q = torch.zeros((B, Hkv, Dk), dtype=torch.bfloat16, device=DEV)
    kp = torch.zeros((2, Hkv, PS, Dk), dtype=torch.bfloat16, device=DEV)
    vp = torch.zeros((2, Hkv, PS, Dv), dtype=torch.bfloat16, device=DEV)
    pt = torch.zeros((B, 1), dtype=torch.int32, device=DEV)
    gl = torch.ones(B, dtype=torch.int32, device=DEV)
    with pytest.raises(RuntimeError, match="unsupported"):
        ops.attn_decode_partial(q, kp, vp, pt, gl, 1.0, 1, n_workgroups=2)
