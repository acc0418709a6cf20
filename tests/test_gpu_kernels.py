"""GPU parity of the gfx950 kernels through the C-ABI (ops layer) against the
oracle: fp64 closed forms and the C restatement of the reference CPU kernels.

Bar: appends and page indexing bit-exact; outputs within 2e-2 abs/rel; fp32
LSE within 1e-3.
"""
import numpy as np
import pytest
import torch

from oracle import attn_np as O
from oracle import port
from scope_amd import ops
from tests.gpu_pool import gqa_pool, mla_pool, page_layout
from tests.helpers import (LSE_ATOL, LSE_RTOL, OUT_ATOL, OUT_RTOL, assert_close,
                           bf16_randn, bits)

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _say(msg):
    print(msg, flush=True)


# ---------------------------------------------------------------------------
# append


@pytest.mark.parametrize("n_new_seq", [[1, 1, 1, 1], [5, 70, 1], [64, 3]])
def test_kv_append_bit_exact(n_new_seq):
    _say(f"kv_append n_new_seq={n_new_seq}")
    B, Hkv, D, PS = 3, 8, 128, 64
    total = sum(n_new_seq)
    table, num_pages = page_layout([total] * B, PS, seed=7)
    k_pages = torch.zeros((num_pages, Hkv, PS, D), dtype=torch.bfloat16, device=DEV)
    v_pages = torch.zeros_like(k_pages)
    pt = torch.from_numpy(table).to(DEV)
    gl = torch.zeros(B, dtype=torch.int32, device=DEV)
    ks, vs = [], []
    for i, n in enumerate(n_new_seq):
        k = bf16_randn((B, Hkv, n, D), 100 + i)
        v = bf16_randn((B, Hkv, n, D), 200 + i)
        ops.kv_append(k.to(DEV), v.to(DEV), k_pages, v_pages, pt, gl)
        ks.append(k); vs.append(v)
    torch.cuda.synchronize()
    assert gl.cpu().tolist() == [total] * B
    want_k = torch.cat(ks, 2)
    want_v = torch.cat(vs, 2)
    kp, vp = bits(k_pages), bits(v_pages)
    for b in range(B):
        for h in range(Hkv):
            got_k = O.gather_paged(kp, table, [total] * B, head=h)[b]
            got_v = O.gather_paged(vp, table, [total] * B, head=h)[b]
            assert np.array_equal(got_k, bits(want_k[b, h]))
            assert np.array_equal(got_v, bits(want_v[b, h]))
    # untouched pages stay zero
    used = set(table[table >= 0].ravel().tolist())
    for pid in range(num_pages):
        if pid not in used:
            assert not kp[pid].any()
    # update_len=False leaves lengths alone
    ops.kv_append(ks[0].to(DEV), vs[0].to(DEV), k_pages, v_pages, pt,
                  torch.zeros(B, dtype=torch.int32, device=DEV), update_len=False)
    torch.cuda.synchronize()


def test_latent_append_bit_exact_strided():
    _say("latent_append strided")
    B, PS = 2, 64
    steps = [1, 63, 2, 100]
    total = sum(steps)
    table, num_pages = page_layout([total] * B, PS, seed=9)
    lat = torch.zeros((num_pages, PS, 576), dtype=torch.bfloat16, device=DEV)
    pt = torch.from_numpy(table).to(DEV)
    gl = torch.zeros(B, dtype=torch.int32, device=DEV)
    full = []
    for i, n in enumerate(steps):
        kv = bf16_randn((B, n, 576), 300 + i).to(DEV)  # kv_a_proj-like [B, n, 576]
        c, pe = kv[..., :512], kv[..., 512:]           # strided views (row stride 576)
        ops.latent_append(c, pe, lat, pt, gl)
        full.append(kv.cpu())
    torch.cuda.synchronize()
    assert gl.cpu().tolist() == [total] * B
    want = torch.cat(full, 1)
    got = O.gather_paged(bits(lat), table, [total] * B)
    for b in range(B):
        assert np.array_equal(got[b], bits(want[b]))


# ---------------------------------------------------------------------------
# GQA partial


def _gqa_check(lens, Hkv, G, PS=64, wg=0, seed=1, sigma=1.0, port_check=True):
    D = 128
    B = len(lens)
    _say(f"gqa lens={list(lens)[:8]}{'...' if B > 8 else ''} Hkv={Hkv} G={G} PS={PS} wg={wg}")
    k_pages, v_pages, pt, gl, ks, vs = gqa_pool(lens, Hkv, D, PS, seed, DEV, sigma)
    q = bf16_randn((B, Hkv * G, D), seed + 77, sigma)
    scale = D ** -0.5
    out, lse = ops.gqa_decode_partial(q.to(DEV), k_pages, v_pages, pt, gl, scale,
                                      max(lens), n_workgroups=wg)
    torch.cuda.synchronize()
    out, lse = out.cpu().numpy(), lse.cpu().numpy()
    qb = bits(q).reshape(B, Hkv, G, D)
    for b in range(B):
        want, wl = O.gqa_attention_fp64(qb[b], bits(ks[b]), bits(vs[b]), scale)
        assert_close(out[b].reshape(Hkv, G, D), want, OUT_ATOL, OUT_RTOL, f"out b={b}")
        assert_close(lse[b].reshape(Hkv, G), wl, LSE_ATOL, LSE_RTOL, f"lse b={b}")
        if port_check and lens[b] > 0:
            po, pm, ps = port.cpu_attn(qb[b], bits(ks[b]), bits(vs[b]), scale,
                                       normalize=True, n_threads=8)
            assert_close(out[b].reshape(Hkv, G, D), po, OUT_ATOL, OUT_RTOL, f"port b={b}")
            assert_close(lse[b].reshape(Hkv, G), (pm + np.log(ps))[..., 0],
                         LSE_ATOL, LSE_RTOL, f"port lse b={b}")
    return out, lse


def test_gqa_config1_qwen3_single_partition():
    # B=1, 32 q heads / 4 KV heads, D 128, L 4096 in one partition
    _gqa_check([4096], Hkv=4, G=8, seed=1000)


@pytest.mark.parametrize("G", [1, 2, 4, 8, 16])
def test_gqa_group_sizes(G):
    _gqa_check([300, 64, 1], Hkv=2, G=G, seed=40 + G)


@pytest.mark.parametrize("wg", [0, 1, 3, 7, 64, 1000])
def test_gqa_ragged_lengths_and_workgroups(wg):
    # 1 workgroup walks every row; 3 and 7 split rows across workgroups at
    # odd block boundaries; 1000 exceeds the blocks (capped on the device)
    lens = [0, 1, 31, 32, 33, 63, 64, 65, 127, 1000]
    _gqa_check(lens, Hkv=8, G=4, wg=wg, seed=5)


@pytest.mark.parametrize("wg", [0, 37])
def test_gqa_more_than_64_sequences(wg):
    # 70 sequences: the plan is built by the whole workgroup behind barriers
    lens = [int(x) for x in np.random.default_rng(70 + wg).integers(0, 150, 70)]
    _gqa_check(lens, Hkv=2, G=4, wg=wg, seed=63, port_check=False)


@pytest.mark.parametrize("wg", [0, 2, 5, 9, 40])
def test_gqa_one_kv_head_sequence_aligned_plan(wg):
    # one kv row per sequence: the plan may give every sequence its own splits
    # (0, 9, 40: sequence-aligned; 2, 5: equal shares across sequences)
    _gqa_check([0, 40, 300, 1000, 65], Hkv=1, G=8, wg=wg, seed=9)


def test_gqa_page_size_128_and_32():
    _gqa_check([500, 129], Hkv=4, G=8, PS=128, seed=6)
    _gqa_check([500, 129], Hkv=4, G=8, PS=32, seed=6)


def test_gqa_large_scores_no_overflow():
    # sigma 4 -> scores ~ N(0, 16^2 / ...) large; online rescale must hold
    _gqa_check([700], Hkv=4, G=8, seed=8, sigma=4.0)


def test_gqa_split_invariance_and_page_permutation():
    lens = [3000, 2500]
    k_pages, v_pages, pt, gl, ks, vs = gqa_pool(lens, 8, 128, 64, 11, DEV)
    q = bf16_randn((2, 32, 128), 12).to(DEV)
    res = [ops.gqa_decode_partial(q, k_pages, v_pages, pt, gl, 0.0884, 3000,
                                  n_workgroups=n) for n in (1, 8, 100)]
    # P is rounded to bf16 against each split's running max, so outputs of
    # different split counts differ at the bf16 level; the fp32 sums keep the
    # LSE split-independent to fp32 rounding.
    for o, l in res[1:]:
        assert_close(o.cpu().numpy(), res[0][0].cpu().numpy(), 2e-3, 2e-3, "split inv")
        assert_close(l.cpu().numpy(), res[0][1].cpu().numpy(), 1e-5, 1e-5, "split inv lse")
    # moving pages to other physical ids changes nothing, bit for bit
    perm = torch.randperm(k_pages.shape[0], generator=torch.Generator().manual_seed(3)).to(DEV)
    inv = torch.empty_like(perm); inv[perm] = torch.arange(perm.numel(), device=DEV)
    k2 = torch.empty_like(k_pages); v2 = torch.empty_like(v_pages)
    k2[inv] = k_pages; v2[inv] = v_pages
    pt2 = torch.where(pt >= 0, inv[pt.long().clamp(min=0)].int(), pt)
    o2, l2 = ops.gqa_decode_partial(q, k2, v2, pt2, gl, 0.0884, 3000, n_workgroups=8)
    assert torch.equal(o2, res[1][0]) and torch.equal(l2, res[1][1])


# ---------------------------------------------------------------------------
# MLA partial


def _mla_check(lens, wg=0, seed=3, sigma=0.5, PS=64):
    B, H = len(lens), 16
    _say(f"mla lens={lens} wg={wg} PS={PS}")
    lat, pt, gl, cs, pes = mla_pool(lens, PS, seed, DEV, sigma)
    qn = bf16_randn((B * H, 512), seed + 91, sigma)
    qp = bf16_randn((B * H, 64), seed + 92, sigma)
    scale = 192 ** -0.5
    out, lse = ops.mla_decode_partial(qn.to(DEV), qp.to(DEV), lat, pt, gl, scale,
                                      max(lens), n_workgroups=wg)
    torch.cuda.synchronize()
    out, lse = out.cpu().numpy(), lse.cpu().numpy()
    for b in range(B):
        rows = slice(b * H, (b + 1) * H)
        c, pe = bits(cs[b])[None], bits(pes[b])[None]
        want, wl = O.mla_attention_fp64(bits(qn[rows]), bits(qp[rows]), c, pe, scale)
        assert_close(out[rows], want, OUT_ATOL, OUT_RTOL, f"mla out b={b}")
        assert_close(lse[rows], wl, LSE_ATOL, LSE_RTOL, f"mla lse b={b}")
        if lens[b] > 0:
            po, pm, ps = port.cpu_attn_mla_compressed(bits(qn[rows]), bits(qp[rows]), c, pe,
                                                      scale, n_threads=8)
            assert_close(out[rows], po / ps[:, None], OUT_ATOL, OUT_RTOL, f"port b={b}")
            assert_close(lse[rows], pm + np.log(ps), LSE_ATOL, LSE_RTOL, f"port lse b={b}")


@pytest.mark.parametrize("wg", [0, 1, 3, 17, 500])
def test_mla_ragged(wg):
    _mla_check([0, 1, 37, 300, 1030], wg=wg)


def test_mla_config3_shape_subset():
    # DS-V2-Lite absorbed: H 16, latent 576, N(0, 0.5), L 16384 with r 0.5
    _mla_check([8192, 8192], seed=3000)


@pytest.mark.parametrize("B,wg", [(64, 0), (64, 40), (65, 0), (65, 40)])
def test_mla_plan_at_the_per_wave_limit(B, wg):
    # 64 sequences: every wave builds the plan alone (sequence-aligned when it
    # fits); 65: the workgroup builds the equal-share plan behind barriers
    lens = [int(x) for x in np.random.default_rng(B + wg).integers(0, 200, B)]
    _mla_check(lens, wg=wg, seed=62)


@pytest.mark.parametrize("wg,PS", [(1, 64), (2, 64), (1, 32)])
def test_mla_long_segments_refill_page_windows(wg, PS):
    # a workgroup reads its segment's page ids 64 blocks at a time; segments
    # of 157 and 122 blocks cross one or two window refills
    _mla_check([5000, 2100, 700], wg=wg, seed=61, PS=PS)


# ---------------------------------------------------------------------------
# split reduce and merge


def test_split_reduce_direct():
    # 3 sequences x 3 heads: len 0 -> (0, -inf); len 64 with 64-token splits
    # -> one split, row left untouched; len 200 -> 4 splits merged
    rows, Dv, ns, tps, H = 9, 128, 4, 64, 3
    lens = torch.tensor([0, 64, 200], dtype=torch.int32, device=DEV)
    g = torch.Generator().manual_seed(4)
    po = torch.randn((ns, rows, Dv), generator=g)
    pl = torch.randn((ns, rows), generator=g) * 3
    out = torch.full((rows, Dv), 7.0, device=DEV)
    lse = torch.full((rows,), 7.0, device=DEV)
    ops.split_reduce(po.to(DEV), pl.to(DEV), lens, H, tps, out, lse)
    torch.cuda.synchronize()
    o, l = out.cpu().numpy(), lse.cpu().numpy()
    assert np.all(o[0:3] == 0) and np.all(np.isneginf(l[0:3]))
    assert np.all(o[3:6] == 7.0) and np.all(l[3:6] == 7.0)
    acc = (po[0, 6:9].numpy().astype(np.float64), pl[0, 6:9].numpy().astype(np.float64))
    for s in range(1, 4):
        acc = O.merge_fp64(*acc, po[s, 6:9].numpy(), pl[s, 6:9].numpy())
    assert_close(o[6:9], acc[0], 1e-5, 1e-5, "reduce out")
    assert_close(l[6:9], acc[1], 1e-5, 1e-5, "reduce lse")


def test_split_reduce_merges_valid_splits():
    rows, Dv, ns, tps, H = 2, 512, 5, 32, 2
    lens = torch.tensor([100], dtype=torch.int32, device=DEV)  # 4 valid splits of 5
    g = torch.Generator().manual_seed(5)
    po = torch.randn((ns, rows, Dv), generator=g)
    pl = torch.randn((ns, rows), generator=g) * 4
    out, lse = ops.split_reduce(po.to(DEV), pl.to(DEV), lens, H, tps)
    torch.cuda.synchronize()
    acc = (po[0].numpy().astype(np.float64), pl[0].numpy().astype(np.float64))
    for s in range(1, 4):
        acc = O.merge_fp64(*acc, po[s].numpy(), pl[s].numpy())
    assert_close(out.cpu().numpy(), acc[0], 1e-5, 1e-5, "reduce out")
    assert_close(lse.cpu().numpy(), acc[1], 1e-5, 1e-5, "reduce lse")


@pytest.mark.parametrize("fmt", [ops.PARTIAL_LSE_F32, ops.TRIPLE_UNNORM_F32,
                                 ops.TRIPLE_NORM_BF16, ops.TRIPLE_NORM_F32,
                                 ops.PARTIAL_LSE_BF16])
@pytest.mark.parametrize("Dv", [128, 512])
def test_lse_merge_formats(fmt, Dv):
    _say(f"lse_merge fmt={fmt} Dv={Dv}")
    rows = 40
    rng = np.random.default_rng(fmt * 10 + Dv)
    oa = rng.standard_normal((rows, Dv)).astype(np.float32)
    la = (rng.standard_normal(rows) * 3).astype(np.float32)
    ob = rng.standard_normal((rows, Dv)).astype(np.float32)
    mb = (rng.standard_normal(rows) * 3).astype(np.float32)
    sb = rng.uniform(1, 50, rows).astype(np.float32)
    # empties: row 0 GPU empty, row 1 host empty, row 2 both
    la[0] = -np.inf; oa[0] = 0
    sb[1] = 0.0; mb[1] = -np.inf
    la[2] = -np.inf; oa[2] = 0; sb[2] = 0.0; mb[2] = -np.inf
    if fmt == ops.PARTIAL_LSE_F32:
        lb = np.where(sb > 0, mb + np.log(np.where(sb > 0, sb, 1)), -np.inf).astype(np.float32)
        b = (torch.from_numpy(ob).to(DEV), torch.from_numpy(lb).to(DEV))
        ob_n, lb_n = np.where(sb[:, None] > 0, ob, 0), lb
    elif fmt == ops.TRIPLE_UNNORM_F32:
        ou = np.where(sb[:, None] > 0, ob * sb[:, None], 0).astype(np.float32)
        b = tuple(torch.from_numpy(x).to(DEV) for x in (ou, mb, sb))
        ob_n, lb_n = O.triple_to_partial(ou, mb, sb, normalized=False)
    elif fmt == ops.TRIPLE_NORM_F32:
        b = tuple(torch.from_numpy(x).to(DEV) for x in (ob, mb, sb))
        ob_n, lb_n = O.triple_to_partial(ob, mb, sb, normalized=True)
    elif fmt == ops.PARTIAL_LSE_BF16:  # bf16 out, fp32 lse
        lb = np.where(sb > 0, mb + np.log(np.where(sb > 0, sb, 1)), -np.inf).astype(np.float32)
        ob16 = torch.from_numpy(np.where(sb[:, None] > 0, ob, 0).astype(np.float32)).to(
            torch.bfloat16)
        b = (ob16.to(DEV), torch.from_numpy(lb).to(DEV))
        ob_n, lb_n = ob16.float().numpy(), lb
    else:
        ob16, mb16, sb16 = (torch.from_numpy(x).to(torch.bfloat16) for x in (ob, mb, sb))
        b = tuple(x.to(DEV) for x in (ob16, mb16, sb16))
        ob_n, lb_n = O.triple_to_partial(ob16.float().numpy(), mb16.float().numpy(),
                                         sb16.float().numpy(), normalized=True)
    want_o, want_l = O.merge_fp64(oa, la, ob_n, lb_n)
    for odt in (torch.bfloat16, torch.float32):
        out, lse = ops.lse_merge(torch.from_numpy(oa).to(DEV), torch.from_numpy(la).to(DEV),
                                 b, fmt, out_dtype=odt)
        torch.cuda.synchronize()
        got = out.float().cpu().numpy()
        assert np.isfinite(got).all()
        assert_close(got, want_o, OUT_ATOL if odt == torch.bfloat16 else 1e-5,
                     OUT_RTOL if odt == torch.bfloat16 else 1e-5, "merge out")
        assert_close(lse.cpu().numpy(), want_l, 1e-5, 1e-5, "merge lse")
    assert np.all(got[2] == 0) and np.isneginf(lse.cpu().numpy()[2])


# ---------------------------------------------------------------------------
# fused append + partial (one launch per decode step)


@pytest.mark.parametrize("Hkv,G,wg,PS", [(8, 4, 0, 64), (8, 4, 5, 64), (4, 8, 64, 64),
                                         (2, 16, 3, 64), (8, 4, 5, 32), (4, 8, 0, 96)])
def test_gqa_append_decode_fused_steps(Hkv, G, wg, PS):
    # page sizes 32 and 96 (not a power of two): appends across page ends
    _say(f"gqa fused append+decode Hkv={Hkv} G={G} wg={wg} PS={PS}")
    D = 128
    lens = [0, 1, 63, 64, 200, 777]
    B, steps = len(lens), 3
    total = [L + steps for L in lens]
    k_pages, v_pages, pt, gl, ks, vs = gqa_pool(total, Hkv, D, PS, seed=21)
    # the pool holds all tokens; the partition starts with `lens` of them
    lens2 = torch.zeros((2, B), dtype=torch.int32, device=DEV)
    lens2[0] = torch.tensor(lens, dtype=torch.int32)
    # zero the slots the steps will append into, so the writes are observable
    for b, L in enumerate(lens):
        for t in range(L, L + steps):
            k_pages[pt[b, t // PS].long(), :, t % PS] = 0
            v_pages[pt[b, t // PS].long(), :, t % PS] = 0
    scale = D ** -0.5
    for i in range(steps):
        q = bf16_randn((B, Hkv * G, D), 900 + i)
        k_new = torch.stack([k[:, L + i:L + i + 1] for k, L in zip(ks, lens)]).to(DEV)
        v_new = torch.stack([v[:, L + i:L + i + 1] for v, L in zip(vs, lens)]).to(DEV)
        len_in, len_out = lens2[i % 2], lens2[(i + 1) % 2]
        out, lse = ops.gqa_append_decode_partial(q.to(DEV), k_new.contiguous(),
                                                 v_new.contiguous(), k_pages, v_pages, pt,
                                                 len_in, len_out, scale,
                                                 max(lens) + i + 1, wg)
        torch.cuda.synchronize()
        assert len_out.cpu().tolist() == [L + i + 1 for L in lens]
        assert len_in.cpu().tolist() == [L + i for L in lens]
        o, l = out.cpu().numpy(), lse.cpu().numpy()
        qb = bits(q).reshape(B, Hkv, G, D)
        for b, L in enumerate(lens):
            n = L + i + 1
            want, wl = O.gqa_attention_fp64(qb[b], bits(ks[b][:, :n]), bits(vs[b][:, :n]),
                                            scale)
            assert_close(o[b].reshape(Hkv, G, D), want, OUT_ATOL, OUT_RTOL, f"b={b} i={i}")
            assert_close(l[b].reshape(Hkv, G), wl, LSE_ATOL, LSE_RTOL, f"lse b={b} i={i}")
        # the unfused pair over the pages the fused call wrote gives the same bits
        o2, l2 = ops.gqa_decode_partial(q.to(DEV), k_pages, v_pages, pt, len_out, scale,
                                        max(lens) + i + 1, wg)
        torch.cuda.synchronize()
        assert torch.equal(o2.cpu(), out.cpu()) and torch.equal(l2.cpu(), lse.cpu())
    # pages now hold every appended token, bit for bit
    kp, vp = bits(k_pages), bits(v_pages)
    tab = pt.cpu().numpy()
    for h in range(Hkv):
        gk = O.gather_paged(kp, tab, total, head=h)
        gv = O.gather_paged(vp, tab, total, head=h)
        for b in range(B):
            assert np.array_equal(gk[b], bits(ks[b][h])), (b, h)
            assert np.array_equal(gv[b], bits(vs[b][h])), (b, h)


@pytest.mark.parametrize("Hkv,G,wg", [(8, 4, 0), (8, 8, 7), (2, 16, 64), (1, 1, 300),
                                      (4, 2, 1)])
def test_gqa_append_decode_full_step(Hkv, G, wg):
    """The one-launch whole step (bf16 normalised output): against fp64, its
    fp32 output bit-identical to the one-launch partial's, its bf16 output
    the fp32 one rounded to nearest even, appends bit-exact."""
    _say(f"gqa full step Hkv={Hkv} G={G} wg={wg}")
    D, PS = 128, 64
    lens = [0, 1, 31, 64, 500, 2049]
    B = len(lens)
    total = [L + 1 for L in lens]
    k_pages, v_pages, pt, gl, ks, vs = gqa_pool(total, Hkv, D, PS, seed=23)
    for b, L in enumerate(lens):
        k_pages[pt[b, L // PS].long(), :, L % PS] = 0
        v_pages[pt[b, L // PS].long(), :, L % PS] = 0
    q = bf16_randn((B, Hkv * G, D), 24).to(DEV)
    k_new = torch.stack([k[:, L:L + 1] for k, L in zip(ks, lens)]).to(DEV).contiguous()
    v_new = torch.stack([v[:, L:L + 1] for v, L in zip(vs, lens)]).to(DEV).contiguous()
    len_in = torch.tensor(lens, dtype=torch.int32, device=DEV)
    len_out = torch.zeros_like(len_in)
    scale = D ** -0.5
    ob, of, lse = ops.gqa_append_decode_full(q, k_new, v_new, k_pages, v_pages, pt, len_in,
                                             len_out, scale, max(total), wg, want_fp32=True)
    ob2, lse2 = ops.gqa_append_decode_full(q, k_new, v_new, k_pages, v_pages, pt, len_in,
                                           None, scale, max(total), wg)
    # the partial step appends the same bits again into the same slots
    o1, l1 = ops.gqa_append_decode_partial(q, k_new, v_new, k_pages, v_pages, pt, len_in,
                                           None, scale, max(total), wg)
    torch.cuda.synchronize()
    assert len_out.cpu().tolist() == total
    assert torch.equal(of.cpu(), o1.cpu()) and torch.equal(lse.cpu(), l1.cpu())
    assert torch.equal(ob.cpu(), ob2.cpu()) and torch.equal(lse.cpu(), lse2.cpu())
    assert np.array_equal(bits(ob), bits(of.to(torch.bfloat16)))
    got, gl_ = ob.float().cpu().numpy(), lse.cpu().numpy()
    qb = bits(q).reshape(B, Hkv, G, D)
    for b in range(B):
        want, wl = O.gqa_attention_fp64(qb[b], bits(ks[b]), bits(vs[b]), scale)
        assert_close(got[b].reshape(Hkv, G, D), want, OUT_ATOL, OUT_RTOL, f"b={b}")
        assert_close(gl_[b].reshape(Hkv, G), wl, LSE_ATOL, LSE_RTOL, f"lse b={b}")
    kp, vp = bits(k_pages), bits(v_pages)
    tab = pt.cpu().numpy()
    for h in range(Hkv):
        gk = O.gather_paged(kp, tab, total, head=h)
        gv = O.gather_paged(vp, tab, total, head=h)
        for b in range(B):
            assert np.array_equal(gk[b], bits(ks[b][h])), (b, h)
            assert np.array_equal(gv[b], bits(vs[b][h])), (b, h)


def test_gqa_full_step_bad_lengths_give_nan_rows():
    """A length past the page table's capacity makes its rows NaN (out_bf16,
    out and lse) and len_out -1; the other rows are untouched by it."""
    _say("gqa full step bad length")
    Hkv, G, D, PS = 2, 4, 128, 64
    lens = [100, 300]
    k_pages, v_pages, pt, gl, ks, vs = gqa_pool([L + 1 for L in lens], Hkv, D, PS, seed=25)
    q = bf16_randn((2, Hkv * G, D), 26).to(DEV)
    k_new = torch.stack([k[:, L:L + 1] for k, L in zip(ks, lens)]).to(DEV).contiguous()
    v_new = torch.stack([v[:, L:L + 1] for v, L in zip(vs, lens)]).to(DEV).contiguous()
    cap = pt.shape[1] * PS
    len_in = torch.tensor([lens[0], cap + 5], dtype=torch.int32, device=DEV)
    len_out = torch.zeros_like(len_in)
    ob, of, lse = ops.gqa_append_decode_full(q, k_new, v_new, k_pages, v_pages, pt, len_in,
                                             len_out, D ** -0.5, cap, 3, want_fp32=True)
    torch.cuda.synchronize()
    assert len_out.cpu().tolist() == [lens[0] + 1, -1]
    assert torch.isnan(ob[1].float()).all() and torch.isnan(of[1]).all()
    assert torch.isnan(lse[1]).all()
    qb = bits(q).reshape(2, Hkv, G, D)
    want, wl = O.gqa_attention_fp64(qb[0], bits(ks[0]), bits(vs[0]), D ** -0.5)
    assert_close(ob[0].float().cpu().numpy().reshape(Hkv, G, D), want, OUT_ATOL, OUT_RTOL, "ok")


def test_gqa_one_row_over_many_splits():
    # one row spread over 512 splits (2 blocks each): the combine takes 512
    # pieces
    _say("gqa one row over 512 splits")
    _gqa_check([32768], Hkv=1, G=8, wg=512, seed=31, port_check=False)


def test_gqa_split_capacity_error():
    # 5000 splits > the 4096 pieces a merge takes: rejected on the host before
    # any launch
    k_pages, v_pages, pt, gl, ks, vs = gqa_pool([64], 1, 128, 64, seed=2)
    q = bf16_randn((1, 16, 128), 3).to(DEV)
    with pytest.raises(ops.WsError, match="exceed"):
        ops.gqa_decode_partial(q, k_pages, v_pages, pt, gl, 0.1, 64, n_workgroups=5000)


@pytest.mark.parametrize("wg,lens,PS", [(0, [0, 5, 64, 300], 64), (3, [0, 5, 64, 300], 64),
                                        (1, [0, 5, 300, 4200], 64), (3, [0, 95, 96, 300], 96),
                                        (2, [0, 31, 32, 700], 32)])
def test_mla_append_decode_fused_steps(wg, lens, PS):
    # wg 1 with 4200 tokens: the new token's segment ends two page-id
    # windows past its start; page sizes 96 and 32: appends across page ends
    _say(f"mla fused append+decode wg={wg} lens={lens} PS={PS}")
    H = 16
    B, steps = len(lens), 2
    total = [L + steps for L in lens]
    lat, pt, gl, cs, pes = mla_pool(total, PS, seed=44)
    lens2 = torch.zeros((2, B), dtype=torch.int32, device=DEV)
    lens2[0] = torch.tensor(lens, dtype=torch.int32)
    for b, L in enumerate(lens):
        for t in range(L, L + steps):
            lat[pt[b, t // PS].long(), t % PS] = 0
    scale = 192 ** -0.5
    for i in range(steps):
        qn = bf16_randn((B * H, 512), 600 + i, 0.5)
        qp = bf16_randn((B * H, 64), 700 + i, 0.5)
        kv = torch.stack([torch.cat([c[L + i:L + i + 1], pe[L + i:L + i + 1]], 1)
                          for c, pe, L in zip(cs, pes, lens)]).to(DEV)  # [B, 1, 576]
        c_new, pe_new = kv[..., :512], kv[..., 512:]
        len_in, len_out = lens2[i % 2], lens2[(i + 1) % 2]
        out, lse = ops.mla_append_decode_partial(qn.to(DEV), qp.to(DEV), c_new, pe_new, lat,
                                                 pt, len_in, len_out, scale,
                                                 max(lens) + i + 1, wg)
        torch.cuda.synchronize()
        assert len_out.cpu().tolist() == [L + i + 1 for L in lens]
        o, l = out.cpu().numpy(), lse.cpu().numpy()
        for b, L in enumerate(lens):
            n = L + i + 1
            rows = slice(b * H, (b + 1) * H)
            want, wl = O.mla_attention_fp64(bits(qn[rows]), bits(qp[rows]),
                                            bits(cs[b][:n])[None], bits(pes[b][:n])[None],
                                            scale)
            assert_close(o[rows], want, OUT_ATOL, OUT_RTOL, f"mla b={b} i={i}")
            assert_close(l[rows], wl, LSE_ATOL, LSE_RTOL, f"mla lse b={b} i={i}")
        o2, l2 = ops.mla_decode_partial(qn.to(DEV), qp.to(DEV), lat, pt, len_out, scale,
                                        max(lens) + i + 1, wg)
        torch.cuda.synchronize()
        assert torch.equal(o2.cpu(), out.cpu()) and torch.equal(l2.cpu(), lse.cpu())
    got = O.gather_paged(bits(lat), pt.cpu().numpy(), total)
    for b in range(B):
        assert np.array_equal(got[b], np.concatenate([bits(cs[b]), bits(pes[b])], 1)), b


def test_workspace_shared_across_shapes():
    # one workspace serves GQA and MLA calls of different row counts in turn
    _say("workspace shared across shapes")
    _gqa_check([900, 700], Hkv=2, G=4, wg=9, seed=51, port_check=False)
    _mla_check([700, 650, 600], wg=11, seed=52)
    _gqa_check([800] * 12, Hkv=8, G=4, wg=300, seed=53, port_check=False)
    _mla_check([300], wg=5, seed=54)
    _gqa_check([1000] * 3, Hkv=8, G=8, wg=200, seed=55, port_check=False)


# ---------------------------------------------------------------------------
# deferred-combine step + merge_split


def _host_partial(fmt, rows, Dv, seed):
    """A host partial in format fmt plus its (out, lse) in float64."""
    rng = np.random.default_rng(seed)
    ob = rng.standard_normal((rows, Dv)).astype(np.float32)
    mb = (rng.standard_normal(rows) * 2 + 3).astype(np.float32)
    sb = rng.uniform(1, 40, rows).astype(np.float32)
    sb[1] = 0.0
    mb[1] = -np.inf  # one row without host tokens
    if fmt == ops.PARTIAL_LSE_F32:
        lb = np.where(sb > 0, mb + np.log(np.where(sb > 0, sb, 1)), -np.inf).astype(np.float32)
        dev = (torch.from_numpy(ob).to(DEV), torch.from_numpy(lb).to(DEV))
        return dev, np.where(sb[:, None] > 0, ob, 0), lb
    if fmt == ops.TRIPLE_UNNORM_F32:
        ou = np.where(sb[:, None] > 0, ob * sb[:, None], 0).astype(np.float32)
        dev = tuple(torch.from_numpy(x).to(DEV) for x in (ou, mb, sb))
        o, l = O.triple_to_partial(ou, mb, sb, normalized=False)
        return dev, o, l
    ob16, mb16, sb16 = (torch.from_numpy(x).to(torch.bfloat16) for x in (ob, mb, sb))
    dev = tuple(x.to(DEV) for x in (ob16, mb16, sb16))
    o, l = O.triple_to_partial(ob16.float().numpy(), mb16.float().numpy(),
                               sb16.float().numpy(), normalized=True)
    return dev, o, l


@pytest.mark.parametrize("wg", [0, 3, 64])
@pytest.mark.parametrize("fmt", [None, ops.PARTIAL_LSE_F32, ops.TRIPLE_UNNORM_F32,
                                 ops.TRIPLE_NORM_BF16])
def test_gqa_split_step_and_merge(wg, fmt):
    _say(f"gqa split step wg={wg} fmt={fmt}")
    Hkv, G, D, PS = 8, 4, 128, 64
    lens = [1, 40, 700, 1500]
    B = len(lens)
    total = [L + 1 for L in lens]
    k_pages, v_pages, pt, gl, ks, vs = gqa_pool(total, Hkv, D, PS, seed=61)
    lens2 = torch.zeros((2, B), dtype=torch.int32, device=DEV)
    lens2[0] = torch.tensor(lens, dtype=torch.int32)
    q = bf16_randn((B, Hkv * G, D), 62)
    k_new = torch.stack([k[:, L:L + 1] for k, L in zip(ks, lens)]).to(DEV).contiguous()
    v_new = torch.stack([v[:, L:L + 1] for v, L in zip(vs, lens)]).to(DEV).contiguous()
    scale = D ** -0.5
    step = ops.gqa_append_decode_split(q.to(DEV), k_new, v_new, k_pages, v_pages, pt,
                                       lens2[0], lens2[1], scale, max(lens) + 1, wg)
    rows = B * Hkv * G
    if fmt is None:
        out, lse = ops.merge_split(step, None, out_dtype=torch.float32)
        host_o, host_l = np.zeros((rows, D)), np.full(rows, -np.inf)
    else:
        hb, host_o, host_l = _host_partial(fmt, rows, D, 63)
        out, lse = ops.merge_split(step, hb, fmt, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert lens2[1].cpu().tolist() == total
    qb = bits(q).reshape(B, Hkv, G, D)
    got, gl_ = out.cpu().numpy().reshape(B, Hkv, G, D), lse.cpu().numpy().reshape(B, Hkv, G)
    ho, hl = host_o.reshape(B, Hkv, G, D), host_l.reshape(B, Hkv, G)
    for b in range(B):
        g_o, g_l = O.gqa_attention_fp64(qb[b], bits(ks[b]), bits(vs[b]), scale)
        want, wl = O.merge_fp64(g_o, g_l, ho[b], hl[b])
        assert_close(got[b], want, OUT_ATOL, OUT_RTOL, f"split merged b={b}")
        assert_close(gl_[b], wl, LSE_ATOL, LSE_RTOL, f"split merged lse b={b}")
    # same result as the one-launch step followed by ws_lse_merge (fp32 out)
    lens3 = torch.tensor(lens, dtype=torch.int32, device=DEV)
    o1, l1 = ops.gqa_append_decode_partial(q.to(DEV), k_new, v_new, k_pages, v_pages, pt,
                                           lens3, None, scale, max(lens) + 1, wg)
    if fmt is None:
        o2, l2 = o1.view(rows, D), l1.view(rows)
    else:
        o2, l2 = ops.lse_merge(o1.view(rows, D), l1.view(rows), hb, fmt,
                               out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), o2.cpu().numpy(), 1e-5, 1e-5, "split vs one-launch")
    assert_close(lse.cpu().numpy(), l2.cpu().numpy(), 1e-5, 1e-5, "split vs one-launch lse")


@pytest.mark.parametrize("wg", [0, 5])
def test_mla_split_step_and_merge(wg):
    _say(f"mla split step wg={wg}")
    H, PS = 16, 64
    lens = [3, 300, 2000]
    B = len(lens)
    total = [L + 1 for L in lens]
    lat, pt, gl, cs, pes = mla_pool(total, PS, seed=71)
    lens2 = torch.zeros((2, B), dtype=torch.int32, device=DEV)
    lens2[0] = torch.tensor(lens, dtype=torch.int32)
    qn = bf16_randn((B * H, 512), 72, 0.5)
    qp = bf16_randn((B * H, 64), 73, 0.5)
    kv = torch.stack([torch.cat([c[L:L + 1], pe[L:L + 1]], 1)
                      for c, pe, L in zip(cs, pes, lens)]).to(DEV)
    scale = 192 ** -0.5
    step = ops.mla_append_decode_split(qn.to(DEV), qp.to(DEV), kv[..., :512], kv[..., 512:],
                                       lat, pt, lens2[0], lens2[1], scale, max(lens) + 1, wg)
    rows = B * H
    hb, host_o, host_l = _host_partial(ops.TRIPLE_UNNORM_F32, rows, 512, 74)
    out, lse = ops.merge_split(step, hb, ops.TRIPLE_UNNORM_F32, out_dtype=torch.float32)
    torch.cuda.synchronize()
    got, gl_ = out.cpu().numpy(), lse.cpu().numpy()
    for b in range(B):
        r = slice(b * H, (b + 1) * H)
        g_o, g_l = O.mla_attention_fp64(bits(qn[r]), bits(qp[r]), bits(cs[b])[None],
                                        bits(pes[b])[None], scale)
        want, wl = O.merge_fp64(g_o, g_l, host_o[r], host_l[r])
        assert_close(got[r], want, OUT_ATOL, OUT_RTOL, f"mla split merged b={b}")
        assert_close(gl_[r], wl, LSE_ATOL, LSE_RTOL, f"mla split merged lse b={b}")


@pytest.mark.parametrize("wg", [0, 5, 40])
@pytest.mark.parametrize("fmt", [None, ops.PARTIAL_LSE_F32, ops.TRIPLE_UNNORM_F32,
                                 ops.TRIPLE_NORM_BF16])
def test_mla_merge_split_uv_epilogue(wg, fmt):
    """Merge + W_UV in one launch: its latent equals ws_merge_split's bit for
    bit; out_v equals that latent times W_UV^T (fp64) within bf16 rounding,
    and the fp64 merged attention times W_UV^T within the parity bar."""
    _say(f"mla merge_split_uv wg={wg} fmt={fmt}")
    H, PS, Dout = 16, 64, 128
    lens = [0, 37, 700, 1500]
    B = len(lens)
    total = [L + 1 for L in lens]
    lat, pt, gl, cs, pes = mla_pool(total, PS, seed=81)
    lens2 = torch.zeros((2, B), dtype=torch.int32, device=DEV)
    lens2[0] = torch.tensor(lens, dtype=torch.int32)
    qn = bf16_randn((B * H, 512), 82, 0.5)
    qp = bf16_randn((B * H, 64), 83, 0.5)
    kv = torch.stack([torch.cat([c[L:L + 1], pe[L:L + 1]], 1)
                      for c, pe, L in zip(cs, pes, lens)]).to(DEV)
    w_uv = bf16_randn((H, Dout, 512), 84, 0.05)
    scale = 192 ** -0.5
    step = ops.mla_append_decode_split(qn.to(DEV), qp.to(DEV), kv[..., :512], kv[..., 512:],
                                       lat, pt, lens2[0], lens2[1], scale, max(lens) + 1, wg)
    rows = B * H
    if fmt is None:
        hb, host_o, host_l = None, np.zeros((rows, 512)), np.full(rows, -np.inf)
        f = ops.PARTIAL_LSE_F32
    else:
        hb, host_o, host_l = _host_partial(fmt, rows, 512, 85)
        f = fmt
    ref_lat, ref_lse = ops.merge_split(step, hb, f)
    out_v, latent, lse = ops.merge_split_uv(step, w_uv.to(DEV), hb, f, want_latent=True,
                                            want_lse=True)
    torch.cuda.synchronize()
    assert np.array_equal(bits(latent), bits(ref_lat)), "latent differs from ws_merge_split"
    assert np.array_equal(lse.cpu().numpy(), ref_lse.cpu().numpy())
    wv = bits(w_uv).view(np.uint16)
    w64 = O.as_f64(wv)                                         # [H, Dout, 512]
    lat64 = O.as_f64(bits(ref_lat)).reshape(B, H, 512)
    want_from_latent = np.einsum("bhk,hvk->bhv", lat64, w64).reshape(B, H * Dout)
    got = out_v.float().cpu().numpy()
    # fp32 accumulation of 512 products, then one bf16 rounding
    assert_close(got, want_from_latent, 2e-3, 8e-3, "out_v vs latent @ W_UV^T")
    for b in range(B):
        r = slice(b * H, (b + 1) * H)
        g_o, g_l = O.mla_attention_fp64(bits(qn[r]), bits(qp[r]), bits(cs[b])[None],
                                        bits(pes[b])[None], scale)
        m_o, _ = O.merge_fp64(g_o, g_l, host_o[r], host_l[r])
        want = np.einsum("hk,hvk->hv", m_o, w64).reshape(H * Dout)
        assert_close(got[b], want, OUT_ATOL, OUT_RTOL, f"out_v b={b} vs fp64 attention")
