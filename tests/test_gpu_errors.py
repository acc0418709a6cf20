"""Bad page ids and lengths are errors the caller sees, never clamped reads.

A page id outside [0, num_pages) that a sequence's length reaches, or a length
outside [0, capacity - 1] for a fused step (negative, or no room for the new
token), makes that sequence's outputs and LSE NaN through every later merge;
its fused append is skipped and an invalid length becomes -1 in len_out.  A
multi-token append is all or nothing per sequence: with a bad slot in its
range nothing is written and the length becomes -1.  The other sequences of
the call are unaffected.  The kernels read clamped page ids, so every access
stays inside the pools.
"""
import numpy as np
import pytest
import torch

from oracle import attn_np as O
from scope_amd import ops
from tests.gpu_pool import gqa_pool, mla_pool, page_layout
from tests.helpers import OUT_ATOL, OUT_RTOL, assert_close, bf16_randn, bits

pytestmark = pytest.mark.gpu
DEV = "cuda"
PS = 64


def _say(msg):
    print(msg, flush=True)


def _gqa_case(lens, Hkv=4, G=4, D=128, seed=41):
    """Pools for lens + 1 tokens (room for the appended one), lengths set to lens."""
    k_pages, v_pages, pt, gl, ks, vs = gqa_pool([L + 1 for L in lens], Hkv, D, PS, seed)
    gl.copy_(torch.tensor(lens, dtype=torch.int32, device=DEV))
    B = len(lens)
    q = bf16_randn((B, Hkv * G, D), seed + 1).to(DEV)
    k_new = torch.stack([k[:, -1:] for k in ks]).to(DEV)
    v_new = torch.stack([v[:, -1:] for v in vs]).to(DEV)
    return k_pages, v_pages, pt, gl, ks, vs, q, k_new, v_new


@pytest.mark.parametrize("split", [False, True])
def test_gqa_bad_page_id_poisons_only_its_sequence(split):
    lens = [700, 300, 1000]
    _say(f"gqa bad page id, split={split}")
    k_pages, v_pages, pt, gl, ks, vs, q, k_new, v_new = _gqa_case(lens)
    pt[1, 2] = k_pages.shape[0] + 5  # sequence 1's third page: outside the pool
    before = bits(k_pages)
    len_out = torch.zeros_like(gl)
    scale = 128 ** -0.5
    if split:
        st = ops.gqa_append_decode_split(q, k_new, v_new, k_pages, v_pages, pt, gl, len_out,
                                         scale, max(lens) + 1)
        out, lse = ops.merge_split(st, None, out_dtype=torch.float32)
        out = out.view(q.shape)
        lse = lse.view(q.shape[:2])
    else:
        out, lse = ops.gqa_append_decode_partial(q, k_new, v_new, k_pages, v_pages, pt, gl,
                                                 len_out, scale, max(lens) + 1)
    torch.cuda.synchronize()
    o, l = out.cpu().numpy(), lse.cpu().numpy()
    assert np.isnan(o[1]).all() and np.isnan(l[1]).all()
    assert len_out.cpu().tolist() == [L + 1 for L in lens]
    qb = bits(q).reshape(3, 4, 4, 128)
    for b in (0, 2):
        want, _ = O.gqa_attention_fp64(qb[b], bits(ks[b]), bits(vs[b]), scale)
        assert_close(o[b].reshape(4, 4, 128), want, OUT_ATOL, OUT_RTOL, f"b={b}")
    # the bad sequence's new token went to its (valid) last page; nothing was
    # written anywhere else
    after = bits(k_pages)
    slot_pages = {int(pt[b, lens[b] // PS]) for b in range(3)}
    diff_pages = set(np.argwhere((after != before).any(axis=(1, 2, 3))).ravel().tolist())
    assert diff_pages <= slot_pages


def test_gqa_length_without_room_is_poisoned_not_clamped():
    lens = [127, 300, 60]
    _say("gqa length at capacity")
    k_pages, v_pages, pt, gl, ks, vs, q, k_new, v_new = _gqa_case(lens)
    cap = PS * pt.shape[1]
    gl[0] = cap  # no room for the appended token
    gl[2] = -7
    before = bits(k_pages)
    len_out = torch.zeros_like(gl)
    out, lse = ops.gqa_append_decode_partial(q, k_new, v_new, k_pages, v_pages, pt, gl, len_out,
                                             128 ** -0.5, cap)
    torch.cuda.synchronize()
    o, l = out.cpu().numpy(), lse.cpu().numpy()
    assert np.isnan(o[0]).all() and np.isnan(l[0]).all()
    assert np.isnan(o[2]).all() and np.isnan(l[2]).all()
    assert np.isfinite(o[1]).all() and np.isfinite(l[1]).all()
    assert len_out.cpu().tolist() == [-1, 301, -1]
    after = bits(k_pages)
    for b in (0, 2):  # neither sequence's pages were written
        for p in pt[b].cpu().tolist():
            if p >= 0:
                assert np.array_equal(after[p], before[p]), (b, p)
    # -1 stays an error for the next, non-fused call
    out2, lse2 = ops.gqa_decode_partial(q, k_pages, v_pages, pt, len_out, 128 ** -0.5, cap)
    torch.cuda.synchronize()
    assert np.isnan(out2.cpu().numpy()[[0, 2]]).all()
    assert np.isfinite(out2.cpu().numpy()[1]).all()


@pytest.mark.parametrize("H,bad_new_page", [(16, False), (128, False), (128, True)])
def test_mla_bad_page_and_length_are_poisoned(H, bad_new_page):
    """A page id outside the pool poisons its sequence (NaN), an invalid
    length its own; the other sequence is exact.  128 heads run the one-pass
    kernel; with bad_new_page the appended token's own page id is bad, and
    nothing is written where the clamped id points."""
    lens = [500, 200, 90]
    _say(f"mla bad page id + bad length, H={H}, bad_new_page={bad_new_page}")
    lat, pt, gl, cs, pes = mla_pool([L + 1 for L in lens], PS, seed=43)
    gl.copy_(torch.tensor(lens, dtype=torch.int32, device=DEV))
    pt[0, 3] = -3
    if bad_new_page:
        pt[0, lens[0] // PS] = -5  # clamped to pool page 0
    before = bits(lat[0, lens[0] % PS])
    gl[2] = 10 ** 6
    B = 3
    qn = bf16_randn((B * H, 512), 44, 0.5).to(DEV)
    qp = bf16_randn((B * H, 64), 45, 0.5).to(DEV)
    c_new = torch.stack([c[-1:] for c in cs]).to(DEV)
    pe_new = torch.stack([p[-1:] for p in pes]).to(DEV)
    len_out = torch.zeros_like(gl)
    st = ops.mla_append_decode_split(qn, qp, c_new, pe_new, lat, pt, gl, len_out, 192 ** -0.5,
                                     max(lens) + 1)
    host = (torch.zeros((B * H, 512), device=DEV), torch.full((B * H,), float("-inf"),
                                                             device=DEV))
    out, lse = ops.merge_split(st, host, ops.PARTIAL_LSE_F32, out_dtype=torch.float32)
    torch.cuda.synchronize()
    o, l = out.cpu().numpy(), lse.cpu().numpy()
    assert np.isnan(o[:H]).all() and np.isnan(l[:H]).all()
    assert np.isnan(o[2 * H:]).all() and np.isnan(l[2 * H:]).all()
    assert len_out.cpu().tolist() == [501, 201, -1]
    full = np.concatenate([bits(cs[1]), bits(pes[1])], 1)
    want, _ = O.mla_attention_fp64(bits(qn[H:2 * H]), bits(qp[H:2 * H]), full[None, :, :512],
                                   full[None, :, 512:], 192 ** -0.5)
    assert_close(o[H:2 * H], want, OUT_ATOL, OUT_RTOL, "b=1")
    if bad_new_page:  # the clamped page's slot kept its contents
        assert np.array_equal(bits(lat[0, lens[0] % PS]), before)


@pytest.mark.parametrize("n_new", [1, 40])  # 40 tokens: three chunks + the length kernel
def test_multi_token_append_is_all_or_nothing(n_new):
    _say(f"kv_append with a bad page, n_new={n_new}")
    B, Hkv, D = 3, 8, 128
    table, num_pages = page_layout([200] * B, PS, seed=47)
    pt = torch.from_numpy(table).to(DEV)
    pt[1, 1] = num_pages + 100  # sequence 1's slots 64..127 are in a bad page
    k_pages = torch.zeros((num_pages, Hkv, PS, D), dtype=torch.bfloat16, device=DEV)
    v_pages = torch.zeros_like(k_pages)
    gl = torch.tensor([60, 60, 60], dtype=torch.int32, device=DEV)
    k = bf16_randn((B, Hkv, n_new, D), 48).to(DEV)
    v = bf16_randn((B, Hkv, n_new, D), 49).to(DEV)
    ops.kv_append(k, v, k_pages, v_pages, pt, gl)
    torch.cuda.synchronize()
    reaches = 60 + n_new > 64
    assert gl.cpu().tolist() == [60 + n_new, -1 if reaches else 60 + n_new, 60 + n_new]
    kp = bits(k_pages)
    for b in range(B):
        p0 = int(table[b, 0])
        if b == 1 and reaches:
            assert not kp[[int(x) for x in table[1] if x >= 0]].any()  # nothing written
        else:
            assert np.array_equal(kp[p0, :, 60:min(64, 60 + n_new)],
                                  bits(k[b, :, :min(4, n_new)]))
    # the latent append follows the same rule
    lat = torch.zeros((num_pages, PS, 576), dtype=torch.bfloat16, device=DEV)
    gl2 = torch.tensor([60, 60, 60], dtype=torch.int32, device=DEV)
    c = bf16_randn((B, n_new, 512), 50).to(DEV)
    p = bf16_randn((B, n_new, 64), 51).to(DEV)
    ops.latent_append(c, p, lat, pt, gl2)
    torch.cuda.synchronize()
    assert gl2.cpu().tolist() == gl.cpu().tolist()
    lb = bits(lat)
    if reaches:
        assert not lb[[int(x) for x in table[1] if x >= 0]].any()


def test_merge_keeps_a_poisoned_partial_poisoned():
    rows, Dv = 6, 128
    og = torch.randn((rows, Dv), device=DEV)
    lg = torch.randn((rows,), device=DEV)
    og[2] = float("nan")
    lg[2] = float("nan")
    lg[4] = float("nan")
    hb = (torch.zeros((rows, Dv), device=DEV), torch.full((rows,), float("-inf"), device=DEV))
    out, lse = ops.lse_merge(og, lg, hb, ops.PARTIAL_LSE_F32, out_dtype=torch.float32)
    torch.cuda.synchronize()
    o, l = out.cpu().numpy(), lse.cpu().numpy()
    for r in (2, 4):
        assert np.isnan(o[r]).all() and np.isnan(l[r]), r
    for r in (0, 1, 3, 5):
        assert np.isfinite(o[r]).all() and np.isfinite(l[r]), r
