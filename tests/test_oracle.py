"""Pins the oracle (CPU only): closed forms vs brute force and special cases,
the fp32 / C restatements vs the fp64 closed forms, merge invariants, and the
reference's own checks (kernel/build.py:28-64 self-test shape,
roofline/bench_resident_kv.py:410-459 split/merge check)."""
import math

import numpy as np
import pytest
import torch

from oracle import attn_np as O
from oracle import port
from tests.helpers import assert_close, bf16_randn, bits

RNG = np.random.default_rng(1234)


# ---------------------------------------------------------------------------
# bf16 conversion


def test_bf16_round_trip_matches_torch():
    x = np.concatenate([RNG.standard_normal(4096).astype(np.float32) * 7,
                        np.array([0.0, -0.0, 1e-40, -1e-40, 3.0e38, 65504.0,
                                  1.00390625, 1.01171875, np.inf, -np.inf],
                                 np.float32)])
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(O.f32_to_bf16(x), want)
    # ties round to even: 1 + 2^-8 is halfway between two bf16 values
    assert O.f32_to_bf16(np.float32(1.00390625)) == 0x3F80
    assert np.array_equal(O.bf16_to_f32(want), torch.from_numpy(want.view(np.int16)).view(
        torch.bfloat16).float().numpy())


# ---------------------------------------------------------------------------
# fp64 closed forms


def brute_gqa(q, k, v, scale):
    N, G, _ = q.shape
    S, Dv = k.shape[1], v.shape[2]
    out = np.zeros((N, G, Dv))
    lse = np.zeros((N, G))
    for n in range(N):
        for g in range(G):
            sc = [sum(q[n, g, d] * k[n, t, d] for d in range(q.shape[2])) * scale
                  for t in range(S)]
            mx = max(sc)
            den = sum(math.exp(s - mx) for s in sc)
            lse[n, g] = mx + math.log(den)
            for d in range(Dv):
                out[n, g, d] = sum(math.exp(sc[t] - mx) * v[n, t, d] for t in range(S)) / den
    return out, lse


def test_gqa_fp64_vs_brute_force():
    q = RNG.standard_normal((2, 3, 4))
    k = RNG.standard_normal((2, 5, 4))
    v = RNG.standard_normal((2, 5, 6))
    out, lse = O.gqa_attention_fp64(q, k, v, 0.7)
    bo, bl = brute_gqa(q, k, v, 0.7)
    np.testing.assert_allclose(out, bo, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(lse, bl, rtol=1e-12, atol=1e-12)


def test_gqa_fp64_vs_torch_softmax():
    q = RNG.standard_normal((3, 8, 128))
    k = RNG.standard_normal((3, 300, 128))
    v = RNG.standard_normal((3, 300, 128))
    scale = 128 ** -0.5
    out, lse = O.gqa_attention_fp64(q, k, v, scale)
    sc = torch.from_numpy(q) @ torch.from_numpy(k).transpose(1, 2) * scale
    want = torch.softmax(sc, -1) @ torch.from_numpy(v)
    np.testing.assert_allclose(out, want.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(lse, torch.logsumexp(sc, -1).numpy(), rtol=1e-12)


def test_gqa_special_cases():
    scale = 0.5
    # one token: out = v, lse = score
    q = RNG.standard_normal((1, 2, 8)); k = RNG.standard_normal((1, 1, 8))
    v = RNG.standard_normal((1, 1, 8))
    out, lse = O.gqa_attention_fp64(q, k, v, scale)
    np.testing.assert_allclose(out[0], np.repeat(v[0], 2, 0), rtol=1e-14)
    np.testing.assert_allclose(lse[0], (q[0] @ k[0, 0]) * scale, rtol=1e-14)
    # zero keys: uniform weights -> mean of v, lse = log S
    k0 = np.zeros((1, 7, 8)); v7 = RNG.standard_normal((1, 7, 8))
    out, lse = O.gqa_attention_fp64(q, k0, v7, scale)
    np.testing.assert_allclose(out[0, 0], v7[0].mean(0), rtol=1e-13)
    np.testing.assert_allclose(lse, math.log(7), rtol=1e-14)
    # constant v: out = v whatever the scores
    vc = np.broadcast_to(RNG.standard_normal(8), (1, 7, 8)).copy()
    out, _ = O.gqa_attention_fp64(q, RNG.standard_normal((1, 7, 8)), vc, scale)
    np.testing.assert_allclose(out[0, 1], vc[0, 0], rtol=1e-12)
    # one dominant key
    kd = np.zeros((1, 7, 8)); kd[0, 3] = 100 * q[0, 0] / np.linalg.norm(q[0, 0])
    out, _ = O.gqa_attention_fp64(q[:, :1], kd, v7, 1.0)
    np.testing.assert_allclose(out[0, 0], v7[0, 3], rtol=1e-9)
    # empty partition
    out, lse = O.gqa_attention_fp64(q, np.zeros((1, 0, 8)), np.zeros((1, 0, 8)), scale)
    assert np.all(out == 0) and np.all(np.isneginf(lse))


def test_mla_fp64_equals_gqa_on_concatenated_latent():
    B, H, S = 2, 4, 33
    qn = RNG.standard_normal((B * H, 512)); qp = RNG.standard_normal((B * H, 64))
    c = RNG.standard_normal((B, S, 512)); pe = RNG.standard_normal((B, S, 64))
    out, lse = O.mla_attention_fp64(qn, qp, c, pe, 0.07)
    q = np.concatenate([qn, qp], 1).reshape(B, H, 576)
    k = np.concatenate([c, pe], 2)
    go, gl = O.gqa_attention_fp64(q, k, c, 0.07)
    np.testing.assert_allclose(out, go.reshape(B * H, 512), rtol=1e-12, atol=1e-13)
    np.testing.assert_allclose(lse, gl.reshape(B * H), rtol=1e-13)


def test_mla_fp64_brute_force_tiny():
    B, H, S = 1, 2, 3
    qn = RNG.standard_normal((B * H, 512)); qp = RNG.standard_normal((B * H, 64))
    c = RNG.standard_normal((B, S, 512)); pe = RNG.standard_normal((B, S, 64))
    out, lse = O.mla_attention_fp64(qn, qp, c, pe, 0.1)
    for h in range(H):
        sc = np.array([(qn[h] @ c[0, t] + qp[h] @ pe[0, t]) * 0.1 for t in range(S)])
        w = np.exp(sc - sc.max())
        np.testing.assert_allclose(out[h], (w[:, None] * c[0]).sum(0) / w.sum(), rtol=1e-12)
        np.testing.assert_allclose(lse[h], sc.max() + np.log(w.sum()), rtol=1e-13)


# ---------------------------------------------------------------------------
# merge


def test_merge_split_anywhere_equals_unsplit():
    q = RNG.standard_normal((2, 4, 16)); k = RNG.standard_normal((2, 50, 16))
    v = RNG.standard_normal((2, 50, 16))
    whole = O.gqa_attention_fp64(q, k, v, 0.25)
    for cut in (0, 1, 17, 49, 50):
        a = O.gqa_attention_fp64(q, k[:, :cut], v[:, :cut], 0.25)
        b = O.gqa_attention_fp64(q, k[:, cut:], v[:, cut:], 0.25)
        out, lse = O.merge_fp64(*a, *b)
        np.testing.assert_allclose(out, whole[0], rtol=1e-12, atol=1e-13)
        np.testing.assert_allclose(lse, whole[1], rtol=1e-13)


def test_merge_commutative_associative_identity():
    parts = [(RNG.standard_normal((3, 8)), RNG.standard_normal(3) * 5) for _ in range(3)]
    ab = O.merge_fp64(*parts[0], *parts[1])
    ba = O.merge_fp64(*parts[1], *parts[0])
    np.testing.assert_allclose(ab[0], ba[0], rtol=1e-14)
    left = O.merge_fp64(*ab, *parts[2])
    right = O.merge_fp64(*parts[0], *O.merge_fp64(*parts[1], *parts[2]))
    np.testing.assert_allclose(left[0], right[0], rtol=1e-12)
    np.testing.assert_allclose(left[1], right[1], rtol=1e-13)
    empty = (np.zeros((3, 8)), np.full(3, -np.inf))
    e = O.merge_fp64(*parts[0], *empty)
    np.testing.assert_allclose(e[0], parts[0][0], rtol=1e-15)
    np.testing.assert_allclose(e[1], parts[0][1], rtol=1e-15)
    ee = O.merge_fp64(*empty, *empty)
    assert np.all(ee[0] == 0) and np.all(np.isneginf(ee[1]))


def test_triple_conventions_match_reference_merge():
    # reference merge of unnormalised triples, then o / s, equals merge_fp64 of
    # the converted partials (roofline/bench_resident_kv.py:141-148, 348-350)
    q = RNG.standard_normal((2, 4, 16)); k = RNG.standard_normal((2, 40, 16))
    v = RNG.standard_normal((2, 40, 16))
    trip = []
    for sl in (slice(0, 13), slice(13, 40)):
        sc = np.einsum("ngd,nsd->ngs", q, k[:, sl]) * 0.3
        m = sc.max(-1, keepdims=True); e = np.exp(sc - m)
        trip.append((np.einsum("ngs,nsd->ngd", e, v[:, sl]), m, e.sum(-1, keepdims=True)))
    o, m, s = O.pairwise_merge_triple(*trip[0], *trip[1])
    ref = o / np.maximum(s, 1e-6)
    conv = [O.triple_to_partial(*t, normalized=False) for t in trip]
    out, lse = O.merge_fp64(*conv[0], *conv[1])
    np.testing.assert_allclose(out, ref, rtol=1e-12)
    np.testing.assert_allclose(lse, (m + np.log(s))[..., 0], rtol=1e-13)
    # normalised triple (fused_cpu_attn) converts to the same partial
    n0 = O.triple_to_partial(trip[0][0] / trip[0][2], trip[0][1], trip[0][2], normalized=True)
    np.testing.assert_allclose(n0[0], conv[0][0], rtol=1e-13)


# ---------------------------------------------------------------------------
# fp32 restatements vs fp64


def test_blocked_fp32_restatement_vs_fp64():
    q = RNG.standard_normal((3, 4, 128)).astype(np.float32)
    k = RNG.standard_normal((3, 777, 128)).astype(np.float32)
    v = RNG.standard_normal((3, 777, 128)).astype(np.float32)
    scale = 128 ** -0.5
    out, mx, sm = O.gqa_cpu_kernel_fp32(q, k, v, scale, n_threads=16)
    want, wl = O.gqa_attention_fp64(q, k, v, scale)
    np.testing.assert_allclose(out, want, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(mx[..., 0] + np.log(sm[..., 0]), wl, atol=1e-5)


def test_cpu_tile_len_rule():
    # kernel/cpu_attn.cpp:205-222: rows >= threads -> one tile; else >= 256,
    # multiple of 16 (unless the whole sequence is shorter)
    assert O.cpu_tile_len(4096, 32, 16) == 4096
    assert O.cpu_tile_len(4096, 4, 16) == 1024
    assert O.cpu_tile_len(300, 4, 16) == 256
    assert O.cpu_tile_len(100, 4, 16) == 100
    assert O.cpu_tile_len(1000, 15, 16) == 512


@pytest.mark.parametrize("dtype", ["bf16", "fp32"])
@pytest.mark.parametrize("threads", [1, 3, 8])
def test_c_port_gqa_vs_fp64(dtype, threads):
    N, G, D, S = 4, 8, 128, 1000
    q = bf16_randn((N, G, D), 11); k = bf16_randn((N, S, D), 12); v = bf16_randn((N, S, D), 13)
    qa, ka, va = (bits(t) for t in (q, k, v))
    if dtype == "fp32":
        qa, ka, va = (O.bf16_to_f32(a) for a in (qa, ka, va))
    out, mx, sm = port.cpu_attn(qa, ka, va, D ** -0.5, normalize=True, n_threads=threads)
    want, wl = O.gqa_attention_fp64(bits(q), bits(k), bits(v), D ** -0.5)
    np.testing.assert_allclose(out, want, rtol=1e-4, atol=2e-5)
    np.testing.assert_allclose(mx[..., 0] + np.log(sm[..., 0]), wl, atol=2e-5)
    # unnormalised (fused_cpu_attn_mla convention)
    o2, m2, s2 = port.cpu_attn(qa, ka, va, D ** -0.5, normalize=False, n_threads=threads)
    np.testing.assert_allclose(o2 / s2, want, rtol=1e-4, atol=2e-5)


def test_c_port_strided_rows_and_empty():
    # k/v rows addressed through strides (kernel/cpu_attn.cpp:598-601)
    big = bf16_randn((3, 700, 128), 21)
    k = bits(big)[:, 100:600]
    v = bits(bf16_randn((3, 700, 128), 22))[:, 50:550]
    q = bits(bf16_randn((3, 2, 128), 23))
    out, mx, sm = port.cpu_attn(q, k, v, 0.1, normalize=True, n_threads=4)
    want, _ = O.gqa_attention_fp64(q, np.ascontiguousarray(k), np.ascontiguousarray(v), 0.1)
    np.testing.assert_allclose(out, want, rtol=1e-4, atol=2e-5)
    out, mx, sm = port.cpu_attn(q, k[:, :0], v[:, :0], 0.1)
    assert np.all(out == 0) and np.all(np.isneginf(mx)) and np.all(sm == 0)


@pytest.mark.parametrize("threads", [1, 5, 16])
def test_c_port_mla_compressed_vs_fp64(threads):
    B, H, S = 2, 16, 700
    qn = bits(bf16_randn((B * H, 512), 31, 0.5)); qp = bits(bf16_randn((B * H, 64), 32, 0.5))
    c = bits(bf16_randn((B, S, 512), 33, 0.5)); pe = bits(bf16_randn((B, S, 64), 34, 0.5))
    scale = 192 ** -0.5
    o, mx, sm = port.cpu_attn_mla_compressed(qn, qp, c, pe, scale, n_threads=threads)
    want, wl = O.mla_attention_fp64(qn, qp, c, pe, scale)
    np.testing.assert_allclose(o / sm[:, None], want, rtol=1e-4, atol=2e-5)
    np.testing.assert_allclose(mx + np.log(sm), wl, atol=2e-5)


def test_reference_selftest_shape_blocked():
    # kernel/build.py:28-64 compares fused_cpu_attn (fp32) with a 1024-token
    # blocked online softmax; same structure at B_kv = 16 instead of 512.
    torch.manual_seed(42)
    B, G, D, S = 16, 4, 128, 3072
    q = torch.randn(B, G, D); k = torch.randn(B, S, D); v = torch.randn(B, S, D)
    scale = D ** -0.5
    out_acc = torch.zeros(B, G, D); m_acc = torch.full((B, G, 1), float("-inf"))
    s_acc = torch.zeros(B, G, 1)
    for s0 in range(0, S, 1024):
        sc = torch.bmm(q, k[:, s0:s0 + 1024].transpose(-2, -1)) * scale
        mb = sc.amax(-1, keepdim=True); eb = torch.exp(sc - mb)
        mn = torch.max(m_acc, mb); wo = torch.exp(m_acc - mn); wn = torch.exp(mb - mn)
        s_acc = wo * s_acc + wn * eb.sum(-1, keepdim=True)
        out_acc = wo * out_acc + wn * torch.bmm(eb, v[:, s0:s0 + 1024])
        m_acc = mn
    ref = (out_acc / s_acc).numpy()
    out, mx, sm = port.cpu_attn(q.numpy(), k.numpy(), v.numpy(), scale, n_threads=8)
    np.testing.assert_allclose(out, ref, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(mx, m_acc.numpy(), rtol=1e-6)
    np.testing.assert_allclose(sm, s_acc.numpy(), rtol=1e-4)


def test_reference_kvlen_split_merge_check():
    # roofline/bench_resident_kv.py:410-459 (kvlen mode): three token ranges
    # (streamed [0, gs), resident [gs, gs+n_res), CPU rest) merged pairwise
    # must match the whole at atol = rtol = 2e-2 after the bf16 cast.
    torch.manual_seed(0)
    B, kv, NH, G, D = 2, 4096, 4, 8, 128
    q = torch.randn(B * NH, G, D).to(torch.bfloat16)
    k = torch.randn(B * NH, kv, D).to(torch.bfloat16)
    v = torch.randn(B * NH, kv, D).to(torch.bfloat16)
    scale = D ** -0.5
    qb, kb, vb = bits(q), bits(k), bits(v)
    whole, _ = O.gqa_attention_fp64(qb, kb, vb, scale)
    gs = n_res = kv // 4
    parts = [O.gqa_attention_fp64(qb, kb[:, a:b], vb[:, a:b], scale)
             for a, b in ((0, gs), (gs, gs + n_res), (gs + n_res, kv))]
    m1 = O.merge_fp64(*parts[0], *parts[1])
    out, _ = O.merge_fp64(*m1, *parts[2])
    got = O.bf16_to_f32(O.f32_to_bf16(out.astype(np.float32)))
    ref = O.bf16_to_f32(O.f32_to_bf16(whole.astype(np.float32)))
    assert_close(got, ref, 2e-2, 2e-2, "kvlen split/merge")


# ---------------------------------------------------------------------------
# a planted mistake must fail the pins


def test_planted_mistakes_are_caught():
    q = RNG.standard_normal((2, 3, 8)); k = RNG.standard_normal((2, 9, 8))
    v = RNG.standard_normal((2, 9, 8))
    out, lse = O.gqa_attention_fp64(q, k, v, 0.5)
    bo, bl = brute_gqa(q, k, v, 0.5)
    # wrong scale, transposed operand, dropped max-subtraction term in the lse
    wrong = [O.gqa_attention_fp64(q, k, v, 0.25)[0],
             O.gqa_attention_fp64(q, k[:, ::-1], v, 0.5)[0]]
    for w in wrong:
        assert not np.allclose(w, bo, rtol=1e-6)
    assert not np.allclose(np.log(np.exp(lse) * 2), bl, rtol=1e-6)
