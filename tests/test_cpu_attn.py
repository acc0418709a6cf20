"""The reference CPU extension's surface (scope_amd/cpu_attn.py) on the host
kernels, against the fp64 oracle and the oracle's C restatement of the
reference kernel, in the reference's own output conventions.

Bars: float32 outputs within 2e-2 (bf16 inputs) or 1e-4 (float32 inputs) of
the fp64 closed form; the LSE carried by (max, sum) within 1e-3, or 1e-2
when max and sum are bf16 (the reference's bf16 triple carries about that
much itself).  The key property is the drop-in one: triples of two halves of
a sequence, merged by the reference's _pairwise_merge formula and
normalised, equal attention over the whole sequence.
"""
import numpy as np
import pytest
import torch

from helpers import LSE_ATOL, LSE_RTOL, OUT_ATOL, OUT_RTOL, assert_close, bf16_randn, bits
from oracle import attn_np as O
from scope_amd import cpu_attn as X
from scope_amd import host

pytestmark = pytest.mark.skipif(not host.isa_supported(), reason="CPU lacks AVX-512 BF16")

BF16_LSE_TOL = 1e-2
F32_TOL = 1e-4


def _f32(shape, seed):
    g = torch.Generator(device="cpu").manual_seed(seed)
    return torch.randn(shape, generator=g, dtype=torch.float32)


def _np(t):
    return bits(t) if t.dtype == torch.bfloat16 else t.numpy()


def _lse(m, s):
    m = m.float().numpy()
    s = s.float().numpy()
    with np.errstate(divide="ignore"):
        return m + np.log(s)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_fused_cpu_attn_conventions(dtype):
    N, G, D, S = 6, 4, 128, 333
    q = (bf16_randn((N, G, D), 1) if dtype == torch.bfloat16 else _f32((N, G, D), 1))
    k = (bf16_randn((N, S, D), 2) if dtype == torch.bfloat16 else _f32((N, S, D), 2))
    v = (bf16_randn((N, S, D), 3) if dtype == torch.bfloat16 else _f32((N, S, D), 3))
    scale = D ** -0.5
    o, m, s = X.fused_cpu_attn(q, k, v, scale)
    assert o.dtype == m.dtype == s.dtype == dtype
    assert tuple(o.shape) == (N, G, D) and tuple(m.shape) == tuple(s.shape) == (N, G, 1)
    ow, lw = O.gqa_attention_fp64(_np(q), _np(k), _np(v), scale)
    tol = (OUT_ATOL, BF16_LSE_TOL) if dtype == torch.bfloat16 else (F32_TOL, F32_TOL)
    assert_close(o.float().numpy(), ow, tol[0], tol[0], "out (normalised)")
    assert_close(_lse(m, s)[..., 0], lw, tol[1], tol[1], "max + log(sum)")
    if dtype == torch.float32:
        o2, m2, s2 = X.fused_cpu_attn_fp32(q, k, v, scale)
        assert torch.equal(o, o2) and torch.equal(m, m2) and torch.equal(s, s2)


def test_fused_cpu_attn_matches_the_c_restatement():
    """The normalised out of fused_cpu_attn and the oracle's C port of the
    reference kernel (the same contract) on the same bf16 inputs."""
    from oracle import port
    N, G, D, S = 4, 8, 128, 700
    q, k, v = bf16_randn((N, G, D), 4), bf16_randn((N, S, D), 5), bf16_randn((N, S, D), 6)
    o, m, s = X.fused_cpu_attn(q, k, v, 0.088)
    po, pm, ps = port.cpu_attn(bits(q), bits(k), bits(v), 0.088, normalize=True, n_threads=3)
    assert_close(o.float().numpy(), po, OUT_ATOL, OUT_RTOL, "out vs C port")
    assert_close(_lse(m, s), pm + np.log(ps), BF16_LSE_TOL, BF16_LSE_TOL, "lse vs C port")


def test_fused_cpu_attn_mla_separate_widths_unnormalised():
    N, G, Dk, Dv, S = 16, 1, 192, 128, 257
    q, k, v = bf16_randn((N, G, Dk), 7), bf16_randn((N, S, Dk), 8), bf16_randn((N, S, Dv), 9)
    scale = 192 ** -0.5
    o, m, s = X.fused_cpu_attn_mla(q, k, v, scale)
    assert o.dtype == m.dtype == s.dtype == torch.float32 and tuple(o.shape) == (N, G, Dv)
    ow, lw = O.gqa_attention_fp64(bits(q), bits(k), bits(v), scale)
    assert_close((o / s).numpy(), ow, OUT_ATOL, OUT_RTOL, "out / sum")
    assert_close(_lse(m, s)[..., 0], lw, LSE_ATOL, LSE_RTOL, "max + log(sum)")


def test_fused_cpu_attn_mla_compressed():
    B, H, S = 3, 16, 411
    qp_, qr = bf16_randn((B * H, 512), 10, 0.5), bf16_randn((B * H, 64), 11, 0.5)
    c, pe = bf16_randn((B, S, 512), 12, 0.5), bf16_randn((B, S, 64), 13, 0.5)
    scale = 192 ** -0.5
    o, m, s = X.fused_cpu_attn_mla_compressed(qp_, qr, c, pe, scale)
    assert tuple(o.shape) == (B * H, 512) and tuple(m.shape) == tuple(s.shape) == (B * H,)
    for b in range(B):
        h = slice(b * H, (b + 1) * H)
        ow, lw = O.mla_attention_fp64(bits(qp_[h]), bits(qr[h]), bits(c[b:b + 1]),
                                      bits(pe[b:b + 1]), scale)
        assert_close((o[h] / s[h, None]).numpy(), ow, OUT_ATOL, OUT_RTOL, f"out b={b}")
        assert_close(_lse(m[h], s[h]), lw, LSE_ATOL, LSE_RTOL, f"lse b={b}")


@pytest.mark.parametrize("fn", ["fused_cpu_attn", "fused_cpu_attn_mla", "compressed"])
def test_triples_of_two_halves_merge_to_the_whole(fn):
    """The reference's _pairwise_merge (roofline/bench_resident_kv.py:141-148)
    over this module's triples of two token ranges, then out / sum, is
    attention over the whole range: the property the reference's callers rely
    on."""
    S, cut, scale = 500, 217, 0.07
    if fn == "compressed":
        B, H = 2, 16
        qp_, qr = bf16_randn((B * H, 512), 20, 0.5), bf16_randn((B * H, 64), 21, 0.5)
        c, pe = bf16_randn((B, S, 512), 22, 0.5), bf16_randn((B, S, 64), 23, 0.5)
        t1 = X.fused_cpu_attn_mla_compressed(qp_, qr, c[:, :cut].contiguous(),
                                             pe[:, :cut].contiguous(), scale)
        t2 = X.fused_cpu_attn_mla_compressed(qp_, qr, c[:, cut:].contiguous(),
                                             pe[:, cut:].contiguous(), scale)
        o1, m1, s1 = (t1[0].numpy(), t1[1].numpy()[:, None], t1[2].numpy()[:, None])
        o2, m2, s2 = (t2[0].numpy(), t2[1].numpy()[:, None], t2[2].numpy()[:, None])
        want = np.concatenate([O.mla_attention_fp64(
            bits(qp_[b * H:(b + 1) * H]), bits(qr[b * H:(b + 1) * H]), bits(c[b:b + 1]),
            bits(pe[b:b + 1]), scale)[0] for b in range(B)])
    else:
        N, G, D = 4, 4, 128
        q, k, v = bf16_randn((N, G, D), 24), bf16_randn((N, S, D), 25), bf16_randn((N, S, D), 26)
        f = getattr(X, fn)
        t1 = [x.float().numpy() for x in f(q, k[:, :cut], v[:, :cut], scale)]
        t2 = [x.float().numpy() for x in f(q, k[:, cut:], v[:, cut:], scale)]
        if fn == "fused_cpu_attn":  # normalised: un-normalise as system/mixoffload.py:1334
            t1[0], t2[0] = t1[0] * t1[2], t2[0] * t2[2]
        o1, m1, s1 = t1
        o2, m2, s2 = t2
        want = O.gqa_attention_fp64(bits(q), bits(k), bits(v), scale)[0]
    o, _, s = O.pairwise_merge_triple(o1, m1, s1, o2, m2, s2)
    assert_close(o / s, want, OUT_ATOL, OUT_RTOL, f"{fn}: merged halves")


def test_strided_rows_read_in_place():
    """k / v rows taken from longer buffers (the reference's `[:, :S]` views
    of its pinned caches) give the same result as contiguous copies."""
    N, G, D, cap, S = 3, 4, 128, 96, 70
    q = bf16_randn((N, G, D), 30)
    kb, vb = bf16_randn((N, cap, D), 31), bf16_randn((N, cap, D), 32)
    a = X.fused_cpu_attn(q, kb[:, :S], vb[:, :S], 0.1)
    b = X.fused_cpu_attn(q, kb[:, :S].contiguous(), vb[:, :S].contiguous(), 0.1)
    for x, y in zip(a, b):
        assert torch.equal(x, y)


def test_empty_range_is_the_merge_identity_and_threads():
    q, k = bf16_randn((2, 4, 128), 40), bf16_randn((2, 0, 128), 41)
    o, m, s = X.fused_cpu_attn_mla(q, k, k, 0.1)
    assert torch.all(o == 0) and torch.all(torch.isneginf(m)) and torch.all(s == 0)
    o, m, s = X.fused_cpu_attn_mla_compressed(
        bf16_randn((16, 512), 44), bf16_randn((16, 64), 45), bf16_randn((1, 0, 512), 46),
        bf16_randn((1, 0, 64), 47), 0.1)
    assert tuple(o.shape) == (16, 512) and torch.all(o == 0) and torch.all(s == 0)
    X.set_num_threads(3)
    try:
        assert X.get_num_threads() == 3
        q, k = bf16_randn((2, 4, 128), 42), bf16_randn((2, 50, 128), 43)
        o3 = X.fused_cpu_attn(q, k, k, 0.1)[0]
        X.set_num_threads(1)
        o1 = X.fused_cpu_attn(q, k, k, 0.1)[0]
        np.testing.assert_allclose(o3.float().numpy(), o1.float().numpy(), atol=1e-2)
    finally:
        X._threads = 0
    with pytest.raises(ValueError):
        X.fused_cpu_attn_fp32(q, k, k, 0.1)      # bf16 into the fp32 entry
    with pytest.raises(ValueError):
        X.fused_cpu_attn_mla(q.float(), k.float(), k.float(), 0.1)


def test_reference_self_test_shape_fp32():
    """The reference's own check of fused_cpu_attn's float32 path
    (kernel/build.py:28-64: seed 42, B_kv 512, G 4, D 128, S 3072, against a
    1024-token blocked online softmax in torch), at its full shape, through
    this module.  The reference prints the differences without a threshold;
    here out is within 1e-4 and the LSE carried by (max, sum) within 1e-5."""
    torch.manual_seed(42)
    B, G, D, S = 512, 4, 128, 3072
    q = torch.randn(B, G, D); k = torch.randn(B, S, D); v = torch.randn(B, S, D)
    scale = D ** -0.5
    out_acc = torch.zeros(B, G, D); m_acc = torch.full((B, G, 1), float("-inf"))
    s_acc = torch.zeros(B, G, 1)
    for s0 in range(0, S, 1024):
        sc = torch.bmm(q, k[:, s0:s0 + 1024].transpose(-2, -1)) * scale
        mb = sc.amax(-1, keepdim=True)
        eb = torch.exp(sc - mb)
        mn = torch.max(m_acc, mb)
        wo, wn = torch.exp(m_acc - mn), torch.exp(mb - mn)
        s_acc = wo * s_acc + wn * eb.sum(-1, keepdim=True)
        out_acc = wo * out_acc + wn * torch.bmm(eb, v[:, s0:s0 + 1024])
        m_acc = mn
    ref_out = (out_acc / s_acc).numpy()
    ref_lse = (m_acc + torch.log(s_acc)).numpy()
    o, m, s = X.fused_cpu_attn(q, k, v, scale)
    np.testing.assert_allclose(o.numpy(), ref_out, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(_lse(m, s), ref_lse, rtol=0, atol=1e-5)
