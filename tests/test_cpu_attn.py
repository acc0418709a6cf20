"""The reference CPU extension's surface (scope_amd/cpu_attn.py) on the host
kernels, against the fp64 oracle and the oracle's C restatement of the
reference kernel, in the reference's own output conventions.

Bars: float32 outputs within 2e-2 (bf16 inputs) or 1e-4 (float32 inputs) of
the fp64 closed form; the LSE carried by (max, sum) within 1e-3, or 1e-2
when max and sum are bf16 (the reference's bf16 triple carries about that
much itself); max and sum themselves within 1e-5 / 1e-4 relative of the C
restatement's and of fp64 brute force (one bf16 step when they are bf16).  The key property is the drop-in one: triples of two halves of
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


@pytest.mark.parametrize("D", [16, 48, 80, 112, 240])
def test_fused_cpu_attn_any_multiple_of_16_width(D):
    """Head widths with a last 16-column chunk (the reference kernel takes any
    multiple of 16, kernel/cpu_attn.cpp:583), bf16 inputs, against fp64 and
    the oracle's C restatement."""
    from oracle import port
    N, G, S = 3, 4, 149
    q, k, v = bf16_randn((N, G, D), 10 + D), bf16_randn((N, S, D), 11 + D), bf16_randn((N, S, D), 12 + D)
    scale = D ** -0.5
    o, m, s = X.fused_cpu_attn(q, k, v, scale)
    assert tuple(o.shape) == (N, G, D)
    ow, lw = O.gqa_attention_fp64(bits(q), bits(k), bits(v), scale)
    assert_close(o.float().numpy(), ow, OUT_ATOL, OUT_RTOL, f"out D={D}")
    assert_close(_lse(m, s)[..., 0], lw, BF16_LSE_TOL, BF16_LSE_TOL, f"max + log(sum) D={D}")
    po, pm, ps = port.cpu_attn(bits(q), bits(k), bits(v), scale, normalize=True, n_threads=2)
    assert_close(o.float().numpy(), po, OUT_ATOL, OUT_RTOL, f"out vs C port D={D}")


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


def _bf16_round(x):
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.bfloat16).float().numpy()


def _max_sum_fp64(qf, kf, scale):
    """Brute-force row max of q.k * scale and sum of exp(score - max), fp64:
    q [N, G, D], k [N, S, D]."""
    sc = np.einsum("ngd,nsd->ngs", qf.astype(np.float64), kf.astype(np.float64)) * scale
    mx = sc.max(-1)
    return mx, np.exp(sc - mx[..., None]).sum(-1)


@pytest.mark.parametrize("entry", ["fused_cpu_attn_bf16", "fused_cpu_attn_f32",
                                   "fused_cpu_attn_fp32", "fused_cpu_attn_mla",
                                   "fused_cpu_attn_mla_192"])
def test_max_and_sum_are_the_reference_kernels(entry):
    """The (max, sum) of every dense entry point are the reference kernel's
    own values (kernel/cpu_attn.cpp:540-567, 628-635), not an equivalent
    pair: against the oracle's C restatement of that kernel on the same
    inputs, and against fp64 brute force.  fp32 outputs: max to 1e-5 and sum
    to 1e-4 relative; bf16 outputs (fused_cpu_attn on bf16 inputs): each the
    C restatement's fp32 value rounded to bf16, within one bf16 step (the two
    fp32 values may straddle a rounding boundary).  The unnormalised out of
    fused_cpu_attn_mla is within the output bar of the C restatement's."""
    from oracle import port
    N, G, S = 5, 4, 613
    Dk, Dv = (192, 128) if entry == "fused_cpu_attn_mla_192" else (128, 128)
    f32 = entry in ("fused_cpu_attn_f32", "fused_cpu_attn_fp32")
    if f32:
        q, k, v = _f32((N, G, Dk), 50), _f32((N, S, Dk), 51), _f32((N, S, Dv), 52)
    else:
        q, k, v = bf16_randn((N, G, Dk), 50), bf16_randn((N, S, Dk), 51), bf16_randn((N, S, Dv), 52)
    scale = Dk ** -0.5
    normalize = entry.startswith("fused_cpu_attn_f") or entry == "fused_cpu_attn_bf16"
    fn = getattr(X, "fused_cpu_attn_mla" if entry.startswith("fused_cpu_attn_mla")
                 else ("fused_cpu_attn_fp32" if entry == "fused_cpu_attn_fp32"
                       else "fused_cpu_attn"))
    o, m, s = fn(q, k, v, scale)
    po, pm, ps = port.cpu_attn(_np(q), _np(k), _np(v), scale, normalize=normalize,
                               n_threads=3)
    qf = q.float().numpy()
    kf = k.float().numpy()
    bm, bs = _max_sum_fp64(qf, kf, scale)
    if entry == "fused_cpu_attn_bf16":
        assert m.dtype == s.dtype == torch.bfloat16
        for got, want, what in ((m, pm, "max"), (s, ps, "sum")):
            got = got.float().numpy()
            step = np.abs(_bf16_round(want)) * 2.0 ** -7
            assert np.all(np.abs(got - _bf16_round(want)) <= step), what
            assert np.mean(got == _bf16_round(want)) > 0.9, what
        assert_close(m.float().numpy()[..., 0], bm, 0, 2.0 ** -8, "max vs fp64")
        assert_close(s.float().numpy()[..., 0], bs, 0, 2.0 ** -7, "sum vs fp64")
        return
    assert m.dtype == s.dtype == torch.float32
    assert_close(m.numpy(), pm, 1e-5, 1e-5, "max vs C restatement")
    assert_close(s.numpy(), ps, 0, 1e-4, "sum vs C restatement")
    assert_close(m.numpy()[..., 0], bm, 1e-5, 1e-5, "max vs fp64")
    assert_close(s.numpy()[..., 0], bs, 0, 1e-4, "sum vs fp64")
    tol = 1e-4 if f32 else OUT_ATOL
    scale_o = 1.0 if normalize else np.abs(po).max()
    assert_close(o.numpy() / scale_o, po / scale_o, tol, tol, "out vs C restatement")


def test_max_and_sum_of_mla_compressed_are_the_reference_kernels():
    """fused_cpu_attn_mla_compressed's (max, sum) (kernel/cpu_attn.cpp:1001-1021)
    against the C restatement and fp64 brute force over the 576-wide score;
    the unnormalised out against the C restatement's."""
    from oracle import port
    B, H, S = 3, 16, 517
    qp_, qr = bf16_randn((B * H, 512), 60, 0.5), bf16_randn((B * H, 64), 61, 0.5)
    c, pe = bf16_randn((B, S, 512), 62, 0.5), bf16_randn((B, S, 64), 63, 0.5)
    scale = 192 ** -0.5
    o, m, s = X.fused_cpu_attn_mla_compressed(qp_, qr, c, pe, scale)
    po, pm, ps = port.cpu_attn_mla_compressed(bits(qp_), bits(qr), bits(c), bits(pe), scale,
                                              n_threads=3)
    assert_close(m.numpy(), pm, 1e-5, 1e-5, "max vs C restatement")
    assert_close(s.numpy(), ps, 0, 1e-4, "sum vs C restatement")
    qf = torch.cat([qp_, qr], 1).float().numpy().reshape(B, H, 576)
    kf = torch.cat([c, pe], 2).float().numpy()
    bm, bs = _max_sum_fp64(qf, kf, scale)
    assert_close(m.numpy(), bm.reshape(-1), 1e-5, 1e-5, "max vs fp64")
    assert_close(s.numpy(), bs.reshape(-1), 0, 1e-4, "sum vs fp64")
    mag = np.abs(po).max()
    assert_close(o.numpy() / mag, po / mag, OUT_ATOL, OUT_RTOL, "out vs C restatement")


def test_max_and_sum_planted_mistakes_fail():
    """The checks above catch a max kept in log2 units and a sum taken
    relative to a stale max: both planted in the oracle's brute force, on the
    CPU."""
    q, k = bf16_randn((2, 4, 128), 70), bf16_randn((2, 90, 128), 71)
    _, m, s = X.fused_cpu_attn_mla(q, k, k, 0.1)
    bm, bs = _max_sum_fp64(q.float().numpy(), k.float().numpy(), 0.1)
    with pytest.raises(AssertionError):
        assert_close(m.numpy()[..., 0], bm * 1.4426950408889634, 1e-5, 1e-5, "log2 max")
    with pytest.raises(AssertionError):
        assert_close(s.numpy()[..., 0], bs * np.exp(bm - (bm - 0.5)), 0, 1e-4, "stale max")


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
