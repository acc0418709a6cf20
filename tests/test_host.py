"""Host partial (libwshost.so, include/wshost.h) against the fp64 oracle.

CPU tests: the AVX-512 BF16 kernels run here.  Bar: outputs within 2e-2
abs/rel and LSE within 1e-3 of the closed form, on ragged batches (empty,
single-token, odd, non-multiple-of-32 lengths), every supported head_dim and
group size, thread counts that split rows at arbitrary block boundaries, and
large scores.  Error paths are checked on the host.
"""
import ctypes
import os
import re

import numpy as np
import pytest
import torch

from helpers import LSE_ATOL, LSE_RTOL, OUT_ATOL, OUT_RTOL, assert_close, bf16_randn, bits
from oracle import attn_np as O
from scope_amd import host

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "wshost.h")

needs_isa = pytest.mark.skipif(
    not (os.path.exists(host.LIB_PATH) and host.isa_supported()),
    reason="CPU lacks AVX-512 BF16")


def test_every_declared_symbol_is_exported():
    assert os.path.exists(host.LIB_PATH), "run __graft_entry__.build() first"
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    names = sorted(set(re.findall(r"\b(wh_\w+)\s*\(", text)))
    assert set(names) == set(host.EXPORTS), (names, host.EXPORTS)
    L = ctypes.CDLL(host.LIB_PATH)
    for n in names:
        assert hasattr(L, n), f"{n} not exported"
    assert host.lib().wh_version().decode().startswith("wshost")


def _gqa_case(B, Hkv, G, D, lens, cap, threads, seed, sigma=1.0):
    q = bf16_randn((B, Hkv * G, D), seed, sigma)
    k = bf16_randn((B * Hkv, cap, D), seed + 1)
    v = bf16_randn((B * Hkv, cap, D), seed + 2)
    scale = D ** -0.5
    out, lse = host.gqa_partial_dense(q, k, v, lens, scale, threads)
    for b in range(B):
        L = lens[b]
        rows = slice(b * Hkv, (b + 1) * Hkv)
        ow, lw = O.gqa_attention_fp64(bits(q[b]).reshape(Hkv, G, D), bits(k[rows, :L]),
                                      bits(v[rows, :L]), scale)
        assert_close(out[b].numpy().reshape(Hkv, G, D), ow, OUT_ATOL, OUT_RTOL, f"out b={b}")
        assert_close(lse[b].numpy().reshape(Hkv, G), lw, LSE_ATOL, LSE_RTOL, f"lse b={b}")
    return out, lse


GQA_CASES = [
    # B, Hkv, G, D, lens, cap, threads
    (1, 1, 1, 128, [1], 1, 1),
    (1, 1, 4, 128, [37], 40, 1),
    (2, 2, 4, 128, [100, 0], 128, 3),
    (3, 4, 8, 128, [1000, 33, 517], 1024, 8),
    (2, 8, 4, 128, [64, 65], 96, 16),       # Mixtral grouping, more threads than rows
    (2, 2, 16, 256, [200, 31], 256, 4),
    (2, 2, 2, 96, [77, 64], 80, 2),
    (2, 3, 3, 64, [300, 1], 300, 5),
    (1, 1, 1, 32, [33], 33, 2),
    (1, 2, 4, 160, [95], 100, 3),
    (1, 1, 2, 192, [48], 64, 1),
    (1, 1, 2, 224, [129], 129, 4),
    (3, 1, 8, 128, [0, 0, 0], 16, 4),       # all empty
    # widths with a last 16-column chunk (the reference takes any multiple of 16)
    (1, 1, 1, 16, [40], 40, 1),
    (2, 2, 4, 48, [33, 100], 100, 3),
    (2, 1, 8, 80, [257, 5], 257, 4),
    (1, 2, 2, 112, [64], 64, 2),
    (1, 1, 16, 240, [90], 96, 3),
]


@needs_isa
@pytest.mark.parametrize("B,Hkv,G,D,lens,cap,threads", GQA_CASES)
def test_gqa_partial_matches_oracle(B, Hkv, G, D, lens, cap, threads):
    _gqa_case(B, Hkv, G, D, lens, cap, threads, seed=100 + D + G)


@needs_isa
def test_gqa_partial_large_scores_and_long_row():
    _gqa_case(1, 4, 8, 128, [4096], 4096, 8, seed=7, sigma=4.0)


@needs_isa
def test_gqa_partial_empty_rows_are_merge_identity():
    out, lse = _gqa_case(2, 2, 4, 128, [0, 50], 64, 3, seed=9)
    assert np.all(out[0].numpy() == 0) and np.all(np.isneginf(lse[0].numpy()))


@needs_isa
def test_gqa_partial_independent_of_thread_split():
    B, Hkv, G, D, cap = 4, 2, 4, 128, 2000
    lens = [1999, 31, 1000, 64]
    q = bf16_randn((B, Hkv * G, D), 1)
    k = bf16_randn((B * Hkv, cap, D), 2)
    v = bf16_randn((B * Hkv, cap, D), 3)
    # PV takes the probabilities rounded to bf16 relative to each segment's own
    # running max, so a different split rounds differently (about 2^-9
    # relative per term): outputs agree to 2e-3, LSE (fp32 sums) to 2e-5.
    ref_o, ref_l = host.gqa_partial_dense(q, k, v, lens, 0.09, 1)
    for th in (2, 3, 7, 13, 64):
        o, l = host.gqa_partial_dense(q, k, v, lens, 0.09, th)
        np.testing.assert_allclose(o.numpy(), ref_o.numpy(), atol=2e-3, rtol=2e-3)
        np.testing.assert_allclose(l.numpy(), ref_l.numpy(), atol=2e-5, rtol=2e-5)


def _mla_case(B, lens, cap, threads, seed):
    qn = bf16_randn((B * 16, 512), seed, 0.5)
    qp = bf16_randn((B * 16, 64), seed + 1, 0.5)
    c = bf16_randn((B, cap, 512), seed + 2, 0.5)
    pe = bf16_randn((B, cap, 64), seed + 3, 0.5)
    scale = 192 ** -0.5
    out, lse = host.mla_partial_dense(qn, qp, c, pe, lens, scale, threads)
    for b in range(B):
        L = lens[b]
        h = slice(b * 16, (b + 1) * 16)
        ow, lw = O.mla_attention_fp64(bits(qn[h]), bits(qp[h]), bits(c[b:b + 1, :L]),
                                      bits(pe[b:b + 1, :L]), scale)
        assert_close(out[h].numpy(), ow, OUT_ATOL, OUT_RTOL, f"mla out b={b}")
        assert_close(lse[h].numpy(), lw, LSE_ATOL, LSE_RTOL, f"mla lse b={b}")
    return out, lse


@needs_isa
@pytest.mark.parametrize("B,lens,cap,threads", [
    (1, [1], 1, 1),
    (2, [45, 0], 64, 3),
    (3, [1000, 17, 333], 1024, 8),
    (2, [2048, 1500], 2048, 16),
    (4, [0, 0, 0, 0], 8, 2),
    (1, [31], 33, 4),
])
def test_mla_partial_matches_oracle(B, lens, cap, threads):
    _mla_case(B, lens, cap, threads, seed=200 + B)


@needs_isa
def test_argument_errors():
    q = bf16_randn((1, 4, 128), 0)
    k = bf16_randn((1, 8, 128), 1)
    with pytest.raises(host.WhError, match="outside"):
        host.gqa_partial_dense(q, k, k, [9], 0.1)          # length beyond cap
    with pytest.raises(host.WhError, match="group size"):
        host.gqa_partial_dense(bf16_randn((1, 17, 128), 0), k, k, [4], 0.1)
    with pytest.raises(host.WhError, match="head_dim"):
        host.gqa_partial_dense(bf16_randn((1, 4, 40), 0), bf16_randn((1, 8, 40), 1),
                         bf16_randn((1, 8, 40), 2), [4], 0.1)
    with pytest.raises(ValueError):
        host.gqa_partial_dense(q.float(), k, k, [4], 0.1)  # dtype
    with pytest.raises(ValueError):
        host.gqa_partial_dense(q, k, k[:, :4], [4], 0.1)   # k/v mismatch
    L = host.lib()
    f = ctypes.c_float(0.1)
    rc = L.wh_gqa_partial(None, None, None, None, None, 1, 4, 1, 128, 64, 1, 1, f, None, None, 1)
    assert rc == -1 and b"null" in L.wh_last_error()
    assert L.wh_gqa_partial(None, None, None, None, None, 0, 4, 1, 128, 64, 1, 1, f,
                            None, None, 1) == 0      # empty batch is a no-op
    # page size must be a multiple of 32 once a sequence spans pages
    pools = bf16_randn((4, 1, 48, 128), 3)
    with pytest.raises(host.WhError, match="multiple of 32"):
        host.gqa_partial(q, pools, pools, [[0, 1]], [60], 0.1)
    # every page id a length reaches must be inside the pool
    pools = bf16_randn((2, 1, 32, 128), 3)
    with pytest.raises(host.WhError, match="page_table"):
        host.gqa_partial(q, pools, pools, [[0, 2]], [40], 0.1)
    host.gqa_partial(q, pools, pools, [[0, 2]], [32], 0.1)  # page 1 of the row not reached
    qn = bf16_randn((16, 512), 0)
    with pytest.raises(ValueError):
        host.mla_partial_dense(qn, bf16_randn((16, 64), 1), bf16_randn((1, 8, 576), 2),
                         bf16_randn((1, 8, 64), 3), [4], 0.1)
    with pytest.raises(host.WhError, match="outside"):
        host.mla_partial_dense(qn, bf16_randn((16, 64), 1), bf16_randn((1, 8, 512), 2),
                         bf16_randn((1, 8, 64), 3), [-1], 0.1)


def _paged(rng, lens, page_size, extra_pages=3):
    """A page table that scatters each sequence's pages over a shuffled pool."""
    need = [-(-L // page_size) for L in lens]
    max_pages = max(max(need), 1)
    num_pages = sum(need) + extra_pages
    perm = rng.permutation(num_pages)
    table = np.full((len(lens), max_pages), -1, np.int32)
    k = 0
    for b, n in enumerate(need):
        table[b, :n] = perm[k:k + n]
        k += n
    return torch.from_numpy(table), num_pages


def _gather(pool_u16, table, b, L, page_size):
    """Tokens [0, L) of sequence b from a paged pool [num_pages, ..., page_size, W]
    (token axis -2), concatenated along the token axis."""
    pages = [pool_u16[table[b, p]] for p in range(-(-L // page_size))]
    if not pages:
        return pool_u16[0][..., :0, :]
    return np.concatenate(pages, axis=-2)[..., :L, :]


@needs_isa
@pytest.mark.parametrize("page_size", [32, 64, 128])
def test_gqa_paged_matches_oracle(page_size):
    rng = np.random.default_rng(page_size)
    B, Hkv, G, D = 3, 2, 4, 128
    lens = [page_size * 3 + 5, 0, page_size - 1]
    table, num_pages = _paged(rng, lens, page_size)
    q = bf16_randn((B, Hkv * G, D), 1)
    kp = bf16_randn((num_pages, Hkv, page_size, D), 2)
    vp = bf16_randn((num_pages, Hkv, page_size, D), 3)
    out, lse = host.gqa_partial(q, kp, vp, table, lens, D ** -0.5, 5)
    tb = table.numpy()
    for b, L in enumerate(lens):
        k = _gather(bits(kp), tb, b, L, page_size)
        v = _gather(bits(vp), tb, b, L, page_size)
        ow, lw = O.gqa_attention_fp64(bits(q[b]).reshape(Hkv, G, D), k, v, D ** -0.5)
        assert_close(out[b].numpy().reshape(Hkv, G, D), ow, OUT_ATOL, OUT_RTOL, f"out b={b}")
        assert_close(lse[b].numpy().reshape(Hkv, G), lw, LSE_ATOL, LSE_RTOL, f"lse b={b}")


@needs_isa
@pytest.mark.parametrize("page_size", [32, 64])
def test_mla_paged_pool_matches_oracle(page_size):
    """The GPU pool layout [num_pages, page_size, 576] on the host."""
    rng = np.random.default_rng(page_size + 1)
    B = 3
    lens = [page_size * 4 + 17, 1, 0]
    table, num_pages = _paged(rng, lens, page_size)
    qn = bf16_randn((B * 16, 512), 4, 0.5)
    qp = bf16_randn((B * 16, 64), 5, 0.5)
    pool = bf16_randn((num_pages, page_size, 576), 6, 0.5)
    out, lse = host.mla_partial(qn, qp, pool, table, lens, 192 ** -0.5, 4)
    tb = table.numpy()
    for b, L in enumerate(lens):
        lat = _gather(bits(pool), tb, b, L, page_size)
        h = slice(b * 16, (b + 1) * 16)
        ow, lw = O.mla_attention_fp64(bits(qn[h]), bits(qp[h]), lat[None, :, :512],
                                      lat[None, :, 512:], 192 ** -0.5)
        assert_close(out[h].numpy(), ow, OUT_ATOL, OUT_RTOL, f"mla out b={b}")
        assert_close(lse[h].numpy(), lw, LSE_ATOL, LSE_RTOL, f"mla lse b={b}")


@needs_isa
def test_mla_strided_rows_take_the_gather_path():
    """Token strides other than 512/64 and 576/576 gather each 16 tokens into a
    dense tile first; same results."""
    B, L, W = 2, 100, 640  # 576 used + 64 unused per row
    qn = bf16_randn((B * 16, 512), 7, 0.5)
    qp = bf16_randn((B * 16, 64), 8, 0.5)
    rows = bf16_randn((B, L, W), 9, 0.5)
    flat = rows.view(-1)
    table = torch.arange(B, dtype=torch.int32).view(B, 1)
    out, lse = host._mla_call(qn, qp, flat, W, flat[512:], W, table, [L, L - 33], L, B,
                              192 ** -0.5, 3, None, None)
    for b, n in enumerate([L, L - 33]):
        r = bits(rows[b, :n])
        h = slice(b * 16, (b + 1) * 16)
        ow, lw = O.mla_attention_fp64(bits(qn[h]), bits(qp[h]), r[None, :, :512],
                                      r[None, :, 512:576], 192 ** -0.5)
        assert_close(out[h].numpy(), ow, OUT_ATOL, OUT_RTOL, f"mla out b={b}")
        assert_close(lse[h].numpy(), lw, LSE_ATOL, LSE_RTOL, f"mla lse b={b}")


@needs_isa
def test_prepared_call_reads_its_buffers_at_call_time():
    rng = np.random.default_rng(5)
    B, lens0 = 2, [200, 70]
    table, num_pages = _paged(rng, [256, 128], 64)
    qn = bf16_randn((B * 16, 512), 11, 0.5)
    qp = bf16_randn((B * 16, 64), 12, 0.5)
    pool = bf16_randn((num_pages, 64, 576), 13, 0.5)
    lens = torch.tensor(lens0, dtype=torch.int32)
    call = host.mla_partial(qn, qp, pool, table, lens, 0.07, 3, prepare=True)
    o1, l1 = (x.clone() for x in call())
    want_o, want_l = host.mla_partial(qn, qp, pool, table, lens0, 0.07, 3)
    np.testing.assert_array_equal(o1.numpy(), want_o.numpy())
    # new queries and lengths in place: the same call sees them
    qn.copy_(bf16_randn((B * 16, 512), 14, 0.5))
    lens[1] = 128
    o2, l2 = call()
    want_o, want_l = host.mla_partial(qn, qp, pool, table, [200, 128], 0.07, 3)
    np.testing.assert_array_equal(o2.numpy(), want_o.numpy())
    np.testing.assert_array_equal(l2.numpy(), want_l.numpy())
    assert not np.array_equal(o1.numpy(), o2.numpy())


@needs_isa
@pytest.mark.parametrize("Hkv,G,Dk,Dv,page_size,threads", [
    (16, 1, 192, 128, 64, 7),   # decompressed DeepSeek-V2: 16 heads, 192-wide keys
    (2, 4, 192, 128, 32, 3),
    (3, 2, 96, 96, 64, 4),      # Dk == Dv through the same entry point
    (2, 4, 80, 80, 32, 3),      # a last 16-column chunk
])
def test_attn_partial_separate_key_value_widths(Hkv, G, Dk, Dv, page_size, threads):
    """wh_attn_partial (the fused_cpu_attn_mla contract with Dk != Dv,
    kernel/cpu_attn.cpp:638-672) against fp64 and the oracle's C restatement."""
    from oracle import port
    rng = np.random.default_rng(Dk + Hkv)
    lens = [page_size * 2 + 9, 1, 0, 333]
    B = len(lens)
    table, num_pages = _paged(rng, lens, page_size)
    q = bf16_randn((B, Hkv * G, Dk), 11)
    kp = bf16_randn((num_pages, Hkv, page_size, Dk), 12)
    vp = bf16_randn((num_pages, Hkv, page_size, Dv), 13)
    scale = 192 ** -0.5
    out, lse = host.attn_partial(q, kp, vp, table, lens, scale, threads)
    assert tuple(out.shape) == (B, Hkv * G, Dv)
    tb = table.numpy()
    for b, L in enumerate(lens):
        k = _gather(bits(kp), tb, b, L, page_size)
        v = _gather(bits(vp), tb, b, L, page_size)
        qb = bits(q[b]).reshape(Hkv, G, Dk)
        ow, lw = O.gqa_attention_fp64(qb, k, v, scale)
        assert_close(out[b].numpy().reshape(Hkv, G, Dv), ow, OUT_ATOL, OUT_RTOL, f"out b={b}")
        assert_close(lse[b].numpy().reshape(Hkv, G), lw, LSE_ATOL, LSE_RTOL, f"lse b={b}")
        if L:
            po, pm, ps = port.cpu_attn(qb, np.ascontiguousarray(k), np.ascontiguousarray(v),
                                       scale, normalize=False, n_threads=2)
            assert_close(out[b].numpy().reshape(Hkv, G, Dv), po / ps, OUT_ATOL, OUT_RTOL,
                         f"vs C port b={b}")
            assert_close(lse[b].numpy().reshape(Hkv, G), (pm + np.log(ps))[..., 0], LSE_ATOL,
                         LSE_RTOL, f"lse vs C port b={b}")


def _randn_f32(shape, seed):
    g = torch.Generator(device="cpu").manual_seed(seed)
    return torch.randn(shape, generator=g, dtype=torch.float32)


# fp32 inputs, fp32 arithmetic: within 1e-4 of the fp64 closed form
F32_ATOL = F32_RTOL = 1e-4


@needs_isa
@pytest.mark.parametrize("Hkv,G,Dk,Dv,page_size,threads,lens", [
    (8, 4, 128, 128, 64, 7, [200, 1, 0, 333]),    # Mixtral grouping, ragged, one empty
    (2, 16, 256, 256, 32, 3, [65, 97]),
    (3, 1, 16, 16, 32, 2, [40, 7, 0]),
    (16, 1, 192, 128, 64, 5, [129, 64]),          # decompressed DeepSeek-V2 widths
    (1, 3, 48, 48, 64, 1, [1000]),
    (2, 2, 128, 128, 64, 4, [0, 0]),              # all empty: the merge identity
])
def test_attn_partial_fp32_inputs(Hkv, G, Dk, Dv, page_size, threads, lens):
    """wh_attn_partial_f32 (fused_cpu_attn on float32 inputs,
    kernel/cpu_attn.cpp:572-636, and fused_cpu_attn_fp32, :817-848) against the
    fp64 closed form and the oracle's C restatement run on the same floats."""
    from oracle import port
    rng = np.random.default_rng(Dk + G)
    B = len(lens)
    table, num_pages = _paged(rng, lens, page_size)
    q = _randn_f32((B, Hkv * G, Dk), 21)
    kp = _randn_f32((num_pages, Hkv, page_size, Dk), 22)
    vp = _randn_f32((num_pages, Hkv, page_size, Dv), 23)
    scale = Dk ** -0.5
    out, lse = host.attn_partial(q, kp, vp, table, lens, scale, threads)
    assert out.dtype == torch.float32 and tuple(out.shape) == (B, Hkv * G, Dv)
    tb = table.numpy()
    for b, L in enumerate(lens):
        k = _gather(kp.numpy(), tb, b, L, page_size)
        v = _gather(vp.numpy(), tb, b, L, page_size)
        qb = q[b].numpy().reshape(Hkv, G, Dk)
        ow, lw = O.gqa_attention_fp64(qb, k, v, scale)
        assert_close(out[b].numpy().reshape(Hkv, G, Dv), ow, F32_ATOL, F32_RTOL, f"out b={b}")
        assert_close(lse[b].numpy().reshape(Hkv, G), lw, F32_ATOL, F32_RTOL, f"lse b={b}")
        if L == 0:
            assert np.all(out[b].numpy() == 0) and np.all(np.isneginf(lse[b].numpy()))
            continue
        po, pm, ps = port.cpu_attn(qb, np.ascontiguousarray(k), np.ascontiguousarray(v), scale,
                                   normalize=False, n_threads=2)
        assert_close(out[b].numpy().reshape(Hkv, G, Dv), po / ps, F32_ATOL, F32_RTOL,
                     f"vs C port b={b}")


@needs_isa
def test_attn_partial_fp32_independent_of_thread_split():
    """fp32 probabilities: a different thread split changes only the fp32
    summation order."""
    rng = np.random.default_rng(5)
    lens = [1999, 31, 1000, 64]
    table, num_pages = _paged(rng, lens, 64)
    q = _randn_f32((4, 8, 128), 31)
    kp = _randn_f32((num_pages, 2, 64, 128), 32)
    vp = _randn_f32((num_pages, 2, 64, 128), 33)
    ref_o, ref_l = host.attn_partial(q, kp, vp, table, lens, 0.09, 1)
    for th in (2, 7, 64):
        o, l = host.attn_partial(q, kp, vp, table, lens, 0.09, th)
        np.testing.assert_allclose(o.numpy(), ref_o.numpy(), atol=1e-5, rtol=1e-5)
        np.testing.assert_allclose(l.numpy(), ref_l.numpy(), atol=1e-6, rtol=1e-6)


@needs_isa
def test_attn_partial_fp32_argument_errors():
    kp = _randn_f32((1, 1, 32, 40), 2)
    with pytest.raises(host.WhError, match="multiples of 16"):
        host.attn_partial(_randn_f32((1, 2, 40), 1), kp, kp,
                          torch.zeros((1, 1), dtype=torch.int32), [5], 0.1, 1)
    kp = _randn_f32((1, 1, 32, 64), 2)
    with pytest.raises(ValueError):  # mixed input dtypes
        host.attn_partial(bf16_randn((1, 2, 64), 1), kp, kp,
                          torch.zeros((1, 1), dtype=torch.int32), [5], 0.1, 1)


@needs_isa
def test_attn_partial_rejects_other_width_pairs():
    q = bf16_randn((1, 2, 192), 1)
    kp = bf16_randn((1, 2, 32, 192), 2)
    vp = bf16_randn((1, 2, 32, 64), 3)
    with pytest.raises(host.WhError, match="head_dim"):
        host.attn_partial(q, kp, vp, torch.zeros((1, 1), dtype=torch.int32), [5], 0.1, 1)


@needs_isa
@pytest.mark.parametrize("H,lens,threads", [(32, [300, 0, 77], 5), (128, [1000, 64], 16)])
def test_mla_partial_any_multiple_of_16_heads(H, lens, threads):
    """H = q rows / B as in fused_cpu_attn_mla_compressed (kernel/cpu_attn.cpp:860):
    DeepSeek-V2's 128 heads over one shared latent."""
    B = len(lens)
    cap = max(lens)
    qn = bf16_randn((B * H, 512), 400 + H, 0.5)
    qp = bf16_randn((B * H, 64), 401 + H, 0.5)
    c = bf16_randn((B, cap, 512), 402 + H, 0.5)
    pe = bf16_randn((B, cap, 64), 403 + H, 0.5)
    scale = 192 ** -0.5
    out, lse = host.mla_partial_dense(qn, qp, c, pe, lens, scale, threads)
    assert tuple(out.shape) == (B * H, 512)
    for b, L in enumerate(lens):
        h = slice(b * H, (b + 1) * H)
        ow, lw = O.mla_attention_fp64(bits(qn[h]), bits(qp[h]), bits(c[b:b + 1, :L]),
                                      bits(pe[b:b + 1, :L]), scale)
        assert_close(out[h].numpy(), ow, OUT_ATOL, OUT_RTOL, f"H={H} out b={b}")
        assert_close(lse[h].numpy(), lw, LSE_ATOL, LSE_RTOL, f"H={H} lse b={b}")
    with pytest.raises(ValueError, match="multiple"):
        host.mla_partial_dense(qn[:B * 24], qp[:B * 24], c, pe, lens, scale, threads)


def _bf16_rne_np(x):
    """float32 array -> its bf16 bit patterns, round to nearest even (the
    rounding torch's .to(torch.bfloat16) also uses)."""
    return bits(torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.bfloat16))


@needs_isa
@pytest.mark.parametrize("threads", [1, 5])
def test_bf16_outputs_are_the_fp32_outputs_rounded(threads):
    """wh_gqa_partial_bf16 / wh_mla_partial_bf16 compute exactly what the fp32
    entry points do and round out to bf16 (nearest even); lse is identical."""
    rng = np.random.default_rng(40 + threads)
    ps = 64
    lens = [ps * 3 + 5, 0, 1, 200]
    B = len(lens)
    table, num_pages = _paged(rng, lens, ps)
    Hkv, G, D = 2, 4, 128
    q = bf16_randn((B, Hkv * G, D), 41)
    kp = bf16_randn((num_pages, Hkv, ps, D), 42)
    vp = bf16_randn((num_pages, Hkv, ps, D), 43)
    o32, l32 = host.gqa_partial(q, kp, vp, table, lens, D ** -0.5, threads)
    o16, l16 = host.gqa_partial(q, kp, vp, table, lens, D ** -0.5, threads,
                                out_dtype=torch.bfloat16)
    assert o16.dtype == torch.bfloat16
    assert np.array_equal(bits(o16), _bf16_rne_np(o32.numpy()))
    assert torch.equal(l16, l32)
    qn = bf16_randn((B * 32, 512), 44, 0.5)  # 32 heads: two 16-head groups
    qp = bf16_randn((B * 32, 64), 45, 0.5)
    pool = bf16_randn((num_pages, ps, 576), 46, 0.5)
    m32, n32 = host.mla_partial(qn, qp, pool, table, lens, 192 ** -0.5, threads)
    out = torch.empty((B * 32, 512), dtype=torch.bfloat16)
    m16, n16 = host.mla_partial(qn, qp, pool, table, lens, 192 ** -0.5, threads, out=out)
    assert m16.data_ptr() == out.data_ptr()
    assert np.array_equal(bits(m16), _bf16_rne_np(m32.numpy()))
    assert torch.equal(n16, n32)


@needs_isa
def test_fp32_only_entry_rejects_bf16_out():
    q = bf16_randn((1, 16, 192), 50)
    kp = bf16_randn((1, 16, 64, 192), 51)
    vp = bf16_randn((1, 16, 64, 128), 52)
    with pytest.raises(TypeError, match="float32"):
        host.attn_partial(q, kp, vp, torch.zeros((1, 1), dtype=torch.int32), [10], 0.1,
                          out=torch.empty((1, 16, 128), dtype=torch.bfloat16))
