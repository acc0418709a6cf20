"""Host-side partition arithmetic (CPU only): boundary split, share, policy
table, page pool — product code vs the oracle's restatement and vs brute force."""
import numpy as np
import pytest

from oracle import attn_np as O
from scope_amd import partition as P
from scope_amd.cache import PagePool


def test_lookup_gs_table_points_and_interpolation():
    # table points are returned exactly (system/deepseek.py:127-130)
    for k, g in P.KV_LEN_GS_TABLE.items():
        assert P.lookup_gs(k) == g
    assert P.KV_LEN_GS_TABLE == O.KV_LEN_GS_TABLE
    # clamps at both ends
    assert P.lookup_gs(1) == 1280 and P.lookup_gs(10 ** 7) == 65536
    # interpolation: midpoint of 2048..4096 -> (1280 + 2560) / 2
    assert P.lookup_gs(3072) == 1920
    for L in list(range(1, 140000, 997)) + [2048, 2049, 131071, 131072]:
        assert P.lookup_gs(L) == O.lookup_gs(L)


def test_clamp_gs():
    assert P.clamp_gs(5000, 4096) == 4096
    assert P.clamp_gs(3000, 4096, cache_gs=2048) == 2048
    assert P.clamp_gs(-3, 10) == 0


def _brute_placement(t, n, gs):
    host, gpu = [], []
    for i in range(n):
        pos = t + i
        (host if pos < gs else gpu).append((pos if pos < gs else pos - gs, i))
    return host, gpu


@pytest.mark.parametrize("gs", [0, 1, 5, 64])
def test_boundary_split_enumerated(gs):
    for t in range(0, 80, 3):
        for n in range(0, 9):
            (h0, h1, hs), (g0, g1, gsrc) = P.boundary_split(t, n, gs)
            assert ((h0, h1, hs), (g0, g1, gsrc)) == O.boundary_split(t, n, gs)
            host, gpu = _brute_placement(t, n, gs)
            assert [(h0 + i, hs + i) for i in range(h1 - h0)] == host
            assert [(g0 + i, gsrc + i) for i in range(g1 - g0)] == gpu


def test_gpu_share_is_trailing_floor():
    assert P.gpu_share(1000, 0.25) == 250
    assert P.gpu_share(1001, 0.5) == 500
    assert P.gpu_share(7, 1.0) == 7
    assert P.gpu_share(7, 0.0) == 0
    rng = np.random.default_rng(3)
    for L in rng.integers(1024, 32769, 64):
        for r in (0.25, 0.5, 0.75):
            g = P.gpu_share(int(L), r)
            assert g == int(np.floor(r * int(L))) == O.gpu_share(int(L), r)
    with pytest.raises(ValueError):
        P.gpu_share(10, 1.5)


def test_round_gs_and_pages():
    assert P.round_gs_to(1, 64) == 64 and P.round_gs_to(64, 64) == 64
    assert P.round_gs_to(65, 64) == 128
    assert P.pages_for(0, 64) == 0 and P.pages_for(64, 64) == 1 and P.pages_for(65, 64) == 2


def test_page_pool():
    pool = PagePool(3)
    ids = [pool.alloc() for _ in range(3)]
    assert sorted(ids) == [0, 1, 2] and pool.free == 0
    with pytest.raises(MemoryError):
        pool.alloc()
    pool.release(ids[1])
    assert pool.alloc() == ids[1]


def test_gather_paged_model_roundtrip():
    # a paged pool read back through the page table is the contiguous tensor
    rng = np.random.default_rng(5)
    PS, D, Hkv = 4, 3, 2
    lens = [5, 0, 9]
    perm = rng.permutation(8)
    table = np.full((3, 3), -1, np.int32)
    used = 0
    for b, L in enumerate(lens):
        for p in range(P.pages_for(L, PS)):
            table[b, p] = perm[used]; used += 1
    pages = np.zeros((8, Hkv, PS, D), np.uint16)
    contig = [rng.integers(0, 65535, (Hkv, L, D)).astype(np.uint16) for L in lens]
    for b, L in enumerate(lens):
        for t in range(L):
            pages[table[b, t // PS], :, t % PS] = contig[b][:, t]
    for h in range(Hkv):
        got = O.gather_paged(pages, table, lens, head=h)
        for b in range(3):
            assert np.array_equal(got[b], contig[b][h])
