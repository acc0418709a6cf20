"""The share controller driving a two-sided paged MLA cache on the GPU: the
decode loop measures each layer's GPU partial (events) and host partial
(wall time), the scheduler picks the share within an HBM budget of half the
cache, and the cache moves its pages between steps.  Starting host-heavy
(r = 0.1), the first decision moves to the capacity share and later steps
hold it; every step's merged output matches fp64 attention over all tokens,
before and after the moves.
"""
import pytest
import torch

from oracle import attn_np as O
from scope_amd.paged import PagedMlaCache
from scope_amd.scheduler import ShareController, ShareScheduler, Side
from tests.helpers import (LSE_ATOL, LSE_RTOL, OUT_ATOL, OUT_RTOL, assert_close, bf16_randn,
                           bits)

pytestmark = pytest.mark.gpu
DEV = "cuda"
PS = 64
H = 16
SCALE = 192 ** -0.5


@pytest.mark.parametrize("async_moves", [False, True])
def test_controller_moves_a_paged_mla_cache_to_its_hbm_budget(async_moves):
    # async_moves: the move's copies run under the next steps, which use the
    # old boundaries until the switch
    layers, steps = 3, 4
    lens = [3000, 1500, 800, 5000]
    B = len(lens)
    total = sum(lens) * 1152 * layers
    sched = ShareScheduler(gpu=Side(15e-6, 5e12), host=Side(40e-6, 50e9), xfer_s=40e-6,
                           hbm_budget_bytes=0.5 * total)
    ctl = ShareController(sched, 1152, layers, PS)
    host0 = ctl.targets_for(0.1, lens)
    cache = PagedMlaCache(layers, B, max_tokens=max(lens) + steps, page_size=PS, device=DEV)
    lat = [[bf16_randn((L + steps, 576), 1000 * l + b, 0.5) for b, L in enumerate(lens)]
           for l in range(layers)]
    for l in range(layers):
        for b, L in enumerate(lens):
            cache.load(l, b, lat[l][b][:L, :512], lat[l][b][:L, 512:], host0[b])
    cache.attach(ctl, async_moves=async_moves)
    for s in range(steps):
        for l in range(layers):
            qn = bf16_randn((B * H, 512), 50 + 10 * s + l, 0.5).to(DEV)
            qp = bf16_randn((B * H, 64), 60 + 10 * s + l, 0.5).to(DEV)
            new = torch.stack([lat[l][b][L + s] for b, L in enumerate(lens)]).to(DEV)[:, None]
            out, lse = cache.step(l, qn, qp, new[..., :512], new[..., 512:], SCALE,
                                  host_threads=8, return_lse=True)
            torch.cuda.synchronize()
            got, got_l = out.float().cpu().numpy(), lse.cpu().numpy()
            for b, L in enumerate(lens):
                full = bits(lat[l][b][:L + s + 1])
                rows = slice(b * H, (b + 1) * H)
                want, wl = O.mla_attention_fp64(bits(qn[rows]), bits(qp[rows]),
                                                full[None, :, :512], full[None, :, 512:], SCALE)
                what = f"step {s} layer {l} b {b} (host {cache.host_tokens(b)})"
                assert_close(got[rows], want, OUT_ATOL, OUT_RTOL, what)
                assert_close(got_l[rows], wl, LSE_ATOL, LSE_RTOL, what + " lse")
    print(f"moves {ctl.moves}, shares {ctl.shares}, chosen {ctl.chosen}", flush=True)
    cache.finish_boundaries()
    assert ctl.steps == steps
    assert ctl.moves and ctl.moves[0].step == 1
    assert ctl.moves[0].share_from < 0.15 and abs(ctl.moves[0].share_to - 0.5) < 0.03
    # the GPU side stays within the budget after every decision
    for n, r in enumerate(ctl.shares, start=1):
        W = sum(L + n for L in lens) * 1152
        assert r <= sched.capacity_share(W, layers) + 1e-9
    # the scheduler folded in the measured partials of both sides (an
    # observation shorter than a side's fixed cost carries no rate)
    sides = [h[0] for h in sched.history]
    assert "host" in sides and sides.count("host") + sides.count("gpu") <= 2 * layers * steps
