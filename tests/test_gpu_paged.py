"""Decode steps of the two-sided paged caches (scope_amd/paged.py) on the
GPU, with the native host partial, before and after moving the boundary in
both directions, against fp64 attention over the whole sequence."""
import numpy as np
import pytest
import torch

from helpers import OUT_ATOL, OUT_RTOL, assert_close, bf16_randn, bits
from oracle import attn_np as O
from scope_amd.paged import PagedKVCache, PagedMlaCache

pytestmark = pytest.mark.gpu
DEV = "cuda"
PS = 64


def _say(msg):
    print(msg, flush=True)


def test_paged_mla_steps_across_boundary_moves():
    B, H, layers = 3, 16, 2
    lens = [700, 130, 64]
    hosts = [256, 64, 0]
    scale = 192 ** -0.5
    steps = 3
    total = max(lens) + steps
    cache = PagedMlaCache(layers, B, max_tokens=total + PS, page_size=PS, device=DEV)
    lat = {}
    for layer in range(layers):
        for b, (L, h) in enumerate(zip(lens, hosts)):
            lat[layer, b] = torch.cat([bf16_randn((L + steps, 512), 10 * layer + b, 0.5),
                                       bf16_randn((L + steps, 64), 10 * layer + b + 5, 0.5)],
                                      dim=1)
            x = lat[layer, b]
            cache.load(layer, b, x[:L, :512].contiguous(), x[:L, 512:].contiguous(), h)
    shares = [None, 0.2, 0.9]   # start, share down (GPU -> host), share up
    for s, share in enumerate(shares):
        if share is not None:
            cache.set_share(share)
        _say(f"paged mla step {s} share={share} host={[cache.host_tokens(b) for b in range(B)]}")
        for layer in range(layers):
            pos = [lens[b] + s for b in range(B)]
            new = torch.stack([lat[layer, b][pos[b]] for b in range(B)]).view(B, 1, 576)
            qn = bf16_randn((B * H, 512), 900 + 10 * s + layer, 0.5)
            qp = bf16_randn((B * H, 64), 950 + 10 * s + layer, 0.5)
            out = cache.step(layer, qn.to(DEV), qp.to(DEV), new[..., :512].contiguous().to(DEV),
                             new[..., 512:].contiguous().to(DEV), scale, host_threads=3)
            torch.cuda.synchronize()
            got = out.float().cpu().numpy()
            for b in range(B):
                full = bits(lat[layer, b][:pos[b] + 1])
                hh = slice(b * H, (b + 1) * H)
                want, _ = O.mla_attention_fp64(bits(qn[hh]), bits(qp[hh]), full[None, :, :512],
                                               full[None, :, 512:], scale)
                assert_close(got[hh], want, OUT_ATOL, OUT_RTOL, f"step {s} layer {layer} b={b}")
    for b in range(B):
        assert cache.seq_len(b) == lens[b] + steps


def test_paged_mla_steps_while_begun_boundary_moves_copy():
    """Decode steps queued while a begun move's page copies run on the side
    stream use the current boundaries; after the switch, the new ones."""
    B, H, layers = 3, 16, 2
    lens = [900, 300, 64]
    hosts = [256, 0, 0]
    scale = 192 ** -0.5
    steps = 6
    cache = PagedMlaCache(layers, B, max_tokens=max(lens) + steps + PS, page_size=PS, device=DEV)
    lat = {}
    for layer in range(layers):
        for b, (L, h) in enumerate(zip(lens, hosts)):
            lat[layer, b] = bf16_randn((L + steps, 576), 70 + 10 * layer + b, 0.5)
            x = lat[layer, b]
            cache.load(layer, b, x[:L, :512].contiguous(), x[:L, 512:].contiguous(), h)
    # (boundaries to begin before the step, poll / finish after it)
    plan = [(None, None), ([768, 256, 0], "poll"), (None, "finish"), ([0, 0, 64], None),
            (None, "poll"), (None, "finish")]
    for s, (targets, after) in enumerate(plan):
        if targets is not None:
            assert cache.begin_boundaries(targets)
        _say(f"paged mla step {s} begin={targets} moving={cache.moving} "
             f"host={[cache.host_tokens(b) for b in range(B)]}")
        for layer in range(layers):
            pos = [lens[b] + s for b in range(B)]
            new = torch.stack([lat[layer, b][pos[b]] for b in range(B)]).view(B, 1, 576)
            qn = bf16_randn((B * H, 512), 600 + 10 * s + layer, 0.5)
            qp = bf16_randn((B * H, 64), 650 + 10 * s + layer, 0.5)
            out = cache.step(layer, qn.to(DEV), qp.to(DEV), new[..., :512].contiguous().to(DEV),
                             new[..., 512:].contiguous().to(DEV), scale, host_threads=3)
            got = out.float().cpu().numpy()
            for b in range(B):
                full = bits(lat[layer, b][:pos[b] + 1])
                hh = slice(b * H, (b + 1) * H)
                want, _ = O.mla_attention_fp64(bits(qn[hh]), bits(qp[hh]), full[None, :, :512],
                                               full[None, :, 512:], scale)
                assert_close(got[hh], want, OUT_ATOL, OUT_RTOL, f"step {s} layer {layer} b={b}")
        if after == "poll":
            cache.poll_boundaries()
        elif after == "finish":
            cache.finish_boundaries()
            assert not cache.moving and cache.last_kept == []
    assert [cache.host_tokens(b) for b in range(B)] == [0, 0, 64]
    for b in range(B):
        assert cache.seq_len(b) == lens[b] + steps


def test_paged_gqa_steps_while_a_begun_boundary_move_copies():
    B, Hkv, G, D = 2, 8, 4, 128
    lens = [900, 200]
    hosts = [448, 0]
    scale = D ** -0.5
    steps = 3
    cache = PagedKVCache(1, B, Hkv, D, max_tokens=max(lens) + steps + PS, page_size=PS,
                         device=DEV)
    ks = [bf16_randn((Hkv, L + steps, D), 310 + b) for b, L in enumerate(lens)]
    vs = [bf16_randn((Hkv, L + steps, D), 410 + b) for b, L in enumerate(lens)]
    for b, (L, h) in enumerate(zip(lens, hosts)):
        cache.load(0, b, ks[b][:, :L].contiguous(), vs[b][:, :L].contiguous(), h)
    for s, targets in enumerate([[64, 128], None, None]):
        if targets is not None:
            assert cache.begin_boundaries(targets)   # seq 0 to the GPU, seq 1 to the host
        _say(f"paged gqa step {s} moving={cache.moving} "
             f"host={[cache.host_tokens(b) for b in range(B)]}")
        pos = [lens[b] + s for b in range(B)]
        k_new = torch.stack([ks[b][:, pos[b]:pos[b] + 1] for b in range(B)]).to(DEV)
        v_new = torch.stack([vs[b][:, pos[b]:pos[b] + 1] for b in range(B)]).to(DEV)
        q = bf16_randn((B, Hkv * G, D), 510 + s)
        out = cache.step(0, q.to(DEV), k_new, v_new, scale, host_threads=3)
        got = out.float().cpu().numpy()
        qb = bits(q).reshape(B, Hkv, G, D)
        for b in range(B):
            want, _ = O.gqa_attention_fp64(qb[b], bits(ks[b][:, :pos[b] + 1]),
                                           bits(vs[b][:, :pos[b] + 1]), scale)
            assert_close(got[b].reshape(Hkv, G, D), want, OUT_ATOL, OUT_RTOL, f"step {s} b={b}")
        if s == 1:
            cache.finish_boundaries()
    assert [cache.host_tokens(b) for b in range(B)] == [64, 128]


def test_paged_gqa_steps_across_boundary_moves():
    B, Hkv, G, D, layers = 2, 8, 4, 128, 1
    lens = [900, 200]
    hosts = [448, 128]
    scale = D ** -0.5
    steps = 3
    cache = PagedKVCache(layers, B, Hkv, D, max_tokens=max(lens) + steps + PS, page_size=PS,
                         device=DEV)
    ks = [bf16_randn((Hkv, L + steps, D), 300 + b) for b, L in enumerate(lens)]
    vs = [bf16_randn((Hkv, L + steps, D), 400 + b) for b, L in enumerate(lens)]
    for b, (L, h) in enumerate(zip(lens, hosts)):
        cache.load(0, b, ks[b][:, :L].contiguous(), vs[b][:, :L].contiguous(), h)
    for s, share in enumerate([None, 0.1, 0.95]):
        if share is not None:
            cache.set_share(share)
        _say(f"paged gqa step {s} share={share} host={[cache.host_tokens(b) for b in range(B)]}")
        pos = [lens[b] + s for b in range(B)]
        k_new = torch.stack([ks[b][:, pos[b]:pos[b] + 1] for b in range(B)]).to(DEV)
        v_new = torch.stack([vs[b][:, pos[b]:pos[b] + 1] for b in range(B)]).to(DEV)
        q = bf16_randn((B, Hkv * G, D), 500 + s)
        out = cache.step(0, q.to(DEV), k_new, v_new, scale, host_threads=3)
        torch.cuda.synchronize()
        got = out.float().cpu().numpy()
        qb = bits(q).reshape(B, Hkv, G, D)
        for b in range(B):
            want, _ = O.gqa_attention_fp64(qb[b], bits(ks[b][:, :pos[b] + 1]),
                                           bits(vs[b][:, :pos[b] + 1]), scale)
            assert_close(got[b].reshape(Hkv, G, D), want, OUT_ATOL, OUT_RTOL, f"step {s} b={b}")


def test_paged_mla_step_with_uv_epilogue_and_absorbed_query():
    """The full MLA attention block of a decode step: W_UK absorption of the
    raw query, the two-sided step, merge + W_UV in one launch; against fp64
    attention over the whole sequence with the same weights."""
    from scope_amd.paged import absorb_q
    B, H, Dout = 2, 16, 128
    lens, hosts = [300, 90], [128, 64]
    scale = 192 ** -0.5
    cache = PagedMlaCache(1, B, max_tokens=max(lens) + PS + 1, page_size=PS, device=DEV)
    lat = [torch.cat([bf16_randn((L + 1, 512), 40 + b, 0.5), bf16_randn((L + 1, 64), 45 + b, 0.5)],
                     dim=1) for b, L in enumerate(lens)]
    for b, (L, h) in enumerate(zip(lens, hosts)):
        cache.load(0, b, lat[b][:L, :512].contiguous(), lat[b][:L, 512:].contiguous(), h)
    w_uk = bf16_randn((H, 128, 512), 50, 0.05)
    w_uv = bf16_randn((H, Dout, 512), 51, 0.05)
    q_raw = bf16_randn((B, H, 128), 52, 1.0)
    qn = absorb_q(q_raw.to(DEV), w_uk.to(DEV))
    qp = bf16_randn((B * H, 64), 53, 0.5).to(DEV)
    new = torch.stack([lat[b][lens[b]] for b in range(B)]).view(B, 1, 576).to(DEV)
    out_v = cache.step(0, qn, qp, new[..., :512].contiguous(), new[..., 512:].contiguous(),
                       scale, host_threads=2, w_uv=w_uv.to(DEV))
    torch.cuda.synchronize()
    assert out_v.shape == (B, H * Dout) and out_v.dtype == torch.bfloat16
    got = out_v.float().cpu().numpy()
    qn_bits = bits(qn)   # the absorbed query as the step saw it (bf16)
    want_qn = np.einsum("bhd,hdk->bhk", O.as_f64(bits(q_raw)), O.as_f64(bits(w_uk)))
    assert_close(O.as_f64(qn_bits).reshape(B, H, 512), want_qn, 2e-2, 2e-2, "absorbed q")
    for b in range(B):
        full = bits(lat[b][:lens[b] + 1])
        hh = slice(b * H, (b + 1) * H)
        m_o, _ = O.mla_attention_fp64(qn_bits[hh], bits(qp.cpu())[hh], full[None, :, :512],
                                      full[None, :, 512:], scale)
        want = np.einsum("hk,hvk->hv", m_o, O.as_f64(bits(w_uv))).reshape(H * Dout)
        assert_close(got[b], want, OUT_ATOL, OUT_RTOL, f"out_v b={b}")


def test_layer_driver_failure_after_the_step_keeps_lengths_consistent():
    """A host-side failure after the split step was launched (here: a host
    length past the host page table) raises with stage 1; the cache counts
    the token the step appended, and the next step attends over it."""
    from scope_amd.layer import WlError

    B, H, layers = 2, 16, 1
    lens = [300, 129]
    hosts = [128, 64]
    scale = 192 ** -0.5
    cache = PagedMlaCache(layers, B, max_tokens=512, page_size=PS, device=DEV)
    lat = [torch.cat([bf16_randn((L + 2, 512), 70 + b, 0.5), bf16_randn((L + 2, 64), 75 + b, 0.5)],
                     dim=1) for b, L in enumerate(lens)]
    for b, (L, h) in enumerate(zip(lens, hosts)):
        cache.load(0, b, lat[b][:L, :512].contiguous(), lat[b][:L, 512:].contiguous(), h)
    cap = cache.host.table.shape[1] * PS
    good = int(cache.host.lens[1])
    cache.host.lens[1] = cap + PS  # the host partial refuses it, after the GPU step
    new = torch.stack([lat[b][lens[b]] for b in range(B)]).view(B, 1, 576).to(DEV)
    qn = bf16_randn((B * H, 512), 80, 0.5).to(DEV)
    qp = bf16_randn((B * H, 64), 81, 0.5).to(DEV)
    with pytest.raises(WlError) as err:
        cache.step(0, qn, qp, new[..., :512].contiguous(), new[..., 512:].contiguous(), scale,
                   host_threads=2)
    assert err.value.stage == 1
    cache.host.lens[1] = good
    torch.cuda.synchronize()
    assert [cache.seq_len(b) for b in range(B)] == [L + 1 for L in lens]
    new2 = torch.stack([lat[b][lens[b] + 1] for b in range(B)]).view(B, 1, 576).to(DEV)
    out = cache.step(0, qn, qp, new2[..., :512].contiguous(), new2[..., 512:].contiguous(),
                     scale, host_threads=2)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    for b in range(B):
        full = bits(lat[b][:lens[b] + 2])
        hh = slice(b * H, (b + 1) * H)
        want, _ = O.mla_attention_fp64(bits(qn[hh]), bits(qp[hh]), full[None, :, :512],
                                       full[None, :, 512:], scale)
        assert_close(got[hh], want, OUT_ATOL, OUT_RTOL, f"b={b} after the failed step")


def test_paged_gqa_step_on_a_side_stream_matches_the_default_stream():
    """The layer driver runs on the caller's current stream (its query-copy
    event is created on that stream's device): two caches with the same data,
    one stepped on a side stream, give bit-identical outputs."""
    B, Hkv, G, D = 2, 4, 4, 128
    lens, hosts = [200, 77], [128, 64]
    scale = D ** -0.5
    caches = [PagedKVCache(1, B, Hkv, D, max_tokens=max(lens) + PS, page_size=PS, device=DEV)
              for _ in range(2)]
    ks = [bf16_randn((Hkv, L + 1, D), 600 + b) for b, L in enumerate(lens)]
    vs = [bf16_randn((Hkv, L + 1, D), 610 + b) for b, L in enumerate(lens)]
    for c in caches:
        for b, (L, h) in enumerate(zip(lens, hosts)):
            c.load(0, b, ks[b][:, :L].contiguous(), vs[b][:, :L].contiguous(), h)
    k_new = torch.stack([ks[b][:, lens[b]:lens[b] + 1] for b in range(B)]).to(DEV)
    v_new = torch.stack([vs[b][:, lens[b]:lens[b] + 1] for b in range(B)]).to(DEV)
    q = bf16_randn((B, Hkv * G, D), 620).to(DEV)
    out0 = caches[0].step(0, q, k_new, v_new, scale, host_threads=2)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        out1 = caches[1].step(0, q, k_new, v_new, scale, host_threads=2)
    side.synchronize()
    assert np.array_equal(bits(out0), bits(out1))
    qb = bits(q.cpu()).reshape(B, Hkv, G, D)
    got = out1.float().cpu().numpy()
    for b in range(B):
        want, _ = O.gqa_attention_fp64(qb[b], bits(ks[b]), bits(vs[b]), scale)
        assert_close(got[b].reshape(Hkv, G, D), want, OUT_ATOL, OUT_RTOL, f"b={b}")


def test_paged_mla_step_with_more_sequences_than_one_wave_plans():
    """B = 70 sequences (past the 64 a single wave plans): the step falls back
    to the workgroup-wide plan, ragged lengths, a host share on some
    sequences; against fp64 over every sequence."""
    B, H = 70, 16
    rng = np.random.default_rng(70)
    lens = [int(x) for x in rng.integers(1, 300, B)]
    hosts = [PS * int(rng.integers(0, 3)) if L > 2 * PS else 0 for L in lens]
    hosts = [min(h, (L // PS) * PS) for h, L in zip(hosts, lens)]
    scale = 192 ** -0.5
    cache = PagedMlaCache(1, B, max_tokens=max(lens) + PS, page_size=PS, device=DEV)
    lat = [torch.cat([bf16_randn((L + 1, 512), 1000 + b, 0.5),
                      bf16_randn((L + 1, 64), 2000 + b, 0.5)], dim=1) for b, L in enumerate(lens)]
    for b, (L, h) in enumerate(zip(lens, hosts)):
        cache.load(0, b, lat[b][:L, :512].contiguous(), lat[b][:L, 512:].contiguous(), h)
    new = torch.stack([lat[b][lens[b]] for b in range(B)]).view(B, 1, 576).to(DEV)
    qn = bf16_randn((B * H, 512), 3000, 0.5)
    qp = bf16_randn((B * H, 64), 3001, 0.5)
    out = cache.step(0, qn.to(DEV), qp.to(DEV), new[..., :512].contiguous(),
                     new[..., 512:].contiguous(), scale, host_threads=4)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    for b in range(B):
        full = bits(lat[b][:lens[b] + 1])
        hh = slice(b * H, (b + 1) * H)
        want, _ = O.mla_attention_fp64(bits(qn[hh]), bits(qp[hh]), full[None, :, :512],
                                       full[None, :, 512:], scale)
        assert_close(got[hh], want, OUT_ATOL, OUT_RTOL, f"b={b} (L={lens[b]}, host={hosts[b]})")


def test_paged_mla_steps_overlap_a_large_begun_move():
    """A move large enough to outlast a decode step (16 layers x 4 sequences
    x 4096 tokens, host -> HBM, 302 MB): the steps are launched without
    synchronising between layers, whether the copies were still in flight
    when each step started is recorded (cache._move.event), and the first
    step must have started under them.  Sampled layers of every step match
    fp64 attention over the whole sequence."""
    B, H, layers, L = 4, 16, 16, 4096
    scale = 192 ** -0.5
    steps = 3
    cache = PagedMlaCache(layers, B, max_tokens=L + steps + PS, page_size=PS,
                          host_pages=B * (L // PS + 2), gpu_pages=B * (L // PS + 4), device=DEV)
    lat = {}
    for layer in range(layers):
        for b in range(B):
            lat[layer, b] = bf16_randn((L + steps, 576), 2000 + 10 * layer + b, 0.5)
            x = lat[layer, b]
            cache.load(layer, b, x[:L, :512].contiguous(), x[:L, 512:].contiguous(), L)
    torch.cuda.synchronize()
    assert cache.begin_boundaries([0] * B)
    under_copies = []
    outs = {}
    for s in range(steps):
        m = cache._move
        under_copies.append(m is not None and m.event is not None and not m.event.query())
        _say(f"large move: step {s} starts with the copies in flight: {under_copies[-1]} "
             f"host={[cache.host_tokens(b) for b in range(B)]}")
        for layer in range(layers):
            pos = [L + s] * B
            new = torch.stack([lat[layer, b][pos[b]] for b in range(B)]).view(B, 1, 576)
            qn = bf16_randn((B * H, 512), 3000 + 100 * s + layer, 0.5)
            qp = bf16_randn((B * H, 64), 3500 + 100 * s + layer, 0.5)
            out = cache.step(layer, qn.to(DEV), qp.to(DEV), new[..., :512].contiguous().to(DEV),
                             new[..., 512:].contiguous().to(DEV), scale, host_threads=8)
            if layer in (0, layers - 1):
                outs[s, layer] = (out, qn, qp)
        if s == 1:
            cache.finish_boundaries()
    torch.cuda.synchronize()
    assert under_copies[0], "the first step finished queueing after the copies ended"
    assert [cache.host_tokens(b) for b in range(B)] == [0] * B
    for (s, layer), (out, qn, qp) in outs.items():
        got = out.float().cpu().numpy()
        for b in (0, B - 1):
            full = bits(lat[layer, b][:L + s + 1])
            hh = slice(b * H, (b + 1) * H)
            want, _ = O.mla_attention_fp64(bits(qn[hh]), bits(qp[hh]), full[None, :, :512],
                                           full[None, :, 512:], scale)
            assert_close(got[hh], want, OUT_ATOL, OUT_RTOL, f"step {s} layer {layer} b={b}")
    for b in range(B):
        assert cache.seq_len(b) == L + steps
