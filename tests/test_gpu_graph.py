"""Decode steps captured in HIP graphs (torch.cuda.CUDAGraph) and replayed.

The split step (fused append + partial) and its merge with a device-resident
host partial are captured twice, once per parity of the double-buffered
lengths (step s reads lengths[s % 2] and writes lengths[1 - s % 2]), and a
decode loop alternates the two graphs.  The library's launches record no
memset and allocate nothing, so they capture as plain kernel nodes.  Every
replay, with the test's own eager work and synchronisations between replays,
must equal bit for bit what the same calls give eagerly on a copy of the
state (outputs, lengths, and at the end the pools); the first replay, with
an empty host partial, is also checked against fp64 attention over every
token.
"""
import pytest
import torch

from oracle import attn_np as O
from scope_amd import ops
from tests.gpu_pool import gqa_pool, mla_pool
from tests.helpers import (LSE_ATOL, LSE_RTOL, OUT_ATOL, OUT_RTOL, assert_close,
                           bf16_randn, bits)

pytestmark = pytest.mark.gpu
DEV = "cuda"
PS = 64


def _say(msg):
    print(msg, flush=True)


def _host_operand(rows, Dv, s):
    """(out fp32 [rows, Dv], lse [rows]) of a host partial: empty at s == 0,
    seeded values after."""
    if s == 0:
        return (torch.zeros((rows, Dv)), torch.full((rows,), float("-inf")))
    g = torch.Generator().manual_seed(4000 + s)
    return (torch.randn((rows, Dv), generator=g), torch.randn(rows, generator=g) + 3.0)


def _clear_tail(pools, pt, lens, full):
    """Zero the slots of tokens [lens[b], full[b]) (the ones the steps append),
    so the final pool comparison sees the appends themselves."""
    for b, (L, F) in enumerate(zip(lens, full)):
        t = torch.arange(L, F, device=DEV)
        pid = pt[b, t // PS].long()
        for pool in pools:
            if pool.dim() == 4:   # [P, Hkv, PS, D]
                pool[pid, :, t % PS] = 0
            else:                 # [P, PS, 576]
                pool[pid, t % PS] = 0


def _capture(fn):
    """fn() captured in a graph on a side stream (the capture stream)."""
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            res = fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    return graph, res


def test_gqa_split_step_and_merge_replayed_from_two_graphs():
    B, Hkv, G, D = 3, 8, 4, 128
    Hq = Hkv * G
    lens = [700, 64, 1]
    steps = 6
    scale = D ** -0.5
    full = [L + steps for L in lens]
    k_pages, v_pages, pt, _, ks, vs = gqa_pool(full, Hkv, D, PS, seed=31)
    _clear_tail([k_pages, v_pages], pt, lens, full)
    max_len = max(full)
    nwg, wsb = ops.decode_plan(0, B * Hkv, G, max_len)

    def state():
        lens2 = torch.zeros((2, B), dtype=torch.int32, device=DEV)
        lens2[0] = torch.tensor(lens, dtype=torch.int32)
        return {"k": k_pages.clone(), "v": v_pages.clone(), "lens": lens2,
                "ws": torch.zeros(wsb, dtype=torch.uint8, device=DEV),
                "out": torch.empty((B * Hq, D), dtype=torch.bfloat16, device=DEV),
                "lse": torch.empty(B * Hq, dtype=torch.float32, device=DEV)}

    ins = {"q": torch.zeros((B, Hq, D), dtype=torch.bfloat16, device=DEV),
           "kn": torch.zeros((B, Hkv, 1, D), dtype=torch.bfloat16, device=DEV),
           "vn": torch.zeros((B, Hkv, 1, D), dtype=torch.bfloat16, device=DEV),
           "h_out": torch.zeros((B * Hq, D), dtype=torch.float32, device=DEV),
           "h_lse": torch.zeros(B * Hq, dtype=torch.float32, device=DEV)}

    def run(st, k):
        step = ops.gqa_append_decode_split(ins["q"], ins["kn"], ins["vn"], st["k"], st["v"], pt,
                                           st["lens"][k], st["lens"][1 - k], scale, max_len,
                                           n_workgroups=nwg, workspace=st["ws"])
        ops.merge_split(step, (ins["h_out"], ins["h_lse"]), ops.PARTIAL_LSE_F32,
                        out=st["out"], lse_out=st["lse"])

    run(state(), 0)  # loads the kernels and caches the plan, on a throwaway state
    run(state(), 1)
    torch.cuda.synchronize()
    sg, se = state(), state()
    graphs = [_capture(lambda k=k: run(sg, k))[0] for k in (0, 1)]
    for s in range(steps):
        _say(f"gqa graph replay step {s}")
        q = bf16_randn((B, Hq, D), 500 + s)
        pos = [L + s for L in lens]
        ins["q"].copy_(q)
        ins["kn"].copy_(torch.stack([ks[b][:, pos[b]:pos[b] + 1] for b in range(B)]))
        ins["vn"].copy_(torch.stack([vs[b][:, pos[b]:pos[b] + 1] for b in range(B)]))
        h_out, h_lse = _host_operand(B * Hq, D, s)
        ins["h_out"].copy_(h_out)
        ins["h_lse"].copy_(h_lse)
        graphs[s % 2].replay()
        torch.cuda.synchronize()
        run(se, s % 2)
        torch.cuda.synchronize()
        assert torch.equal(sg["out"], se["out"]), s
        assert torch.equal(sg["lse"], se["lse"]), s
        assert torch.equal(sg["lens"], se["lens"]), s
        assert sg["lens"][(s + 1) % 2].tolist() == [L + 1 for L in pos]
        if s == 0:
            got = sg["out"].float().cpu().numpy().reshape(B, Hkv, G, D)
            got_l = sg["lse"].cpu().numpy().reshape(B, Hkv, G)
            qb = bits(q).reshape(B, Hkv, G, D)
            for b in range(B):
                want, wl = O.gqa_attention_fp64(qb[b], bits(ks[b][:, :pos[b] + 1]),
                                                bits(vs[b][:, :pos[b] + 1]), scale)
                assert_close(got[b], want, OUT_ATOL, OUT_RTOL, f"b={b}")
                assert_close(got_l[b], wl, LSE_ATOL, LSE_RTOL, f"b={b} lse")
    assert torch.equal(sg["k"], se["k"]) and torch.equal(sg["v"], se["v"])
    k_all, _, _, _, _, _ = gqa_pool(full, Hkv, D, PS, seed=31)  # every token in place
    assert torch.equal(sg["k"], k_all)


def test_mla_split_step_and_uv_merge_replayed_from_two_graphs():
    B, H, Dout = 4, 16, 128
    lens = [900, 64, 31, 300]
    steps = 6
    scale = 192 ** -0.5
    full = [L + steps for L in lens]
    lat, pt, _, cs, pes = mla_pool(full, PS, seed=33)
    _clear_tail([lat], pt, lens, full)
    rows = B * H
    max_len = max(full)
    nwg, wsb = ops.decode_plan(1, B, H, max_len)
    w_uv = bf16_randn((H, Dout, 512), 77, 0.05).to(DEV)

    def state():
        lens2 = torch.zeros((2, B), dtype=torch.int32, device=DEV)
        lens2[0] = torch.tensor(lens, dtype=torch.int32)
        return {"lat": lat.clone(), "lens": lens2,
                "ws": torch.zeros(wsb, dtype=torch.uint8, device=DEV)}

    ins = {"qn": torch.zeros((rows, 512), dtype=torch.bfloat16, device=DEV),
           "qp": torch.zeros((rows, 64), dtype=torch.bfloat16, device=DEV),
           "kv": torch.zeros((B, 1, 576), dtype=torch.bfloat16, device=DEV),
           "h_out": torch.zeros((rows, 512), dtype=torch.float32, device=DEV),
           "h_lse": torch.zeros(rows, dtype=torch.float32, device=DEV)}

    def run(st, k):
        kv = ins["kv"]
        step = ops.mla_append_decode_split(ins["qn"], ins["qp"], kv[..., :512], kv[..., 512:],
                                           st["lat"], pt, st["lens"][k], st["lens"][1 - k],
                                           scale, max_len, n_workgroups=nwg, workspace=st["ws"])
        return ops.merge_split_uv(step, w_uv, (ins["h_out"], ins["h_lse"]),
                                  ops.PARTIAL_LSE_F32, want_latent=True, want_lse=True)

    run(state(), 0)
    run(state(), 1)
    torch.cuda.synchronize()
    sg, se = state(), state()
    caps = [_capture(lambda k=k: run(sg, k)) for k in (0, 1)]
    for s in range(steps):
        _say(f"mla graph replay step {s}")
        qn = bf16_randn((rows, 512), 600 + s, 0.5)
        qp = bf16_randn((rows, 64), 650 + s, 0.5)
        pos = [L + s for L in lens]
        ins["qn"].copy_(qn)
        ins["qp"].copy_(qp)
        ins["kv"].copy_(torch.stack([torch.cat([cs[b][pos[b]], pes[b][pos[b]]])
                                     for b in range(B)])[:, None])
        h_out, h_lse = _host_operand(rows, 512, s)
        ins["h_out"].copy_(h_out)
        ins["h_lse"].copy_(h_lse)
        graph, (g_v, g_lat, g_lse) = caps[s % 2]
        graph.replay()
        torch.cuda.synchronize()
        e_v, e_lat, e_lse = run(se, s % 2)
        torch.cuda.synchronize()
        assert torch.equal(g_v, e_v) and torch.equal(g_lat, e_lat), s
        assert torch.equal(g_lse, e_lse), s
        assert torch.equal(sg["lens"], se["lens"]), s
        if s == 0:
            got = g_lat.float().cpu().numpy()
            got_l = g_lse.cpu().numpy()
            for b in range(B):
                hh = slice(b * H, (b + 1) * H)
                want, wl = O.mla_attention_fp64(bits(qn[hh]), bits(qp[hh]),
                                                bits(cs[b][:pos[b] + 1])[None],
                                                bits(pes[b][:pos[b] + 1])[None], scale)
                assert_close(got[hh], want, OUT_ATOL, OUT_RTOL, f"b={b}")
                assert_close(got_l[hh], wl, LSE_ATOL, LSE_RTOL, f"b={b} lse")
    assert torch.equal(sg["lat"], se["lat"])
    assert torch.equal(sg["lat"], mla_pool(full, PS, seed=33)[0])  # every token in place
