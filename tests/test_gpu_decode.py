"""End-to-end partitioned decode steps on the GPU (host partial from the
oracle's C restatement of the reference CPU kernels, or this package's native
host partial) and the reference-API drop-ins, against fp64 attention over the
whole sequence."""
import numpy as np
import pytest
import torch

from oracle import attn_np as O
from oracle import port
from scope_amd import ops, reference_api
from scope_amd.cache import GqaGpuPartition, PartitionedKVCache, PartitionedLatentCache
from scope_amd.decode import NATIVE, partitioned_gqa_decode, partitioned_mla_decode
from scope_amd.partition import gpu_share
from tests.helpers import (LSE_ATOL, LSE_RTOL, OUT_ATOL, OUT_RTOL, assert_close,
                           bf16_randn, bits)

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _say(msg):
    print(msg, flush=True)


def oracle_fused_cpu_attn_bf16(q, k, v, scale):
    """fused_cpu_attn contract on bf16 CPU tensors -> bf16 (out, max, sum)
    (kernel/cpu_attn.cpp:631-634), computed by the oracle's C restatement."""
    o, m, s = port.cpu_attn(bits(q), bits(k), bits(v), scale, normalize=True, n_threads=8)
    to16 = lambda a: torch.from_numpy(a).to(torch.bfloat16)
    return to16(o), to16(m), to16(s)


def oracle_fused_cpu_attn_mla(q, k, v, scale):
    o, m, s = port.cpu_attn(bits(q), bits(k), bits(v), scale, normalize=False, n_threads=8)
    return torch.from_numpy(o), torch.from_numpy(m), torch.from_numpy(s)


def oracle_mla_compressed(q_proj, q_pe, c, pe, scale):
    o, m, s = port.cpu_attn_mla_compressed(bits(q_proj), bits(q_pe), bits(c), bits(pe),
                                           scale, n_threads=8)
    return torch.from_numpy(o), torch.from_numpy(m), torch.from_numpy(s)


@pytest.mark.parametrize("r", [0.25, 0.5, 0.75])
@pytest.mark.parametrize("cpu", ["fused_cpu_attn_bf16", "fused_cpu_attn_mla", NATIVE])
def test_partitioned_gqa_step_mixtral_shape(r, cpu):
    # Mixtral layer shape (32 q / 8 KV heads, D 128), variable lengths,
    # trailing floor(r*L) tokens on the GPU, one appended token per step.
    B, Hkv, G, D = 4, 8, 4, 128
    rng = np.random.default_rng(int(r * 100))
    lens = rng.integers(100, 2000, B)
    _say(f"partitioned gqa r={r} cpu={cpu} lens={lens.tolist()}")
    scale = D ** -0.5
    k_all = [bf16_randn((Hkv, int(L) + 1, D), 500 + b) for b, L in enumerate(lens)]
    v_all = [bf16_randn((Hkv, int(L) + 1, D), 600 + b) for b, L in enumerate(lens)]
    g = [gpu_share(int(L), r) for L in lens]
    cache = PartitionedKVCache(1, B, Hkv, D, max_host=int(lens.max()),
                               max_gpu=max(g) + 64, device=DEV)
    for b, L in enumerate(lens):
        h = int(L) - g[b]
        cache.load_host(0, b, k_all[b][:, :h], v_all[b][:, :h])
        cache.gpu.load_sequence(0, b, k_all[b][:, h:L].to(DEV), v_all[b][:, h:L].to(DEV))
    k_new = torch.stack([k[:, -1:] for k in k_all]).to(DEV)
    v_new = torch.stack([v[:, -1:] for v in v_all]).to(DEV)
    q = bf16_randn((B, Hkv * G, D), 777)
    fn = {"fused_cpu_attn_bf16": oracle_fused_cpu_attn_bf16,
          "fused_cpu_attn_mla": oracle_fused_cpu_attn_mla, NATIVE: NATIVE}[cpu]
    fmt = cpu if cpu != NATIVE else "fused_cpu_attn_bf16"
    out = partitioned_gqa_decode(cache, 0, q.to(DEV), scale, fn, cpu_format=fmt,
                                 k_new=k_new, v_new=v_new, host_threads=3)
    torch.cuda.synchronize()
    assert out.shape == (B, Hkv * G, 1, D) and out.dtype == torch.bfloat16
    got = out.float().cpu().numpy()[:, :, 0]
    qb = bits(q).reshape(B, Hkv, G, D)
    for b in range(B):
        want, _ = O.gqa_attention_fp64(qb[b], bits(k_all[b]), bits(v_all[b]), scale)
        assert_close(got[b].reshape(Hkv, G, D), want, OUT_ATOL, OUT_RTOL, f"b={b}")
    assert cache.gpu.lens[0].tolist() == [gg + 1 for gg in g]


@pytest.mark.parametrize("host_fn", ["oracle", NATIVE])
def test_partitioned_mla_step_boundary_crossing(host_fn):
    # DS-V2-Lite absorbed shape: 16 heads, 576 latent, host segment gs tokens;
    # the appended tokens cross the boundary (system/deepseek.py:181-188).
    B, H, gs, L0 = 2, 16, 96, 90
    scale = 192 ** -0.5
    _say(f"partitioned mla boundary crossing host={host_fn}")
    cache = PartitionedLatentCache(1, B, max_seq=400, gs=gs, device=DEV)
    c_all = bf16_randn((B, 300, 512), 901, 0.5)
    pe_all = bf16_randn((B, 300, 64), 902, 0.5)
    cache.append(0, c_all[:, :L0], pe_all[:, :L0])          # all on the host
    cache.append(0, c_all[:, L0:L0 + 10], pe_all[:, L0:L0 + 10])  # 6 host + 4 GPU
    assert cache.gpu.lens[0].tolist() == [4, 4]
    cache.append(0, c_all[:, 100:299], pe_all[:, 100:299])
    qn = bf16_randn((B * H, 512), 903, 0.5)
    qp = bf16_randn((B * H, 64), 904, 0.5)
    out = partitioned_mla_decode(cache, 0, qn.to(DEV), qp.to(DEV), scale,
                                 oracle_mla_compressed if host_fn == "oracle" else NATIVE,
                                 c_new=c_all[:, 299:300].to(DEV), pe_new=pe_all[:, 299:300].to(DEV),
                                 host_threads=4)
    torch.cuda.synchronize()
    assert cache.seq_len(0) == 300 and cache.gpu.lens[0].tolist() == [300 - gs] * B
    want, _ = O.mla_attention_fp64(bits(qn), bits(qp), bits(c_all), bits(pe_all), scale)
    assert_close(out.float().cpu().numpy(), want, OUT_ATOL, OUT_RTOL, "mla merged")
    # host segment holds exactly the leading gs tokens
    (hc, hpe), _ = cache.get(0)
    assert np.array_equal(bits(hc), bits(c_all[:, :gs]))


def test_gpu_only_step_without_host_partial():
    B, Hkv, G, D = 2, 4, 8, 128
    part = GqaGpuPartition(1, B, Hkv, D, max_tokens=1000, device=DEV)
    ks = [bf16_randn((Hkv, 300 + 200 * b, D), 40 + b) for b in range(B)]
    vs = [bf16_randn((Hkv, 300 + 200 * b, D), 50 + b) for b in range(B)]
    for b in range(B):
        part.load_sequence(0, b, ks[b].to(DEV), vs[b].to(DEV))
    q = bf16_randn((B, Hkv * G, D), 60)
    out, lse = part.attend(0, q.to(DEV), D ** -0.5)
    torch.cuda.synchronize()
    qb = bits(q).reshape(B, Hkv, G, D)
    for b in range(B):
        want, wl = O.gqa_attention_fp64(qb[b], bits(ks[b]), bits(vs[b]), D ** -0.5)
        assert_close(out[b].cpu().numpy().reshape(Hkv, G, D), want, OUT_ATOL, OUT_RTOL, "out")
        assert_close(lse[b].cpu().numpy().reshape(Hkv, G), wl, LSE_ATOL, LSE_RTOL, "lse")
    part.reset()
    assert part.pool.free == part.num_pages and part.max_len(0) == 0


def test_reference_api_local_bmm_softmax_and_merge():
    # roofline/bench_resident_kv.py:410-459 kvlen check on the GPU kernels:
    # three token ranges merged pairwise match the whole within 2e-2.
    B, kv, NH, G, D = 2, 4096, 4, 8, 128
    q = bf16_randn((B * NH, G, D), 71)
    k = bf16_randn((B * NH, kv, D), 72)
    v = bf16_randn((B * NH, kv, D), 73)
    scale = D ** -0.5
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    gs = n_res = kv // 4
    parts = [reference_api.local_bmm_softmax(qd, kd[:, a:b].contiguous(),
                                             vd[:, a:b].contiguous(), scale)
             for a, b in ((0, gs), (gs, gs + n_res), (gs + n_res, kv))]
    o1, m1, s1 = reference_api.pairwise_merge(*parts[0], *parts[1])
    o2, m2, s2 = reference_api.pairwise_merge(o1, m1, s1, *parts[2])
    got = (o2 / s2.clamp(min=1e-6)).to(torch.bfloat16).float().cpu().numpy()
    ow, mw, sw = reference_api.local_bmm_softmax(qd, kd, vd, scale)
    whole = (ow / sw.clamp(min=1e-6)).to(torch.bfloat16).float().cpu().numpy()
    want, wl = O.gqa_attention_fp64(bits(q), bits(k), bits(v), scale)
    assert_close(got, want, OUT_ATOL, OUT_RTOL, "split/merge")
    assert_close(whole, want, OUT_ATOL, OUT_RTOL, "whole")
    assert_close(mw[..., 0].cpu().numpy(), wl, LSE_ATOL, LSE_RTOL, "lse")
    assert_close(m2[..., 0].cpu().numpy(), wl, LSE_ATOL, LSE_RTOL, "merged lse")


def test_reference_flow_with_the_cpu_extension_drop_in():
    """run_kvlen_resident's three ranges (roofline/bench_resident_kv.py:314-352)
    with every partial behind a reference signature: the CPU range through
    scope_amd.cpu_attn.fused_cpu_attn (bf16 normalised triple, un-normalised
    as system/mixoffload.py:1334 does), the resident range through
    resident_layer, the streamed range through local_bmm_softmax, merged by
    pairwise_merge; against fp64 over the whole range."""
    from scope_amd import cpu_attn
    N, kv, G, D = 8, 3000, 4, 128
    q = bf16_randn((N, G, D), 91)
    k = bf16_randn((N, kv + 1, D), 92)
    v = bf16_randn((N, kv + 1, D), 93)
    scale = D ** -0.5
    cpu_end, res_end = 1100, 2100          # CPU [0, 1100), resident [1100, 2100] + new token
    oc, mc, sc = cpu_attn.fused_cpu_attn(q, k[:, :cpu_end], v[:, :cpu_end], scale)
    oc = (oc.float() * sc.float()).to(DEV)
    mc, sc = mc.float().to(DEV), sc.float().to(DEV)
    qd = q.to(DEV)
    kr = k[:, cpu_end:res_end + 1].contiguous().to(DEV)
    vr = v[:, cpu_end:res_end + 1].contiguous().to(DEV)
    new_k, new_v = kr[:, -1:].clone(), vr[:, -1:].clone()
    kr[:, -1:] = 0
    vr[:, -1:] = 0
    parts = [reference_api.resident_layer(qd, kr, vr, new_k, new_v, scale),
             reference_api.local_bmm_softmax(qd, k[:, res_end + 1:].contiguous().to(DEV),
                                             v[:, res_end + 1:].contiguous().to(DEV), scale)]
    o1, m1, s1 = reference_api.pairwise_merge(oc, mc, sc, *parts[0])
    o2, m2, s2 = reference_api.pairwise_merge(o1, m1, s1, *parts[1])
    got = (o2 / s2.clamp(min=1e-6)).to(torch.bfloat16).float().cpu().numpy()
    want, wl = O.gqa_attention_fp64(bits(q), bits(k), bits(v), scale)
    assert_close(got, want, OUT_ATOL, OUT_RTOL, "three ranges")
    assert_close(m2[..., 0].cpu().numpy(), wl, 1e-2, 1e-2, "merged lse (bf16 CPU triple)")


def test_reference_api_resident_layer():
    N, cap, G, D = 8, 513, 4, 128
    k = bf16_randn((N, cap, D), 81).to(DEV)
    v = bf16_randn((N, cap, D), 82).to(DEV)
    nk = bf16_randn((N, 1, D), 83).to(DEV)
    nv = bf16_randn((N, 1, D), 84).to(DEV)
    q = bf16_randn((N, G, D), 85).to(DEV)
    o, m, s = reference_api.resident_layer(q, k, v, nk, nv, D ** -0.5)
    torch.cuda.synchronize()
    assert torch.equal(k[:, -1:], nk) and torch.equal(v[:, -1:], nv)
    want, wl = O.gqa_attention_fp64(bits(q), bits(k), bits(v), D ** -0.5)
    assert_close((o / s).cpu().numpy(), want, OUT_ATOL, OUT_RTOL, "resident")
    z = reference_api.resident_layer(q, k[:, :0], v[:, :0], nk, nv, 1.0)
    assert torch.all(z[0] == 0) and torch.all(torch.isinf(z[1]))


def test_split_steps_share_the_partition_workspace_in_order():
    """Two layers' split steps reuse the partition's workspace: merging each
    step before the next is correct; merging a step after a later step has
    reused the workspace is refused."""
    B, Hkv, G, D = 2, 4, 8, 128
    part = GqaGpuPartition(2, B, Hkv, D, max_tokens=600, device=DEV)
    ks = [[bf16_randn((Hkv, 300 + 100 * b + 1, D), 70 + 10 * l + b) for b in range(B)]
          for l in range(2)]
    vs = [[bf16_randn((Hkv, 300 + 100 * b + 1, D), 80 + 10 * l + b) for b in range(B)]
          for l in range(2)]
    for l in range(2):
        for b in range(B):
            part.load_sequence(l, b, ks[l][b][:, :-1].to(DEV), vs[l][b][:, :-1].to(DEV))
    q = bf16_randn((B, Hkv * G, D), 90)
    outs = []
    for l in range(2):
        kn = torch.stack([ks[l][b][:, -1:] for b in range(B)]).to(DEV)
        vn = torch.stack([vs[l][b][:, -1:] for b in range(B)]).to(DEV)
        st = part.step_split(l, q.to(DEV), kn, vn, D ** -0.5, n_workgroups=13)
        outs.append(ops.merge_split(st, None, out_dtype=torch.float32)[0])
    torch.cuda.synchronize()
    qb = bits(q).reshape(B, Hkv, G, D)
    for l in range(2):
        got = outs[l].cpu().numpy().reshape(B, Hkv, G, D)
        for b in range(B):
            want, _ = O.gqa_attention_fp64(qb[b], bits(ks[l][b]), bits(vs[l][b]), D ** -0.5)
            assert_close(got[b], want, OUT_ATOL, OUT_RTOL, f"layer {l} b={b}")
    kn = torch.stack([ks[0][b][:, -1:] for b in range(B)]).to(DEV)
    st0 = part.step_split(0, q.to(DEV), kn, kn, D ** -0.5)
    part.step_split(1, q.to(DEV), kn, kn, D ** -0.5)
    with pytest.raises(RuntimeError, match="reused"):
        ops.merge_split(st0)
