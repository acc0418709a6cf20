"""numpy restatement of the reference decode-attention math (oracle; tests only).

Every function cites the reference file:line it restates.  Arrays are numpy;
bf16 data is carried as uint16 bit patterns.

Pinning (tests/test_oracle.py):
  * fp64 closed forms are checked against brute-force per-element loops on
    tiny inputs, against closed-form special cases (one token, uniform scores,
    a dominant key, constant V) and against torch.softmax/logsumexp in fp64.
  * the fp32 blocked online softmax is checked against the fp64 closed form.
  * the merge is checked for split-anywhere = unsplit (the reference's own
    check, roofline/bench_resident_kv.py:446-454), commutativity,
    associativity and the empty-partition identity.
  * the integer model (boundary split, trailing share, pages) is checked by
    enumeration on small cases.
"""
from __future__ import annotations

import math

import numpy as np

# ---------------------------------------------------------------------------
# bf16 bit helpers


def bf16_to_f32(u16: np.ndarray) -> np.ndarray:
    """Widen bf16 bit patterns to float32 (exact)."""
    u16 = np.asarray(u16, dtype=np.uint16)
    return (u16.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """Round float32 to bf16 bit patterns, round-to-nearest-even; NaN stays NaN."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        rounded = rounded.copy()
        rounded[nan] = 0x7FC0
    return rounded


def as_f64(a: np.ndarray) -> np.ndarray:
    a = np.asarray(a)
    if a.dtype == np.uint16:
        return bf16_to_f32(a).astype(np.float64)
    return a.astype(np.float64)


# ---------------------------------------------------------------------------
# fp64 closed forms


def gqa_attention_fp64(q, k, v, scale):
    """softmax(q k^T * scale) v and its log-sum-exp, in float64.

    q [N, G, Dk], k [N, S, Dk], v [N, S, Dv] -> out [N, G, Dv] (normalised),
    lse [N, G] (natural log).  S == 0 gives (0, -inf), the empty partition of
    roofline/bench_resident_kv.py:263-267.  Same math as the GPU partial
    roofline/bench_resident_kv.py:150-157 and the CPU partial
    kernel/cpu_attn.cpp:572-636 before their roundings.
    """
    q, k, v = as_f64(q), as_f64(k), as_f64(v)
    N, G, _ = q.shape
    S, Dv = k.shape[1], v.shape[2]
    if S == 0:
        return np.zeros((N, G, Dv)), np.full((N, G), -np.inf)
    # matmul (BLAS) rather than einsum: the full-size parity tests call this
    # over sequences of up to 131072 tokens
    s = np.matmul(q, k.transpose(0, 2, 1)) * float(scale)
    m = s.max(axis=-1, keepdims=True)
    e = np.exp(s - m)
    l = e.sum(axis=-1, keepdims=True)
    out = np.matmul(e, v) / l
    return out, (m + np.log(l))[..., 0]


def mla_attention_fp64(q_nope, q_pe, c_kv, k_pe, scale):
    """Absorbed-MLA decode attention in float64.

    q_nope [B*H, 512] (already times W_UK), q_pe [B*H, 64], c_kv [B, S, 512],
    k_pe [B, S, 64]; score = (q_nope . c + q_pe . pe) * scale, out = p . c.
    Returns out [B*H, 512] normalised and lse [B*H].  Row b*H + h as in
    system/deepseek.py:337-338 and kernel/cpu_attn.cpp:909-910; formula of
    system/deepseek.py:378-388.
    """
    qn, qp, c, pe = as_f64(q_nope), as_f64(q_pe), as_f64(c_kv), as_f64(k_pe)
    B, S = c.shape[0], c.shape[1]
    H = qn.shape[0] // B
    qn = qn.reshape(B, H, -1)
    qp = qp.reshape(B, H, -1)
    if S == 0:
        return np.zeros((B * H, c.shape[2])), np.full((B * H,), -np.inf)
    s = (np.matmul(qn, c.transpose(0, 2, 1)) + np.matmul(qp, pe.transpose(0, 2, 1))) \
        * float(scale)
    m = s.max(axis=-1, keepdims=True)
    e = np.exp(s - m)
    l = e.sum(axis=-1, keepdims=True)
    out = np.matmul(e, c) / l
    return out.reshape(B * H, -1), (m + np.log(l))[..., 0].reshape(B * H)


def merge_fp64(out_a, lse_a, out_b, lse_b):
    """LSE merge of two normalised partials (natural-log lse), float64.

    Restates _pairwise_merge + final normalise
    (roofline/bench_resident_kv.py:141-148, 345-350) in the (out, lse) form;
    both-empty gives (0, -inf) as the reference's clamp(min=1e-6) does.
    """
    oa, ob = np.asarray(out_a, np.float64), np.asarray(out_b, np.float64)
    la, lb = np.asarray(lse_a, np.float64), np.asarray(lse_b, np.float64)
    M = np.maximum(la, lb)
    finite = np.isfinite(M)
    Ms = np.where(finite, M, 0.0)
    wa = np.where(np.isfinite(la), np.exp(la - Ms), 0.0)
    wb = np.where(np.isfinite(lb), np.exp(lb - Ms), 0.0)
    den = wa + wb
    safe = np.where(den > 0, den, 1.0)
    out = (wa[..., None] * oa + wb[..., None] * ob) / safe[..., None]
    out = np.where(finite[..., None], out, 0.0)
    lse = np.where(finite, Ms + np.log(safe), -np.inf)
    return out, lse


# ---------------------------------------------------------------------------
# reference triple conventions (o, max, sum)


def triple_to_partial(o, m, s, normalized: bool):
    """(o, max, sum) -> (out normalised, lse).

    normalized=False: o is the unnormalised accumulator returned by
    _local_bmm_softmax / fused_cpu_attn_mla / fused_cpu_attn_mla_compressed
    (roofline/bench_resident_kv.py:150-157, kernel/cpu_attn.cpp:638-672,
    852-1022).  normalized=True: o is fused_cpu_attn's normalised output
    (kernel/cpu_attn.cpp:566-567); system/mixoffload.py:1334 re-multiplies it
    by sum before merging, which this conversion makes unnecessary.
    """
    o = np.asarray(o, np.float64)
    m = np.asarray(m, np.float64).reshape(o.shape[:-1])
    s = np.asarray(s, np.float64).reshape(o.shape[:-1])
    pos = s > 0
    lse = np.where(pos, m + np.log(np.where(pos, s, 1.0)), -np.inf)
    if normalized:
        out = np.where(pos[..., None], o, 0.0)
    else:
        out = np.where(pos[..., None], o / np.where(pos, s, 1.0)[..., None], 0.0)
    return out, lse


def pairwise_merge_triple(o1, m1, s1, o2, m2, s2):
    """_pairwise_merge exactly as written (roofline/bench_resident_kv.py:141-148)."""
    mx = np.maximum(m1, m2)
    with np.errstate(invalid="ignore"):
        w1 = np.exp(m1 - mx)
        w2 = np.exp(m2 - mx)
    w1 = np.nan_to_num(w1)
    w2 = np.nan_to_num(w2)
    return w1 * o1 + w2 * o2, mx, w1 * s1 + w2 * s2


# ---------------------------------------------------------------------------
# fp32 online softmax with the reference CPU kernel's tiling


def cpu_tile_len(seq: int, rows: int, n_threads: int) -> int:
    """Sequence tile length of the GQA CPU kernel (kernel/cpu_attn.cpp:205-222)."""
    target = 1
    if rows < n_threads:
        target = max((n_threads + rows - 1) // rows, 2)
    tile = (seq + target - 1) // target
    tile = ((tile + 15) // 16) * 16
    tile = max(tile, 256)
    return min(tile, seq)


def online_softmax_fp32(q, k, v, scale, block=8):
    """fp32 online softmax over one row: q [G, Dk], k [S, Dk], v [S, Dv].

    Per `block` tokens: scores, new max, exp rescale of the running (sum, out),
    as in kernel/cpu_attn.cpp:282-298.  Returns unnormalised out, max, sum.
    """
    q = np.asarray(q, np.float32)
    k = np.asarray(k, np.float32)
    v = np.asarray(v, np.float32)
    G, Dv = q.shape[0], v.shape[1]
    o = np.zeros((G, Dv), np.float32)
    m = np.full((G,), -np.inf, np.float32)
    s = np.zeros((G,), np.float32)
    for t0 in range(0, k.shape[0], block):
        sc = (q @ k[t0:t0 + block].T) * np.float32(scale)
        nm = np.maximum(m, sc.max(axis=1))
        eo = np.exp(m - nm).astype(np.float32)
        e = np.exp(sc - nm[:, None]).astype(np.float32)
        s = eo * s + e.sum(axis=1)
        o = o * eo[:, None] + e @ v[t0:t0 + block]
        m = nm
    return o, m, s


def gqa_cpu_kernel_fp32(q, k, v, scale, n_threads=16, normalize=True):
    """Restatement of fused_cpu_attn's tiled online softmax + tile merge.

    kernel/cpu_attn.cpp:193-570 (tiling 205-222, per-tile online softmax
    282-347, tile merge 533-569).  Inputs as float arrays (bf16 widened by the
    caller); returns (out, max [N,G,1], sum [N,G,1]), out normalised when
    normalize is True.
    """
    q = np.asarray(q, np.float32)
    k = np.asarray(k, np.float32)
    v = np.asarray(v, np.float32)
    N, G, _ = q.shape
    S, Dv = k.shape[1], v.shape[2]
    out = np.zeros((N, G, Dv), np.float32)
    mx = np.full((N, G, 1), -np.inf, np.float32)
    sm = np.zeros((N, G, 1), np.float32)
    if S == 0:
        return out, mx, sm
    tile = cpu_tile_len(S, N, n_threads)
    for n in range(N):
        parts = [online_softmax_fp32(q[n], k[n, t:t + tile], v[n, t:t + tile], scale)
                 for t in range(0, S, tile)]
        gm = np.max([p[1] for p in parts], axis=0)
        o = np.zeros((G, Dv), np.float32)
        gs = np.zeros((G,), np.float32)
        for po, pm, ps in parts:
            w = np.exp(pm - gm).astype(np.float32)
            gs += w * ps
            o += w[:, None] * po
        if normalize:
            o = o / gs[:, None]
        out[n], mx[n, :, 0], sm[n, :, 0] = o, gm, gs
    return out, mx, sm


# ---------------------------------------------------------------------------
# partition / page / boundary integer model

KV_LEN_GS_TABLE = {
    2048: 1280, 4096: 2560, 8192: 4096, 16384: 6144,
    32768: 12288, 65536: 32768, 131072: 65536,
}


def lookup_gs(total_kv: int) -> int:
    """CPU token count by linear interpolation (system/deepseek.py:132-142)."""
    keys = sorted(KV_LEN_GS_TABLE)
    if total_kv <= keys[0]:
        return KV_LEN_GS_TABLE[keys[0]]
    if total_kv >= keys[-1]:
        return KV_LEN_GS_TABLE[keys[-1]]
    for k0, k1 in zip(keys, keys[1:]):
        if k0 <= total_kv <= k1:
            g0, g1 = KV_LEN_GS_TABLE[k0], KV_LEN_GS_TABLE[k1]
            return int(g0 + (g1 - g0) * (total_kv - k0) / (k1 - k0))
    return total_kv // 2


def boundary_split(t: int, n: int, gs: int):
    """Split new tokens [t, t+n) at the CPU/GPU boundary gs.

    Restates system/deepseek.py:181-188: returns ((c0, c1, src0), (g0, g1, src1))
    = host slots [c0, c1) from source offset src0, and GPU-partition slots
    [g0, g1) (relative to gs) from source offset src1.
    """
    t0, t1 = min(t, gs), min(t + n, gs)
    g0, g1 = max(t, gs) - gs, max(t + n, gs) - gs
    return (t0, t1, t0 - t), (g0, g1, g0 + gs - t)


def gpu_share(L: int, r: float) -> int:
    """GPU tokens of a sequence of length L at share r: the trailing floor(r*L)."""
    return int(math.floor(r * L))


def pages_needed(n_tokens: int, page_size: int = 64) -> int:
    return (n_tokens + page_size - 1) // page_size


def gather_paged(pages: np.ndarray, page_table: np.ndarray, lens, head=None):
    """Reassemble contiguous per-sequence tokens from a paged pool.

    pages [P, Hkv, PS, D] (GQA, head selects the KV head) or [P, PS, W] (MLA).
    Token t of sequence b is pages[page_table[b, t // PS], ..., t % PS, :].
    """
    out = []
    for b, L in enumerate(lens):
        rows = []
        for t in range(int(L)):
            pid = page_table[b, t // (pages.shape[-2])]
            off = t % pages.shape[-2]
            rows.append(pages[pid, head, off] if head is not None else pages[pid, off])
        out.append(np.stack(rows) if rows else np.zeros((0, pages.shape[-1]), pages.dtype))
    return out
