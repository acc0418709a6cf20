"""ws_gqa_append_decode_partial_noalloc against ws_gqa_append_decode_partial,
through the C ABI: the same step (fused append + split-KV GQA partial +
combine) with the split pieces in the library's static scratch instead of a
caller workspace.  Outputs, lengths and the appended pages must be bit-identical
to the workspace entry point's, on two calls in a row (the second smaller, so
stale contents of the shared scratch from the first would show), and a plan
that needs more scratch than the library holds is refused before any launch.
"""
import ctypes

import numpy as np
import pytest
import torch

from gpu_pool import gqa_pool
from helpers import bits
from scope_amd import ops

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _lib():
    L = ops.lib()
    vp, i32, f32, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_size_t
    L.ws_gqa_append_decode_partial_noalloc.restype = i32
    L.ws_gqa_append_decode_partial_noalloc.argtypes = [vp] * 8 + [i32] * 9 + [f32, vp, vp, vp]
    L.ws_noalloc_scratch_bytes.restype = sz
    L.ws_noalloc_scratch_bytes.argtypes = []
    return L


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def _setup(L, lens, Hkv, G, seed, n_splits):
    """A fresh seeded pool and the no-alloc step over it: returns (call,
    tensors), call(stream) making the call on `stream` (a ctypes handle)."""
    D, PS = 128, 64
    B = len(lens)
    k_pages, v_pages, table, gpu_len, _, _ = gqa_pool([L_ + 1 for L_ in lens], Hkv, D, PS, seed)
    gpu_len.copy_(torch.tensor(lens, dtype=torch.int32, device=DEV))
    g = torch.Generator(device="cpu").manual_seed(seed + 7)
    q = (torch.randn((B, Hkv * G, D), generator=g)).to(torch.bfloat16).to(DEV)
    k_new = (torch.randn((B, Hkv, 1, D), generator=g)).to(torch.bfloat16).to(DEV)
    v_new = (torch.randn((B, Hkv, 1, D), generator=g)).to(torch.bfloat16).to(DEV)
    out = torch.full((B, Hkv * G, D), float("nan"), dtype=torch.float32, device=DEV)
    lse = torch.full((B, Hkv * G), float("nan"), dtype=torch.float32, device=DEV)
    len_out = torch.zeros(B, dtype=torch.int32, device=DEV)
    t = dict(q=q, k_new=k_new, v_new=v_new, k_pages=k_pages, v_pages=v_pages, table=table,
             gpu_len=gpu_len, out=out, lse=lse, len_out=len_out)

    def call(stream):
        return L.ws_gqa_append_decode_partial_noalloc(
            _p(q), _p(k_new), _p(v_new), _p(k_pages), _p(v_pages), _p(table), _p(gpu_len),
            _p(len_out), B, Hkv * G, Hkv, D, PS, table.shape[1], k_pages.shape[0],
            max(lens) + 1, n_splits, ctypes.c_float(D ** -0.5), _p(out), _p(lse), stream)

    return call, t


def _step(L, use_noalloc, lens, Hkv, G, seed, n_splits):
    """One fused step over a fresh seeded pool; returns (out, lse, len_out,
    k_pages, v_pages) after the call."""
    D, PS = 128, 64
    B = len(lens)
    # room for the appended token in every sequence's last page
    k_pages, v_pages, table, gpu_len, _, _ = gqa_pool([L_ + 1 for L_ in lens], Hkv, D, PS, seed)
    gpu_len.copy_(torch.tensor(lens, dtype=torch.int32, device=DEV))
    g = torch.Generator(device="cpu").manual_seed(seed + 7)
    q = (torch.randn((B, Hkv * G, D), generator=g)).to(torch.bfloat16).to(DEV)
    k_new = (torch.randn((B, Hkv, 1, D), generator=g)).to(torch.bfloat16).to(DEV)
    v_new = (torch.randn((B, Hkv, 1, D), generator=g)).to(torch.bfloat16).to(DEV)
    out = torch.full((B, Hkv * G, D), float("nan"), dtype=torch.float32, device=DEV)
    lse = torch.full((B, Hkv * G), float("nan"), dtype=torch.float32, device=DEV)
    len_out = torch.zeros(B, dtype=torch.int32, device=DEV)
    max_len = max(lens) + 1
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    args_head = (_p(q), _p(k_new), _p(v_new), _p(k_pages), _p(v_pages), _p(table), _p(gpu_len),
                 _p(len_out), B, Hkv * G, Hkv, D, PS, table.shape[1], k_pages.shape[0], max_len,
                 n_splits, ctypes.c_float(D ** -0.5), _p(out), _p(lse))
    torch.cuda.synchronize()
    if use_noalloc:
        rc = L.ws_gqa_append_decode_partial_noalloc(*args_head, stream)
        ws = None
    else:
        n, wsb = ops.decode_plan(0, B * Hkv, G, max_len, n_splits)
        ws = torch.zeros(max(wsb, 256), dtype=torch.uint8, device=DEV)
        rc = L.ws_gqa_append_decode_partial(*args_head, _p(ws), ctypes.c_size_t(wsb), stream)
    assert rc == 0, L.ws_last_error().decode()
    torch.cuda.synchronize()
    return out.cpu(), lse.cpu(), len_out.cpu(), bits(k_pages), bits(v_pages)


@pytest.mark.parametrize("splits", [0, 37])
def test_noalloc_matches_workspace_entry_point(splits):
    L = _lib()
    # two calls in a row, the second with a smaller batch and shorter rows
    cases = [([1500, 33, 700, 2048, 64, 1], 8, 4, 31),
             ([300, 5, 97], 4, 8, 32)]
    for lens, Hkv, G, seed in cases:
        print(f"noalloc vs workspace: lens={lens} Hkv={Hkv} G={G} splits={splits}", flush=True)
        got = _step(L, True, lens, Hkv, G, seed, splits)
        want = _step(L, False, lens, Hkv, G, seed, splits)
        for a, b, what in zip(got, want, ("out", "lse", "len_out", "k_pages", "v_pages")):
            a = np.asarray(a)
            b = np.asarray(b)
            assert a.shape == b.shape, what
            assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), f"{what} differs"
        assert np.isfinite(np.asarray(got[0])).all() and np.isfinite(np.asarray(got[1])).all()
        assert np.asarray(got[2]).tolist() == [x + 1 for x in lens]


def test_noalloc_refuses_plans_beyond_its_scratch():
    L = _lib()
    cap = L.ws_noalloc_scratch_bytes()
    assert cap == 8 << 20
    # 2048 sequences x 8 KV heads x group 16 need far more than the scratch:
    # refused on the host before any launch (the pointers are never used)
    t = torch.zeros(64, dtype=torch.float32, device=DEV)
    n, need = ops.decode_plan(0, 2048 * 8, 16, 4096, 0)
    assert need > cap
    p = _p(t)
    rc = L.ws_gqa_append_decode_partial_noalloc(
        p, p, p, p, p, p, p, p, 2048, 128, 8, 128, 64, 64, 1, 4096, 0,
        ctypes.c_float(0.1), p, p, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == -3  # WS_EWORKSPACE
    assert b"static" in L.ws_last_error()


def test_noalloc_captured_in_a_graph_replays_bit_for_bit():
    """The entry point under HIP graph capture (torch.cuda.graph): after an
    eager call on the device (its first call there looks up the scratch
    address, which must not happen during a capture), a captured call
    replays three times, with the state restored and the test's own eager
    work between replays, each time bit for bit what the eager call gave."""
    L = _lib()
    lens, Hkv, G, seed = [900, 17, 300, 64], 4, 8, 41
    call, t = _setup(L, lens, Hkv, G, seed, 0)
    keep = {k: v.clone() for k, v in t.items()}
    torch.cuda.synchronize()
    rc = call(ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0, L.ws_last_error().decode()
    torch.cuda.synchronize()
    names = ("out", "lse", "len_out", "k_pages", "v_pages")
    want = {k: t[k].clone() for k in names}

    def restore():
        for k, v in keep.items():
            t[k].copy_(v)
        torch.cuda.synchronize()

    restore()
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            rc = call(ctypes.c_void_p(side.cuda_stream))
    assert rc == 0, L.ws_last_error().decode()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    for rep in range(3):
        print(f"noalloc graph replay {rep}", flush=True)
        restore()
        graph.replay()
        torch.cuda.synchronize()
        for k in names:
            a, b = t[k].cpu(), want[k].cpu()
            assert torch.equal(a.view(torch.uint8) if a.dtype != torch.int32 else a,
                               b.view(torch.uint8) if b.dtype != torch.int32 else b), \
                f"replay {rep}: {k} differs from the eager call"
    assert t["len_out"].cpu().tolist() == [x + 1 for x in lens]
