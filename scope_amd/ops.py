"""Operator surface of the GPU KV partition over the gfx950 C-ABI library.

Thin ctypes layer: validates shapes/dtypes/devices, passes data pointers and
the current HIP stream to scope_amd/lib/libwsgpu.so (include/wsgpu.h) and
raises on any error.  There is no fallback: if the library is missing or a
tensor is not on a GPU, the call fails.

Tensor conventions (all CUDA/HIP tensors, contiguous):
  GQA pools   k_pages, v_pages  [num_pages, Hkv, page_size, D] bfloat16
  MLA pool    latent_pages      [num_pages, page_size, 576]    bfloat16
  page_table  [B, max_pages] int32, gpu_len [B] int32
  partials    (out fp32 normalised, lse fp32 natural log); empty = (0, -inf)
"""
from __future__ import annotations

import ctypes
import os

import numpy as np
import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libwsgpu.so")

# Entry points declared in include/wsgpu.h.
EXPORTS = (
    "ws_last_error",
    "ws_version",
    "ws_kv_append",
    "ws_latent_append",
    "ws_decode_plan",
    "ws_attn_decode_plan",
    "ws_gqa_decode_partial",
    "ws_gqa_append_decode_partial",
    "ws_mla_decode_partial",
    "ws_mla_append_decode_partial",
    "ws_gqa_append_decode_split",
    "ws_gqa_append_decode_full",
    "ws_mla_append_decode_split",
    "ws_merge_split",
    "ws_mla_merge_split_uv",
    "ws_split_reduce",
    "ws_lse_merge",
    "ws_attn_decode_partial",
    "ws_attn_append_decode_partial",
    "ws_copy",
    "ws_copy_pages",
    "ws_noalloc_scratch_bytes",
    "ws_gqa_append_decode_partial_noalloc",
)

# Formats of the second operand of lse_merge (include/wsgpu.h).
PARTIAL_LSE_F32 = 0
TRIPLE_UNNORM_F32 = 1
TRIPLE_NORM_BF16 = 2
TRIPLE_NORM_F32 = 3
PARTIAL_LSE_BF16 = 4

MLA_LATENT = 576
MLA_C = 512
MLA_PE = 64


class WsError(RuntimeError):
    """A libwsgpu entry point returned an error."""


_lib = None


def lib() -> ctypes.CDLL:
    """Load libwsgpu.so (torch is imported first so that the process keeps a
    single HIP runtime)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is not built; run `python -m scope_amd._build` "
                "(or __graft_entry__.build())")
        L = ctypes.CDLL(LIB_PATH)
        vp, i32, i64, f32, sz = (ctypes.c_void_p, ctypes.c_int, ctypes.c_int64,
                                 ctypes.c_float, ctypes.c_size_t)
        L.ws_last_error.restype = ctypes.c_char_p
        L.ws_last_error.argtypes = []
        L.ws_version.restype = ctypes.c_char_p
        L.ws_version.argtypes = []
        L.ws_kv_append.restype = i32
        L.ws_kv_append.argtypes = [vp, vp, vp, vp, vp, vp, i32, i32, i32, i32,
                                   i32, i32, i32, i32, vp]
        L.ws_latent_append.restype = i32
        L.ws_latent_append.argtypes = [vp, i64, vp, i64, vp, vp, vp, i32, i32,
                                       i32, i32, i32, i32, vp]
        L.ws_decode_plan.restype = i32
        L.ws_decode_plan.argtypes = [i32, i32, i32, i32, i32,
                                     ctypes.POINTER(i32), ctypes.POINTER(sz)]
        L.ws_attn_decode_plan.restype = i32
        L.ws_attn_decode_plan.argtypes = [i32, i32, i32, i32, i32, i32,
                                          ctypes.POINTER(i32), ctypes.POINTER(sz)]
        L.ws_gqa_decode_partial.restype = i32
        L.ws_gqa_decode_partial.argtypes = [vp, vp, vp, vp, vp, i32, i32, i32,
                                            i32, i32, i32, i32, i32, i32, f32,
                                            vp, vp, vp, sz, vp]
        L.ws_gqa_append_decode_partial.restype = i32
        L.ws_gqa_append_decode_partial.argtypes = [vp, vp, vp, vp, vp, vp, vp, vp,
                                                   i32, i32, i32, i32, i32, i32, i32,
                                                   i32, i32, f32, vp, vp, vp, sz, vp]
        L.ws_gqa_append_decode_full.restype = i32
        L.ws_gqa_append_decode_full.argtypes = [vp] * 8 + [i32] * 9 + [f32, vp, vp, vp, vp, sz,
                                                                        vp]
        L.ws_mla_decode_partial.restype = i32
        L.ws_mla_decode_partial.argtypes = [vp, vp, vp, vp, vp, i32, i32, i32,
                                            i32, i32, i32, i32, f32, vp, vp,
                                            vp, sz, vp]
        L.ws_mla_append_decode_partial.restype = i32
        L.ws_mla_append_decode_partial.argtypes = [vp, vp, vp, i64, vp, i64, vp, vp,
                                                   vp, vp, i32, i32, i32, i32, i32,
                                                   i32, i32, f32, vp, vp, vp, sz, vp]
        L.ws_gqa_append_decode_split.restype = i32
        L.ws_gqa_append_decode_split.argtypes = L.ws_gqa_append_decode_partial.argtypes
        L.ws_mla_append_decode_split.restype = i32
        L.ws_mla_append_decode_split.argtypes = L.ws_mla_append_decode_partial.argtypes
        L.ws_merge_split.restype = i32
        L.ws_merge_split.argtypes = [vp, i32, i32, i32, i32, i32, i32, vp, vp, vp, sz,
                                     vp, vp, vp, i32, vp, vp, vp, vp]
        L.ws_mla_merge_split_uv.restype = i32
        L.ws_mla_merge_split_uv.argtypes = [vp, i32, i32, i32, i32, vp, vp, vp, sz, vp, vp, vp,
                                            i32, vp, i32, vp, vp, vp, vp]
        L.ws_split_reduce.restype = i32
        L.ws_split_reduce.argtypes = [vp, vp, vp, i32, i32, i32, i32, i32, vp,
                                      vp, vp]
        L.ws_attn_decode_partial.restype = i32
        L.ws_attn_decode_partial.argtypes = [vp] * 5 + [i32] * 10 + [f32, vp, vp, vp, sz, vp]
        L.ws_attn_append_decode_partial.restype = i32
        L.ws_attn_append_decode_partial.argtypes = [vp] * 8 + [i32] * 10 + [f32, vp, vp, vp,
                                                                             sz, vp]
        L.ws_copy.restype = i32
        L.ws_copy.argtypes = [vp, vp, sz, vp]
        L.ws_copy_pages.restype = i32
        L.ws_copy_pages.argtypes = [vp, i64, vp, i32, vp, i64, vp, i32, i32, i32, i64, i32, vp]
        L.ws_noalloc_scratch_bytes.restype = sz
        L.ws_noalloc_scratch_bytes.argtypes = []
        L.ws_gqa_append_decode_partial_noalloc.restype = i32
        L.ws_gqa_append_decode_partial_noalloc.argtypes = [vp] * 8 + [i32] * 9 + [f32, vp, vp,
                                                                               vp]
        L.ws_lse_merge.restype = i32
        L.ws_lse_merge.argtypes = [vp, vp, vp, vp, vp, i32, vp, vp, vp, i32,
                                   i32, vp]
        _lib = L
    return _lib


def _check(rc: int, name: str) -> None:
    if rc != 0:
        raise WsError(f"{name}: {lib().ws_last_error().decode()} (rc={rc})")


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(device: torch.device):
    """The current HIP stream of `device` (the raw handle torch launches on)."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    return ctypes.c_void_p(torch._C._cuda_getCurrentRawStream(idx))


def _require(t: torch.Tensor, name: str, dtype: torch.dtype, device=None,
             ndim=None, contiguous=True) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a tensor")
    if not t.is_cuda:
        raise ValueError(f"{name} must be on a GPU (got {t.device})")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype} (got {t.dtype})")
    if device is not None and t.device != device:
        raise ValueError(f"{name} is on {t.device}, expected {device}")
    if ndim is not None and t.dim() != ndim:
        raise ValueError(f"{name} must have {ndim} dims (got {tuple(t.shape)})")
    if contiguous and not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


# ---------------------------------------------------------------------------
# workspace

_workspaces: dict = {}


def _workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """Scratch for the split partials of the one-launch entry points, one per
    (device, stream): calls on one stream reuse it in stream order, calls on
    different streams never share it.  Grown on demand (the old buffer is
    freed through torch's stream-ordered allocator, so a launch still
    queued on this stream keeps its memory until it ran).  Each call writes
    the slots it reads back, so no initial contents are needed."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    key = (idx, torch._C._cuda_getCurrentRawStream(idx))
    ws = _workspaces.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        _workspaces[key] = ws
    return ws


_plans: dict = {}


def decode_plan(kind: int, rows_kv: int, heads: int, max_len: int,
                n_workgroups: int = 0):
    """(n_splits, workspace_bytes) of a decode call: kind 0 = GQA
    (rows_kv = B * Hkv, heads = group size), 1 = MLA (rows_kv = B, heads = 16).
    A split is one wave for GQA and one workgroup for MLA; the keyword keeps
    the name n_workgroups.  0 lets the library choose for the current
    device."""
    # the answer depends on the arguments and the current device only (a
    # decode loop asks the same question for every layer of a step)
    key = (kind, rows_kv, heads, max_len, n_workgroups,
           torch.cuda.current_device() if torch.cuda.is_initialized() else -1)
    hit = _plans.get(key)
    if hit is not None:
        return hit
    n, wsb = ctypes.c_int(0), ctypes.c_size_t(0)
    _check(lib().ws_decode_plan(kind, rows_kv, heads, max_len, n_workgroups,
                                ctypes.byref(n), ctypes.byref(wsb)), "ws_decode_plan")
    if len(_plans) > 4096:
        _plans.clear()
    _plans[key] = (n.value, wsb.value)
    return n.value, wsb.value


def gqa_plan(rows_kv: int, heads: int, Dk: int, Dv: int, max_len: int,
             n_workgroups: int = 0):
    """decode_plan kind 0 at key width Dk and value width Dv
    (ws_attn_decode_plan; kind 0 itself sizes the workspace for 128)."""
    if Dk == 128 and Dv == 128:
        return decode_plan(0, rows_kv, heads, max_len, n_workgroups)
    key = ("attn", rows_kv, heads, Dk, Dv, max_len, n_workgroups,
           torch.cuda.current_device() if torch.cuda.is_initialized() else -1)
    hit = _plans.get(key)
    if hit is not None:
        return hit
    n, wsb = ctypes.c_int(0), ctypes.c_size_t(0)
    _check(lib().ws_attn_decode_plan(rows_kv, heads, Dk, Dv, max_len, n_workgroups,
                                     ctypes.byref(n), ctypes.byref(wsb)),
           "ws_attn_decode_plan")
    if len(_plans) > 4096:
        _plans.clear()
    _plans[key] = (n.value, wsb.value)
    return n.value, wsb.value


# ---------------------------------------------------------------------------
# transfers


def copy_(dst: torch.Tensor, src: torch.Tensor) -> torch.Tensor:
    """dst.copy_(src) by the library's copy kernel (ws_copy) on the current
    stream of the GPU side: one of them on the GPU, the other on the GPU or in
    pinned host memory.  Used for a layer's query to the host partial, where
    a DMA copy's set-up latency sits on every layer's critical path."""
    if dst.dtype != src.dtype or dst.numel() != src.numel():
        raise ValueError("copy_: dst and src must have the same dtype and size")
    gpu = dst if dst.is_cuda else src
    if not gpu.is_cuda:
        raise ValueError("copy_: one side must be on a GPU")
    for t, n in ((dst, "dst"), (src, "src")):
        if not t.is_contiguous():
            raise ValueError(f"copy_: {n} must be contiguous")
        if t.is_cuda and t.device != gpu.device:
            raise ValueError("copy_: tensors on two GPUs")
        if not t.is_cuda and not t.is_pinned():
            raise ValueError(f"copy_: {n} must be on the GPU or in pinned host memory")
    _check(lib().ws_copy(_ptr(dst), _ptr(src), dst.numel() * dst.element_size(),
                         _stream(gpu.device)), "ws_copy")
    return dst


def copy_pages(dst_pool: torch.Tensor, dst_ids, src_pool: torch.Tensor, src_ids,
               max_workgroups: int = 0) -> None:
    """dst_pool[:, dst_ids[i]] = src_pool[:, src_ids[i]] for every layer, by
    the library's page-copy kernel (ws_copy_pages) on the current stream of
    the GPU side.  Pools are [layers, num_pages, *page] of one dtype; one of
    them on the GPU, the other on the same GPU or in pinned host memory (the
    kernel crosses the host link itself: no host gather, no staging).
    max_workgroups bounds the kernel's grid (0: the library's default)."""
    if dst_pool.dtype != src_pool.dtype or dst_pool.dim() < 2 or \
            dst_pool.shape[0] != src_pool.shape[0] or dst_pool.shape[2:] != src_pool.shape[2:]:
        raise ValueError("copy_pages: pools must match in dtype, layers and page shape")
    gpu = dst_pool if dst_pool.is_cuda else src_pool
    if not gpu.is_cuda:
        raise ValueError("copy_pages: one pool must be on a GPU")
    for t, n in ((dst_pool, "dst_pool"), (src_pool, "src_pool")):
        if not t.is_contiguous():
            raise ValueError(f"copy_pages: {n} must be contiguous")
        if t.is_cuda and t.device != gpu.device:
            raise ValueError("copy_pages: pools on two GPUs")
        if not t.is_cuda and not t.is_pinned():
            raise ValueError(f"copy_pages: {n} must be on the GPU or in pinned host memory")
    di = np.asarray(dst_ids, np.int64).reshape(-1)
    si = np.asarray(src_ids, np.int64).reshape(-1)
    if di.shape != si.shape:
        raise ValueError("copy_pages: dst_ids and src_ids differ in length")
    if di.size == 0:
        return
    for ids, pool, n in ((di, dst_pool, "dst_ids"), (si, src_pool, "src_ids")):
        if ids.min() < 0 or ids.max() >= pool.shape[1]:
            raise ValueError(f"copy_pages: {n} outside [0, {pool.shape[1]})")
    ids = torch.from_numpy(np.stack([di, si]).astype(np.int32)).to(gpu.device)
    page_bytes = dst_pool[0, 0].numel() * dst_pool.element_size()
    _check(lib().ws_copy_pages(
        _ptr(dst_pool), dst_pool.stride(0) * dst_pool.element_size(), _ptr(ids[0]),
        dst_pool.shape[1], _ptr(src_pool), src_pool.stride(0) * src_pool.element_size(),
        _ptr(ids[1]), src_pool.shape[1], int(di.size), dst_pool.shape[0], page_bytes,
        int(max_workgroups), _stream(gpu.device)), "ws_copy_pages")


# ---------------------------------------------------------------------------
# append


def kv_append(k_new, v_new, k_pages, v_pages, page_table, gpu_len, update_len=True):
    """Write k_new/v_new [B, Hkv, n_new, D] at slots gpu_len[b].. of each
    sequence's pages (bit copies), then gpu_len += n_new if update_len."""
    dev = k_pages.device
    _require(k_new, "k_new", torch.bfloat16, dev, 4)
    _require(v_new, "v_new", torch.bfloat16, dev, 4)
    _require(k_pages, "k_pages", torch.bfloat16, dev, 4)
    _require(v_pages, "v_pages", torch.bfloat16, dev, 4)
    _require(page_table, "page_table", torch.int32, dev, 2)
    _require(gpu_len, "gpu_len", torch.int32, dev, 1)
    B, Hkv, n_new, D = k_new.shape
    P, Hkv2, PS, D2 = k_pages.shape
    if v_new.shape != k_new.shape or v_pages.shape != k_pages.shape:
        raise ValueError("k/v shapes differ")
    if Hkv2 != Hkv or D2 != D or page_table.shape[0] != B or gpu_len.shape[0] != B:
        raise ValueError(
            f"shape mismatch: new {tuple(k_new.shape)} pages {tuple(k_pages.shape)} "
            f"page_table {tuple(page_table.shape)} gpu_len {tuple(gpu_len.shape)}")
    _check(lib().ws_kv_append(_ptr(k_new), _ptr(v_new), _ptr(k_pages), _ptr(v_pages),
                              _ptr(page_table), _ptr(gpu_len), B, Hkv, D, n_new, PS,
                              page_table.shape[1], P, int(bool(update_len)),
                              _stream(dev)), "ws_kv_append")


def latent_append(c_new, pe_new, latent_pages, page_table, gpu_len, update_len=True):
    """Write c_new [B, n_new, 512] and pe_new [B, n_new, 64] as the 576-wide
    latent at slots gpu_len[b].. of each sequence's pages."""
    dev = latent_pages.device
    for t, n in ((c_new, "c_new"), (pe_new, "pe_new")):
        _require(t, n, torch.bfloat16, dev, 3, contiguous=False)
        if t.stride(2) != 1 or t.stride(0) != t.shape[1] * t.stride(1):
            raise ValueError(f"{n} must be [B, n, W] with unit last stride and "
                             "batch stride n * row stride")
    _require(latent_pages, "latent_pages", torch.bfloat16, dev, 3)
    _require(page_table, "page_table", torch.int32, dev, 2)
    _require(gpu_len, "gpu_len", torch.int32, dev, 1)
    B, n_new, W = c_new.shape
    P, PS, L = latent_pages.shape
    if W != MLA_C or pe_new.shape != (B, n_new, MLA_PE) or L != MLA_LATENT:
        raise ValueError("latent layout is 512 c_kv + 64 k_pe = 576")
    if page_table.shape[0] != B or gpu_len.shape[0] != B:
        raise ValueError("page_table/gpu_len batch mismatch")
    _check(lib().ws_latent_append(_ptr(c_new), c_new.stride(1), _ptr(pe_new),
                                  pe_new.stride(1), _ptr(latent_pages), _ptr(page_table),
                                  _ptr(gpu_len), B, n_new, PS, page_table.shape[1], P,
                                  int(bool(update_len)), _stream(dev)),
           "ws_latent_append")


# ---------------------------------------------------------------------------
# decode partials


def gqa_decode_partial(q, k_pages, v_pages, page_table, gpu_len, scale, max_len,
                       n_workgroups=0, out=None, lse=None):
    """Split-KV GQA decode attention over the pooled tokens.

    q [B, Hq, D] bf16 -> (out [B, Hq, D] fp32 normalised, lse [B, Hq] fp32).
    max_len must bound every gpu_len[b] (the host's mirror of the lengths).
    """
    dev = k_pages.device
    _require(q, "q", torch.bfloat16, dev, 3)
    _require(k_pages, "k_pages", torch.bfloat16, dev, 4)
    _require(v_pages, "v_pages", torch.bfloat16, dev, 4)
    _require(page_table, "page_table", torch.int32, dev, 2)
    _require(gpu_len, "gpu_len", torch.int32, dev, 1)
    B, Hq, D = q.shape
    P, Hkv, PS, D2 = k_pages.shape
    if v_pages.shape != k_pages.shape or D2 != D:
        raise ValueError("k/v page pools must match q's head_dim")
    if page_table.shape[0] != B or gpu_len.shape[0] != B:
        raise ValueError("page_table/gpu_len batch mismatch")
    if out is None:
        out = torch.empty((B, Hq, D), dtype=torch.float32, device=dev)
    if lse is None:
        lse = torch.empty((B, Hq), dtype=torch.float32, device=dev)
    _require(out, "out", torch.float32, dev, 3)
    _require(lse, "lse", torch.float32, dev, 2)
    nwg, wsb = gqa_plan(B * Hkv, Hq // Hkv, D, D, int(max_len), int(n_workgroups))
    ws = _workspace(dev, wsb)
    _check(lib().ws_gqa_decode_partial(
        _ptr(q), _ptr(k_pages), _ptr(v_pages), _ptr(page_table), _ptr(gpu_len),
        B, Hq, Hkv, D, PS, page_table.shape[1], P, int(max_len), nwg, float(scale),
        _ptr(out), _ptr(lse), _ptr(ws), wsb, _stream(dev)), "ws_gqa_decode_partial")
    return out, lse


def attn_decode_partial(q, k_pages, v_pages, page_table, gpu_len, scale, max_len,
                        n_workgroups=0, k_new=None, v_new=None, len_out=None, out=None,
                        lse=None):
    """Decode attention with separate key / value widths (ws_attn_decode_partial,
    or ws_attn_append_decode_partial with k_new / v_new): q [B, Hq, Dk],
    k_pages [P, Hkv, PS, Dk], v_pages [P, Hkv, PS, Dv] bf16 ->
    (out [B, Hq, Dv] fp32 normalised, lse [B, Hq] fp32).  (Dk, Dv) is
    (64, 64), (128, 128), (256, 256), or (192, 128) with one query head
    per KV head.  With k_new [B, Hkv, 1, Dk] / v_new [B, Hkv, 1, Dv], token
    gpu_len[b] is appended
    first (fused step; len_out gets the new lengths, max_len must bound
    gpu_len + 1)."""
    dev = k_pages.device
    _require(q, "q", torch.bfloat16, dev, 3)
    _require(k_pages, "k_pages", torch.bfloat16, dev, 4)
    _require(v_pages, "v_pages", torch.bfloat16, dev, 4)
    _require(page_table, "page_table", torch.int32, dev, 2)
    _require(gpu_len, "gpu_len", torch.int32, dev, 1)
    B, Hq, Dk = q.shape
    P, Hkv, PS, Dk2 = k_pages.shape
    Dv = v_pages.shape[3]
    if Dk2 != Dk or v_pages.shape[:3] != k_pages.shape[:3]:
        raise ValueError(f"pools {tuple(k_pages.shape)} / {tuple(v_pages.shape)} do not "
                         f"match q {tuple(q.shape)}")
    if page_table.shape[0] != B or gpu_len.shape[0] != B:
        raise ValueError("page_table/gpu_len batch mismatch")
    if out is None:
        out = torch.empty((B, Hq, Dv), dtype=torch.float32, device=dev)
    if lse is None:
        lse = torch.empty((B, Hq), dtype=torch.float32, device=dev)
    _require(out, "out", torch.float32, dev, 3)
    _require(lse, "lse", torch.float32, dev, 2)
    nwg, wsb = gqa_plan(B * Hkv, Hq // Hkv, Dk, Dv, int(max_len), int(n_workgroups))
    ws = _workspace(dev, wsb)
    tail = (B, Hq, Hkv, Dk, Dv, PS, page_table.shape[1], P, int(max_len), nwg, float(scale),
            _ptr(out), _ptr(lse), _ptr(ws), wsb, _stream(dev))
    if k_new is None:
        _check(lib().ws_attn_decode_partial(_ptr(q), _ptr(k_pages), _ptr(v_pages),
                                            _ptr(page_table), _ptr(gpu_len), *tail),
               "ws_attn_decode_partial")
        return out, lse
    _require(k_new, "k_new", torch.bfloat16, dev, 4)
    _require(v_new, "v_new", torch.bfloat16, dev, 4)
    if k_new.shape != (B, Hkv, 1, Dk) or v_new.shape != (B, Hkv, 1, Dv):
        raise ValueError(f"k_new / v_new must be [B, Hkv, 1, Dk] / [B, Hkv, 1, Dv]")
    if len_out is not None:
        _require(len_out, "len_out", torch.int32, dev, 1)
        if len_out.shape[0] != B or len_out.data_ptr() == gpu_len.data_ptr():
            raise ValueError("len_out must be a separate [B] int32 tensor")
    _check(lib().ws_attn_append_decode_partial(
        _ptr(q), _ptr(k_new), _ptr(v_new), _ptr(k_pages), _ptr(v_pages), _ptr(page_table),
        _ptr(gpu_len), _ptr(len_out), *tail), "ws_attn_append_decode_partial")
    return out, lse


def mla_decode_partial(q_nope, q_pe, latent_pages, page_table, gpu_len, scale, max_len,
                       n_workgroups=0, out=None, lse=None):
    """Split-KV absorbed-MLA decode attention over the pooled latents.

    q_nope [B*H, 512] bf16 (W_UK-absorbed), q_pe [B*H, 64] bf16 ->
    (out [B*H, 512] fp32 normalised, lse [B*H] fp32).
    """
    dev = latent_pages.device
    _require(q_nope, "q_nope", torch.bfloat16, dev, 2)
    _require(q_pe, "q_pe", torch.bfloat16, dev, 2)
    _require(latent_pages, "latent_pages", torch.bfloat16, dev, 3)
    _require(page_table, "page_table", torch.int32, dev, 2)
    _require(gpu_len, "gpu_len", torch.int32, dev, 1)
    P, PS, L = latent_pages.shape
    B = page_table.shape[0]
    rows = q_nope.shape[0]
    if L != MLA_LATENT or q_nope.shape[1] != MLA_C or q_pe.shape != (rows, MLA_PE):
        raise ValueError("MLA layout is q_nope 512 + q_pe 64 over a 576 latent")
    if B == 0 or rows % B or gpu_len.shape[0] != B:
        raise ValueError("rows must be B * H with B = page_table.shape[0]")
    H = rows // B
    if out is None:
        out = torch.empty((rows, MLA_C), dtype=torch.float32, device=dev)
    if lse is None:
        lse = torch.empty((rows,), dtype=torch.float32, device=dev)
    _require(out, "out", torch.float32, dev, 2)
    _require(lse, "lse", torch.float32, dev, 1)
    nwg, wsb = decode_plan(1, B, H, int(max_len), int(n_workgroups))
    ws = _workspace(dev, wsb)
    _check(lib().ws_mla_decode_partial(
        _ptr(q_nope), _ptr(q_pe), _ptr(latent_pages), _ptr(page_table), _ptr(gpu_len),
        B, H, PS, page_table.shape[1], P, int(max_len), nwg, float(scale),
        _ptr(out), _ptr(lse), _ptr(ws), wsb, _stream(dev)), "ws_mla_decode_partial")
    return out, lse


def gqa_append_decode_partial(q, k_new, v_new, k_pages, v_pages, page_table, len_in,
                              len_out, scale, max_len, n_workgroups=0, out=None,
                              lse=None):
    """Append k_new/v_new [B, Hkv, 1, D] at position len_in[b] of each sequence
    and attend over the partition including it, in one launch.  len_out[b] =
    len_in[b] + 1 (len_out may be None; it must not be len_in).  max_len must
    bound every len_in[b] + 1.  Returns (out [B, Hq, D] fp32, lse [B, Hq])."""
    dev = k_pages.device
    _require(q, "q", torch.bfloat16, dev, 3)
    _require(k_new, "k_new", torch.bfloat16, dev, 4)
    _require(v_new, "v_new", torch.bfloat16, dev, 4)
    _require(k_pages, "k_pages", torch.bfloat16, dev, 4)
    _require(v_pages, "v_pages", torch.bfloat16, dev, 4)
    _require(page_table, "page_table", torch.int32, dev, 2)
    _require(len_in, "len_in", torch.int32, dev, 1)
    B, Hq, D = q.shape
    P, Hkv, PS, D2 = k_pages.shape
    if v_pages.shape != k_pages.shape or D2 != D:
        raise ValueError("k/v page pools must match q's head_dim")
    if k_new.shape != (B, Hkv, 1, D) or v_new.shape != k_new.shape:
        raise ValueError(f"k_new/v_new must be [B, Hkv, 1, D] = {(B, Hkv, 1, D)}")
    if page_table.shape[0] != B or len_in.shape[0] != B:
        raise ValueError("page_table/len_in batch mismatch")
    if len_out is not None:
        _require(len_out, "len_out", torch.int32, dev, 1)
        if len_out.shape[0] != B or len_out.data_ptr() == len_in.data_ptr():
            raise ValueError("len_out must be a separate [B] int32 tensor")
    if out is None:
        out = torch.empty((B, Hq, D), dtype=torch.float32, device=dev)
    if lse is None:
        lse = torch.empty((B, Hq), dtype=torch.float32, device=dev)
    _require(out, "out", torch.float32, dev, 3)
    _require(lse, "lse", torch.float32, dev, 2)
    nwg, wsb = gqa_plan(B * Hkv, Hq // Hkv, D, D, int(max_len), int(n_workgroups))
    ws = _workspace(dev, wsb)
    _check(lib().ws_gqa_append_decode_partial(
        _ptr(q), _ptr(k_new), _ptr(v_new), _ptr(k_pages), _ptr(v_pages), _ptr(page_table),
        _ptr(len_in), _ptr(len_out), B, Hq, Hkv, D, PS, page_table.shape[1], P,
        int(max_len), nwg, float(scale), _ptr(out), _ptr(lse), _ptr(ws), wsb,
        _stream(dev)), "ws_gqa_append_decode_partial")
    return out, lse


def gqa_append_decode_full(q, k_new, v_new, k_pages, v_pages, page_table, len_in, len_out,
                           scale, max_len, n_workgroups=0, out_bf16=None, out=None, lse=None,
                           want_fp32=False):
    """The whole decode step of a partition that holds every token (no host
    share): gqa_append_decode_partial that also writes the normalised output
    in bf16 (the step launch and its combine launch).  Returns (out_bf16
    [B, Hq, D], lse [B, Hq]) or, with want_fp32 (or an `out` given),
    (out_bf16, out fp32, lse)."""
    dev = k_pages.device
    for t, n, dt, nd in ((q, "q", torch.bfloat16, 3), (k_new, "k_new", torch.bfloat16, 4),
                         (v_new, "v_new", torch.bfloat16, 4),
                         (k_pages, "k_pages", torch.bfloat16, 4),
                         (v_pages, "v_pages", torch.bfloat16, 4),
                         (page_table, "page_table", torch.int32, 2),
                         (len_in, "len_in", torch.int32, 1)):
        _require(t, n, dt, dev, nd)
    B, Hq, D = q.shape
    P, Hkv, PS, D2 = k_pages.shape
    if v_pages.shape != k_pages.shape or D2 != D:
        raise ValueError("k/v page pools must match q's head_dim")
    if k_new.shape != (B, Hkv, 1, D) or v_new.shape != k_new.shape:
        raise ValueError(f"k_new/v_new must be [B, Hkv, 1, D] = {(B, Hkv, 1, D)}")
    if page_table.shape[0] != B or len_in.shape[0] != B:
        raise ValueError("page_table/len_in batch mismatch")
    if len_out is not None:
        _require(len_out, "len_out", torch.int32, dev, 1)
        if len_out.shape[0] != B or len_out.data_ptr() == len_in.data_ptr():
            raise ValueError("len_out must be a separate [B] int32 tensor")
    if out_bf16 is None:
        out_bf16 = torch.empty((B, Hq, D), dtype=torch.bfloat16, device=dev)
    _require(out_bf16, "out_bf16", torch.bfloat16, dev, 3)
    give_fp32 = want_fp32 or out is not None
    if out is None:  # the step's fp32 partial (finalised in place by the combine)
        out = torch.empty((B, Hq, D), dtype=torch.float32, device=dev)
    _require(out, "out", torch.float32, dev, 3)
    if lse is None:
        lse = torch.empty((B, Hq), dtype=torch.float32, device=dev)
    _require(lse, "lse", torch.float32, dev, 2)
    if out_bf16.shape != q.shape or out.shape != q.shape or lse.shape != (B, Hq):
        raise ValueError("out_bf16/out must be [B, Hq, D] and lse [B, Hq]")
    nwg, wsb = gqa_plan(B * Hkv, Hq // Hkv, D, D, int(max_len), int(n_workgroups))
    ws = _workspace(dev, wsb)
    _check(lib().ws_gqa_append_decode_full(
        _ptr(q), _ptr(k_new), _ptr(v_new), _ptr(k_pages), _ptr(v_pages), _ptr(page_table),
        _ptr(len_in), _ptr(len_out), B, Hq, Hkv, D, PS, page_table.shape[1], P,
        int(max_len), nwg, float(scale), _ptr(out_bf16), _ptr(out), _ptr(lse), _ptr(ws), wsb,
        _stream(dev)), "ws_gqa_append_decode_full")
    return (out_bf16, out, lse) if give_fp32 else (out_bf16, lse)


def gqa_append_decode_partial_noalloc(q, k_new, v_new, k_pages, v_pages, page_table, len_in,
                                      len_out, scale, max_len, out, lse, n_workgroups=0):
    """gqa_append_decode_partial without a workspace or any allocation: the
    caller passes out [B, Hq, D] fp32 and lse [B, Hq] fp32, and the split
    pieces live in the library's static scratch (ws_noalloc_scratch_bytes()
    per GPU).  Calls that overlap on one GPU race on that scratch; calls on
    one stream do not.  Usable under HIP graph capture."""
    dev = k_pages.device
    for t, n, dt, nd in ((q, "q", torch.bfloat16, 3), (k_new, "k_new", torch.bfloat16, 4),
                         (v_new, "v_new", torch.bfloat16, 4), (k_pages, "k_pages", torch.bfloat16, 4),
                         (v_pages, "v_pages", torch.bfloat16, 4),
                         (page_table, "page_table", torch.int32, 2),
                         (len_in, "len_in", torch.int32, 1), (out, "out", torch.float32, 3),
                         (lse, "lse", torch.float32, 2)):
        _require(t, n, dt, dev, nd)
    B, Hq, D = q.shape
    P, Hkv, PS, D2 = k_pages.shape
    if v_pages.shape != k_pages.shape or D2 != D or out.shape != q.shape or \
            lse.shape != (B, Hq):
        raise ValueError("k/v pools, out and lse must match q")
    if k_new.shape != (B, Hkv, 1, D) or v_new.shape != k_new.shape:
        raise ValueError(f"k_new/v_new must be [B, Hkv, 1, D] = {(B, Hkv, 1, D)}")
    if page_table.shape[0] != B or len_in.shape[0] != B:
        raise ValueError("page_table/len_in batch mismatch")
    if len_out is not None:
        _require(len_out, "len_out", torch.int32, dev, 1)
        if len_out.shape[0] != B or len_out.data_ptr() == len_in.data_ptr():
            raise ValueError("len_out must be a separate [B] int32 tensor")
    _check(lib().ws_gqa_append_decode_partial_noalloc(
        _ptr(q), _ptr(k_new), _ptr(v_new), _ptr(k_pages), _ptr(v_pages), _ptr(page_table),
        _ptr(len_in), _ptr(len_out), B, Hq, Hkv, D, PS, page_table.shape[1], P, int(max_len),
        int(n_workgroups), float(scale), _ptr(out), _ptr(lse), _stream(dev)),
        "ws_gqa_append_decode_partial_noalloc")
    return out, lse


def mla_append_decode_partial(q_nope, q_pe, c_new, pe_new, latent_pages, page_table,
                              len_in, len_out, scale, max_len, n_workgroups=0,
                              out=None, lse=None):
    """Append the new latent (c_new [B, 1, 512], pe_new [B, 1, 64], unit last
    stride) at position len_in[b] and attend over the partition including it.
    Returns (out [B*H, 512] fp32, lse [B*H])."""
    dev = latent_pages.device
    _require(q_nope, "q_nope", torch.bfloat16, dev, 2)
    _require(q_pe, "q_pe", torch.bfloat16, dev, 2)
    _require(latent_pages, "latent_pages", torch.bfloat16, dev, 3)
    _require(page_table, "page_table", torch.int32, dev, 2)
    _require(len_in, "len_in", torch.int32, dev, 1)
    B = page_table.shape[0]
    for t, n, w in ((c_new, "c_new", MLA_C), (pe_new, "pe_new", MLA_PE)):
        _require(t, n, torch.bfloat16, dev, 3, contiguous=False)
        if t.shape != (B, 1, w) or t.stride(2) != 1:
            raise ValueError(f"{n} must be [B, 1, {w}] with unit last stride")
    P, PS, L = latent_pages.shape
    rows = q_nope.shape[0]
    if L != MLA_LATENT or q_nope.shape[1] != MLA_C or q_pe.shape != (rows, MLA_PE):
        raise ValueError("MLA layout is q_nope 512 + q_pe 64 over a 576 latent")
    if B == 0 or rows % B or len_in.shape[0] != B:
        raise ValueError("rows must be B * H with B = page_table.shape[0]")
    if len_out is not None:
        _require(len_out, "len_out", torch.int32, dev, 1)
        if len_out.shape[0] != B or len_out.data_ptr() == len_in.data_ptr():
            raise ValueError("len_out must be a separate [B] int32 tensor")
    H = rows // B
    if out is None:
        out = torch.empty((rows, MLA_C), dtype=torch.float32, device=dev)
    if lse is None:
        lse = torch.empty((rows,), dtype=torch.float32, device=dev)
    nwg, wsb = decode_plan(1, B, H, int(max_len), int(n_workgroups))
    ws = _workspace(dev, wsb)
    _check(lib().ws_mla_append_decode_partial(
        _ptr(q_nope), _ptr(q_pe), _ptr(c_new), c_new.stride(0), _ptr(pe_new),
        pe_new.stride(0), _ptr(latent_pages), _ptr(page_table), _ptr(len_in),
        _ptr(len_out), B, H, PS, page_table.shape[1], P, int(max_len), nwg, float(scale),
        _ptr(out), _ptr(lse), _ptr(ws), wsb, _stream(dev)), "ws_mla_append_decode_partial")
    return out, lse


class SplitStep:
    """A deferred-combine decode step: its GPU pieces (out_g/lse_g finals and
    the split partials in `workspace`) wait for merge_split.  Holds every
    buffer the merge reads, so the step's workspace is not reused early."""

    def __init__(self, gpu_len, B, rows_per_seq, heads, Dv, cap, nwg, out_g, lse_g,
                 workspace):
        self.gpu_len, self.B, self.rows_per_seq, self.heads = gpu_len, B, rows_per_seq, heads
        self.Dv, self.cap, self.nwg = Dv, cap, nwg
        self.out_g, self.lse_g, self.workspace = out_g, lse_g, workspace
        self.guard = None  # set by an owner that reuses the workspace

    def check_workspace(self):
        if self.guard is not None and not self.guard():
            raise RuntimeError("this step's workspace was reused by a later step before "
                               "its merge")


def gqa_append_decode_split(q, k_new, v_new, k_pages, v_pages, page_table, len_in,
                            len_out, scale, max_len, n_workgroups=0, workspace=None):
    """Deferred-combine fused step (ws_gqa_append_decode_split): append and
    attend like gqa_append_decode_partial, but rows spread over several
    splits (waves) are combined later by merge_split.  len_out is required (the
    merge reads the post-step lengths).  Returns a SplitStep."""
    dev = k_pages.device
    _require(q, "q", torch.bfloat16, dev, 3)
    _require(k_new, "k_new", torch.bfloat16, dev, 4)
    _require(v_new, "v_new", torch.bfloat16, dev, 4)
    _require(k_pages, "k_pages", torch.bfloat16, dev, 4)
    _require(v_pages, "v_pages", torch.bfloat16, dev, 4)
    _require(page_table, "page_table", torch.int32, dev, 2)
    _require(len_in, "len_in", torch.int32, dev, 1)
    _require(len_out, "len_out", torch.int32, dev, 1)
    B, Hq, D = q.shape
    P, Hkv, PS, D2 = k_pages.shape
    if v_pages.shape != k_pages.shape or D2 != D:
        raise ValueError("k/v page pools must match q's head_dim")
    if k_new.shape != (B, Hkv, 1, D) or v_new.shape != k_new.shape:
        raise ValueError(f"k_new/v_new must be [B, Hkv, 1, D] = {(B, Hkv, 1, D)}")
    if page_table.shape[0] != B or len_in.shape[0] != B or len_out.shape[0] != B:
        raise ValueError("page_table/len_in/len_out batch mismatch")
    if len_out.data_ptr() == len_in.data_ptr():
        raise ValueError("len_out must be a separate [B] int32 tensor")
    out = torch.empty((B, Hq, D), dtype=torch.float32, device=dev)
    lse = torch.empty((B, Hq), dtype=torch.float32, device=dev)
    nwg, wsb = gqa_plan(B * Hkv, Hq // Hkv, D, D, int(max_len), int(n_workgroups))
    if workspace is None:
        workspace = torch.zeros(max(wsb, 256), dtype=torch.uint8, device=dev)
    elif workspace.numel() * workspace.element_size() < wsb:
        raise ValueError(f"workspace needs {wsb} bytes")
    return _gqa_split_launch(q, k_new, v_new, k_pages, v_pages, page_table, len_in, len_out,
                             scale, max_len, nwg, out, lse, workspace)


def _gqa_split_launch(q, k_new, v_new, k_pages, v_pages, page_table, len_in, len_out, scale,
                      max_len, nwg, out, lse, workspace) -> SplitStep:
    """The ws_gqa_append_decode_split launch on arguments already checked
    (gqa_append_decode_split, or a cache that owns the pools, page table,
    lengths, partial buffers and workspace); returns the SplitStep."""
    B, Hq, D = q.shape
    P, Hkv, PS, _ = k_pages.shape
    _check(lib().ws_gqa_append_decode_split(
        _ptr(q), _ptr(k_new), _ptr(v_new), _ptr(k_pages), _ptr(v_pages), _ptr(page_table),
        _ptr(len_in), _ptr(len_out), B, Hq, Hkv, D, PS, page_table.shape[1], P,
        int(max_len), nwg, float(scale), _ptr(out), _ptr(lse), _ptr(workspace),
        workspace.numel() * workspace.element_size(), _stream(k_pages.device)),
        "ws_gqa_append_decode_split")
    return SplitStep(len_out, B, Hkv, Hq // Hkv, D, PS * page_table.shape[1], nwg, out, lse,
                     workspace)


def mla_append_decode_split(q_nope, q_pe, c_new, pe_new, latent_pages, page_table,
                            len_in, len_out, scale, max_len, n_workgroups=0,
                            workspace=None):
    """Deferred-combine absorbed-MLA step (ws_mla_append_decode_split);
    finish with merge_split.  Returns a SplitStep."""
    dev = latent_pages.device
    _require(q_nope, "q_nope", torch.bfloat16, dev, 2)
    _require(q_pe, "q_pe", torch.bfloat16, dev, 2)
    _require(latent_pages, "latent_pages", torch.bfloat16, dev, 3)
    _require(page_table, "page_table", torch.int32, dev, 2)
    _require(len_in, "len_in", torch.int32, dev, 1)
    _require(len_out, "len_out", torch.int32, dev, 1)
    B = page_table.shape[0]
    for t, n, w in ((c_new, "c_new", MLA_C), (pe_new, "pe_new", MLA_PE)):
        _require(t, n, torch.bfloat16, dev, 3, contiguous=False)
        if t.shape != (B, 1, w) or t.stride(2) != 1:
            raise ValueError(f"{n} must be [B, 1, {w}] with unit last stride")
    P, PS, L = latent_pages.shape
    rows = q_nope.shape[0]
    if L != MLA_LATENT or q_nope.shape[1] != MLA_C or q_pe.shape != (rows, MLA_PE):
        raise ValueError("MLA layout is q_nope 512 + q_pe 64 over a 576 latent")
    if B == 0 or rows % B or len_in.shape[0] != B or len_out.shape[0] != B:
        raise ValueError("rows must be B * H with B = page_table.shape[0]")
    if len_out.data_ptr() == len_in.data_ptr():
        raise ValueError("len_out must be a separate [B] int32 tensor")
    H = rows // B
    out = torch.empty((rows, MLA_C), dtype=torch.float32, device=dev)
    lse = torch.empty((rows,), dtype=torch.float32, device=dev)
    nwg, wsb = decode_plan(1, B, H, int(max_len), int(n_workgroups))
    if workspace is None:
        workspace = torch.zeros(max(wsb, 256), dtype=torch.uint8, device=dev)
    elif workspace.numel() * workspace.element_size() < wsb:
        raise ValueError(f"workspace needs {wsb} bytes")
    return _mla_split_launch(q_nope, q_pe, c_new, pe_new, latent_pages, page_table, len_in,
                             len_out, scale, max_len, nwg, out, lse, workspace)


def _mla_split_launch(q_nope, q_pe, c_new, pe_new, latent_pages, page_table, len_in, len_out,
                      scale, max_len, nwg, out, lse, workspace) -> SplitStep:
    """The ws_mla_append_decode_split launch on arguments already checked
    (mla_append_decode_split, or a cache that owns the pools, page table,
    lengths, partial buffers and workspace); returns the SplitStep."""
    B = page_table.shape[0]
    P, PS, _ = latent_pages.shape
    H = q_nope.shape[0] // B
    _check(lib().ws_mla_append_decode_split(
        _ptr(q_nope), _ptr(q_pe), _ptr(c_new), c_new.stride(0), _ptr(pe_new),
        pe_new.stride(0), _ptr(latent_pages), _ptr(page_table), _ptr(len_in),
        _ptr(len_out), B, H, PS, page_table.shape[1], P, int(max_len), nwg, float(scale),
        _ptr(out), _ptr(lse), _ptr(workspace), workspace.numel() * workspace.element_size(),
        _stream(latent_pages.device)), "ws_mla_append_decode_split")
    return SplitStep(len_out, B, 1, H, MLA_C, PS * page_table.shape[1], nwg, out, lse,
                     workspace)


def merge_split(step: SplitStep, b=None, fmt=PARTIAL_LSE_F32, out_dtype=torch.bfloat16,
                want_lse=True, out=None, lse_out=None):
    """Finish a deferred-combine step (ws_merge_split): combine its GPU pieces
    with the host partial `b` (formats as lse_merge; None = no host partial),
    normalise.  Returns (out [rows, Dv] in out_dtype, lse [rows] or None)."""
    step.check_workspace()
    dev = step.out_g.device
    rows = step.out_g.numel() // step.Dv
    b_out, b_aux0, b_aux1 = _host_operand(b, fmt, rows, step.Dv, dev)
    if out is None:
        out = torch.empty((rows, step.Dv), dtype=out_dtype, device=dev)
    if want_lse and lse_out is None:
        lse_out = torch.empty((rows,), dtype=torch.float32, device=dev)
    o16, o32 = (out, None) if out.dtype == torch.bfloat16 else (None, out)
    if out.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError("merged output must be bfloat16 or float32")
    ws = step.workspace
    _check(lib().ws_merge_split(
        _ptr(step.gpu_len), step.B, step.rows_per_seq, step.heads, step.Dv, step.cap,
        step.nwg, _ptr(step.out_g), _ptr(step.lse_g), _ptr(ws), ws.numel() * ws.element_size(),
        _ptr(b_out), _ptr(b_aux0), _ptr(b_aux1), int(fmt), _ptr(o16), _ptr(o32),
        _ptr(lse_out if want_lse else None), _stream(dev)), "ws_merge_split")
    return out, (lse_out if want_lse else None)


def _require_operand(t, name, dtype, dev):
    """A merge's host operand: a tensor on `dev`, or a pinned host tensor,
    which the merge kernel reads in place over the host link."""
    if isinstance(t, torch.Tensor) and not t.is_cuda:
        if not t.is_pinned():
            raise ValueError(f"{name} must be on {dev} or in pinned host memory")
        if t.dtype != dtype:
            raise TypeError(f"{name} must be {dtype} (got {t.dtype})")
        if not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous")
        return
    _require(t, name, dtype, dev)


def _host_operand(b, fmt, rows, Dv, dev):
    """Pointers of the host partial `b` in format fmt (None: no host partial),
    validated against rows x Dv."""
    b_out = b_aux0 = b_aux1 = None
    if b is not None:
        if fmt in (PARTIAL_LSE_F32, PARTIAL_LSE_BF16):
            b_out, b_aux0 = b
            _require_operand(b_out, "b.out",
                             torch.float32 if fmt == PARTIAL_LSE_F32 else torch.bfloat16, dev)
            _require_operand(b_aux0, "b.lse", torch.float32, dev)
        elif fmt in (TRIPLE_UNNORM_F32, TRIPLE_NORM_BF16, TRIPLE_NORM_F32):
            b_out, b_aux0, b_aux1 = b
            dt = torch.bfloat16 if fmt == TRIPLE_NORM_BF16 else torch.float32
            _require_operand(b_out, "b.out", dt, dev)
            _require_operand(b_aux0, "b.max", dt, dev)
            _require_operand(b_aux1, "b.sum", dt, dev)
            if b_aux1.numel() != rows:
                raise ValueError("b.sum must have one value per row")
        else:
            raise ValueError(f"unknown host-partial format {fmt}")
        if b_out.numel() != rows * Dv or b_aux0.numel() != rows:
            raise ValueError("host partial does not match the step's rows")
    return b_out, b_aux0, b_aux1


def merge_split_uv(step: SplitStep, w_uv: torch.Tensor, b=None, fmt=PARTIAL_LSE_F32,
                   want_latent=False, want_lse=False):
    """Finish an absorbed-MLA split step with the W_UV epilogue
    (ws_mla_merge_split_uv): w_uv [heads, Dout, 512] bf16.  Returns
    (out_v [B, heads * Dout] bf16, latent [B * heads, 512] bf16 or None,
    lse [B * heads] or None)."""
    step.check_workspace()
    dev = step.out_g.device
    if step.rows_per_seq != 1 or step.Dv != MLA_C:
        raise ValueError("merge_split_uv finishes an MLA step")
    H = step.heads
    _require(w_uv, "w_uv", torch.bfloat16, dev, 3)
    if w_uv.shape[0] != H or w_uv.shape[2] != MLA_C:
        raise ValueError(f"w_uv must be [{H}, Dout, {MLA_C}]")
    Dout = w_uv.shape[1]
    rows = step.B * H
    b_out, b_aux0, b_aux1 = _host_operand(b, fmt, rows, MLA_C, dev)
    out_v = torch.empty((step.B, H * Dout), dtype=torch.bfloat16, device=dev)
    latent = (torch.empty((rows, MLA_C), dtype=torch.bfloat16, device=dev)
              if want_latent else None)
    lse = torch.empty((rows,), dtype=torch.float32, device=dev) if want_lse else None
    ws = step.workspace
    _check(lib().ws_mla_merge_split_uv(
        _ptr(step.gpu_len), step.B, H, step.cap, step.nwg, _ptr(step.out_g), _ptr(step.lse_g),
        _ptr(ws), ws.numel() * ws.element_size(), _ptr(b_out), _ptr(b_aux0), _ptr(b_aux1),
        int(fmt), _ptr(w_uv), Dout, _ptr(latent), _ptr(out_v), _ptr(lse), _stream(dev)),
        "ws_mla_merge_split_uv")
    return out_v, latent, lse


def split_reduce(part_out, part_lse, gpu_len, heads_per_len, tokens_per_split,
                 out=None, lse=None):
    """LSE-combine split partials part_out [n_splits, rows, Dv],
    part_lse [n_splits, rows] (see ws_split_reduce)."""
    dev = part_out.device
    _require(part_out, "part_out", torch.float32, dev, 3)
    _require(part_lse, "part_lse", torch.float32, dev, 2)
    _require(gpu_len, "gpu_len", torch.int32, dev, 1)
    ns, rows, Dv = part_out.shape
    if out is None:
        out = torch.empty((rows, Dv), dtype=torch.float32, device=dev)
    if lse is None:
        lse = torch.empty((rows,), dtype=torch.float32, device=dev)
    _check(lib().ws_split_reduce(_ptr(part_out), _ptr(part_lse), _ptr(gpu_len), rows,
                                 int(heads_per_len), Dv, ns, int(tokens_per_split),
                                 _ptr(out), _ptr(lse), _stream(dev)), "ws_split_reduce")
    return out, lse


# ---------------------------------------------------------------------------
# merge


def lse_merge(out_g, lse_g, b, fmt=PARTIAL_LSE_F32, out_dtype=torch.bfloat16,
              want_lse=True, out=None, lse_out=None):
    """Merge the GPU partial (out_g [..., Dv] fp32, lse_g [...] fp32) with a
    second partial `b`:
      fmt PARTIAL_LSE_F32   b = (out fp32, lse fp32)
      fmt TRIPLE_UNNORM_F32 b = (o unnormalised fp32, max fp32, sum fp32)
      fmt TRIPLE_NORM_BF16  b = (out bf16 normalised, max bf16, sum bf16)
      fmt TRIPLE_NORM_F32   b = (out fp32 normalised, max fp32, sum fp32)
      fmt PARTIAL_LSE_BF16  b = (out bf16 normalised, lse fp32)
    Returns (merged out in out_dtype (bf16 or fp32), lse fp32 or None)."""
    dev = out_g.device
    _require(out_g, "out_g", torch.float32, dev)
    _require(lse_g, "lse_g", torch.float32, dev)
    Dv = out_g.shape[-1]
    rows = out_g.numel() // Dv
    if lse_g.numel() != rows:
        raise ValueError("lse_g must have one value per output row")
    if b is None:
        raise ValueError("lse_merge needs a second partial")
    b_out, b_aux0, b_aux1 = _host_operand(b, fmt, rows, Dv, dev)
    if out is None:
        out = torch.empty(out_g.shape, dtype=out_dtype, device=dev)
    if want_lse and lse_out is None:
        lse_out = torch.empty(lse_g.shape, dtype=torch.float32, device=dev)
    if out.dtype == torch.bfloat16:
        o16, o32 = out, None
    elif out.dtype == torch.float32:
        o16, o32 = None, out
    else:
        raise TypeError("merged output must be bfloat16 or float32")
    _require(out, "out", out.dtype, dev)
    _check(lib().ws_lse_merge(_ptr(out_g), _ptr(lse_g), _ptr(b_out), _ptr(b_aux0),
                              _ptr(b_aux1), int(fmt), _ptr(o16), _ptr(o32),
                              _ptr(lse_out if want_lse else None), rows, Dv,
                              _stream(dev)), "ws_lse_merge")
    return out, (lse_out if want_lse else None)
