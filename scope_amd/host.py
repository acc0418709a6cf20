"""Host partial of the partitioned decode KV cache (scope_amd/lib/libwshost.so).

Attention over the host segment of every sequence, on the CPU, with the
AVX-512 BF16 kernels of include/wshost.h.  It returns the normalised fp32
partial and its natural-log LSE, the form ops.lse_merge / ops.merge_split take
as PARTIAL_LSE_F32.  It is the production counterpart of the reference CPU
kernels (kernel/cpu_attn.cpp:572-1022): one call per layer covers a ragged
batch (each sequence its own length) and releases the GIL (ctypes), so the
calling thread can launch GPU work first and run this while it executes.

Tensor conventions (CPU tensors, contiguous; pinned memory is fine).  The
host segment is paged like the GPU partition (same pool layouts, page table
and lengths), so the boundary moves by copying pages; the *_dense helpers
take the reference's dense host arrays (one page per sequence):
  GQA  q [B, Hq, D] bf16; k_pages, v_pages [num_pages, Hkv, page_size, D]
       bf16 (dense: k, v [B*Hkv, cap, D])
  MLA  q_nope [B*16, 512], q_pe [B*16, 64] bf16; latent_pages
       [num_pages, page_size, 576] bf16 (dense: c [B, cap, 512], pe [B, cap, 64])
  page_table [B, max_pages] int32, lens [B] int32 host tokens
  out  fp32 (or bf16: the *_bf16 entry points) [B, Hq, D] / [B*16, 512];
       lse fp32 [B, Hq] / [B*16]
There is no fallback: a missing library or a CPU without AVX-512 BF16 raises.
"""
from __future__ import annotations

import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libwshost.so")

# Entry points declared in include/wshost.h.
EXPORTS = ("wh_last_error", "wh_version", "wh_isa_supported", "wh_gqa_partial",
           "wh_gqa_partial_bf16", "wh_attn_partial", "wh_attn_partial_f32", "wh_host_read_gbs",
           "wh_mla_partial", "wh_mla_partial_bf16", "wh_attn_triple", "wh_attn_triple_f32",
           "wh_mla_triple")

MLA_HEADS = 16
MLA_C = 512
MLA_PE = 64


class WhError(RuntimeError):
    """A libwshost entry point returned an error."""


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is not built; run `python -m scope_amd._build` "
                "(or __graft_entry__.build())")
        L = ctypes.CDLL(LIB_PATH)
        vp, i32, f32 = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
        L.wh_last_error.restype = ctypes.c_char_p
        L.wh_last_error.argtypes = []
        L.wh_version.restype = ctypes.c_char_p
        L.wh_version.argtypes = []
        L.wh_isa_supported.restype = i32
        L.wh_isa_supported.argtypes = []
        L.wh_gqa_partial.restype = i32
        L.wh_gqa_partial.argtypes = [vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, i32, f32,
                                     vp, vp, i32]
        L.wh_attn_partial.restype = i32
        L.wh_attn_partial.argtypes = [vp, vp, vp, vp, vp] + [i32] * 8 + [f32, vp, vp, i32]
        L.wh_attn_partial_f32.restype = i32
        L.wh_attn_partial_f32.argtypes = L.wh_attn_partial.argtypes
        L.wh_host_read_gbs.restype = ctypes.c_double
        L.wh_host_read_gbs.argtypes = [ctypes.c_size_t, i32, i32]
        L.wh_gqa_partial_bf16.restype = i32
        L.wh_gqa_partial_bf16.argtypes = L.wh_gqa_partial.argtypes
        L.wh_mla_partial.restype = i32
        L.wh_mla_partial.argtypes = [vp, vp, vp, i32, vp, i32, vp, vp] + [i32] * 5 + [f32, vp,
                                                                                     vp, i32]
        L.wh_mla_partial_bf16.restype = i32
        L.wh_mla_partial_bf16.argtypes = L.wh_mla_partial.argtypes
        for name in ("wh_attn_triple", "wh_attn_triple_f32"):
            getattr(L, name).restype = i32
            getattr(L, name).argtypes = [vp, vp, vp, vp, vp] + [i32] * 8 + [f32, i32, vp, vp,
                                                                             vp, i32]
        L.wh_mla_triple.restype = i32
        L.wh_mla_triple.argtypes = [vp, vp, vp, i32, vp, i32, vp, vp] + [i32] * 5 + [
            f32, i32, vp, vp, vp, i32]
        _lib = L
    return _lib


def host_read_gbs(nbytes: int = 1 << 30, threads: int = 0, reps: int = 5) -> float:
    """Streaming read bandwidth of host memory in GB/s with `threads` threads
    (wh_host_read_gbs): the host side's roofline."""
    return float(lib().wh_host_read_gbs(int(nbytes), int(threads), int(reps)))


def isa_supported() -> bool:
    return bool(lib().wh_isa_supported())


def _check(rc: int) -> None:
    if rc != 0:
        raise WhError(f"libwshost error {rc}: {lib().wh_last_error().decode()}")


def _cpu(t: torch.Tensor, dtype, name: str) -> None:
    if t.device.type != "cpu":
        raise ValueError(f"{name} must be a CPU tensor, got {t.device}")
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def _p(t):
    return ctypes.c_void_p(t.data_ptr()) if t.numel() else ctypes.c_void_p(0)


def _lens(lens, B):
    if not isinstance(lens, torch.Tensor):
        lens = torch.as_tensor(lens, dtype=torch.int32)
    lens = lens.to(torch.int32).contiguous()
    if lens.device.type != "cpu" or lens.shape != (B,):
        raise ValueError(f"lens must be a CPU int32 tensor of shape ({B},)")
    return lens


def _table(page_table, B):
    page_table = torch.as_tensor(page_table, dtype=torch.int32)
    if page_table.device.type != "cpu" or page_table.dim() != 2 or page_table.shape[0] != B:
        raise ValueError(f"page_table must be a CPU int32 tensor [B={B}, max_pages]")
    return page_table.contiguous()


def _outputs(out, lse, out_shape, lse_shape, out_dtype=torch.float32):
    """The output buffers: out fp32, or bf16 (the *_bf16 entry points), as
    given or allocated in out_dtype; lse fp32."""
    if out is None:
        out = torch.empty(out_shape, dtype=out_dtype)
    if lse is None:
        lse = torch.empty(lse_shape, dtype=torch.float32)
    if out.dtype not in (torch.float32, torch.bfloat16):
        raise TypeError(f"out must be float32 or bfloat16 (got {out.dtype})")
    _cpu(out, out.dtype, "out")
    _cpu(lse, torch.float32, "lse")
    if tuple(out.shape) != tuple(out_shape) or tuple(lse.shape) != tuple(lse_shape):
        raise ValueError(f"out/lse must be {tuple(out_shape)} / {tuple(lse_shape)}")
    return out, lse


class Prepared:
    """A validated host-partial call bound to its buffers: calling it runs the
    kernel again on whatever the buffers (queries, pools, page table, lengths)
    hold now and overwrites its out / lse.  For decode loops that reuse their
    buffers, it skips the per-call argument checks and marshalling (tens of
    microseconds of Python per call)."""

    def __init__(self, fn, args, keep):
        self._fn = fn
        self._args = args
        self._keep = keep  # the bound tensors stay alive with the call
        self.out, self.lse = keep[-2], keep[-1]

    def __call__(self):
        _check(self._fn(*self._args))
        return self.out, self.lse


def gqa_partial(q: torch.Tensor, k_pages: torch.Tensor, v_pages: torch.Tensor, page_table,
                lens, scale: float, threads: int = 0, out: torch.Tensor | None = None,
                lse: torch.Tensor | None = None, prepare: bool = False,
                out_dtype=torch.float32):
    """(out [B, Hq, D], lse fp32 [B, Hq]) over paged host KV pools
    k_pages / v_pages [num_pages, Hkv, page_size, D] (the GPU pool layout);
    out fp32, or bf16 (wh_gqa_partial_bf16) when out / out_dtype is bf16.
    prepare=True returns a Prepared call instead of running it."""
    B, Hq, D = q.shape
    _cpu(q, torch.bfloat16, "q")
    _cpu(k_pages, torch.bfloat16, "k_pages")
    _cpu(v_pages, torch.bfloat16, "v_pages")
    if k_pages.dim() != 4 or v_pages.shape != k_pages.shape or k_pages.shape[3] != D:
        raise ValueError(f"pools must be [num_pages, Hkv, page_size, {D}], got "
                         f"{tuple(k_pages.shape)} / {tuple(v_pages.shape)}")
    num_pages, Hkv, ps, _ = k_pages.shape
    table = _table(page_table, B)
    lens = _lens(lens, B)
    out, lse = _outputs(out, lse, (B, Hq, D), (B, Hq), out_dtype)
    fn = lib().wh_gqa_partial_bf16 if out.dtype == torch.bfloat16 else lib().wh_gqa_partial
    call = Prepared(fn,
                    (_p(q), _p(k_pages), _p(v_pages), _p(table), _p(lens), B, Hq, Hkv, D, ps,
                     table.shape[1], num_pages, ctypes.c_float(scale), _p(out), _p(lse),
                     int(threads)),
                    (q, k_pages, v_pages, table, lens, out, lse))
    if prepare:
        return call
    call()
    return out, lse


def attn_partial(q: torch.Tensor, k_pages: torch.Tensor, v_pages: torch.Tensor, page_table,
                 lens, scale: float, threads: int = 0, out: torch.Tensor | None = None,
                 lse: torch.Tensor | None = None):
    """gqa_partial with separate key / value widths (wh_attn_partial):
    q [B, Hq, Dk], k_pages [num_pages, Hkv, page_size, Dk], v_pages
    [num_pages, Hkv, page_size, Dv] -> (out fp32 [B, Hq, Dv], lse fp32
    [B, Hq]).  (Dk, Dv): equal, or (192, 128).  bf16 inputs, or float32 ones
    (wh_attn_partial_f32: fp32 FMAs and probabilities, widths multiples of
    16)."""
    B, Hq, Dk = q.shape
    dt = q.dtype if q.dtype in (torch.bfloat16, torch.float32) else torch.bfloat16
    _cpu(q, dt, "q")
    _cpu(k_pages, dt, "k_pages")
    _cpu(v_pages, dt, "v_pages")
    if k_pages.dim() != 4 or v_pages.dim() != 4 or k_pages.shape[:3] != v_pages.shape[:3] \
            or k_pages.shape[3] != Dk:
        raise ValueError(f"pools must be [num_pages, Hkv, page_size, Dk / Dv], got "
                         f"{tuple(k_pages.shape)} / {tuple(v_pages.shape)}")
    num_pages, Hkv, ps, _ = k_pages.shape
    Dv = v_pages.shape[3]
    table = _table(page_table, B)
    lens = _lens(lens, B)
    out, lse = _outputs(out, lse, (B, Hq, Dv), (B, Hq))
    if out.dtype != torch.float32:
        raise TypeError("attn_partial writes a float32 out")
    fn = lib().wh_attn_partial_f32 if dt == torch.float32 else lib().wh_attn_partial
    _check(fn(_p(q), _p(k_pages), _p(v_pages), _p(table), _p(lens), B, Hq, Hkv, Dk, Dv, ps,
              table.shape[1], num_pages, ctypes.c_float(scale), _p(out), _p(lse),
              int(threads)))
    return out, lse


def attn_triple(q: torch.Tensor, k_pages: torch.Tensor, v_pages: torch.Tensor, page_table,
                lens, scale: float, normalize: bool, threads: int = 0):
    """The reference CPU kernel's triple over paged pools (wh_attn_triple /
    _f32): fp32 (out [B, Hq, Dv], row_max [B, Hq], row_sum [B, Hq]) with
    row_max the largest scaled score, row_sum the sum of exp(score - row_max)
    and out divided by row_sum when `normalize`.  Shapes and dtypes as
    attn_partial."""
    B, Hq, Dk = q.shape
    dt = q.dtype if q.dtype in (torch.bfloat16, torch.float32) else torch.bfloat16
    _cpu(q, dt, "q")
    _cpu(k_pages, dt, "k_pages")
    _cpu(v_pages, dt, "v_pages")
    if k_pages.dim() != 4 or v_pages.dim() != 4 or k_pages.shape[:3] != v_pages.shape[:3] \
            or k_pages.shape[3] != Dk:
        raise ValueError(f"pools must be [num_pages, Hkv, page_size, Dk / Dv], got "
                         f"{tuple(k_pages.shape)} / {tuple(v_pages.shape)}")
    num_pages, Hkv, ps, _ = k_pages.shape
    Dv = v_pages.shape[3]
    table = _table(page_table, B)
    lens = _lens(lens, B)
    out = torch.empty((B, Hq, Dv), dtype=torch.float32)
    mx = torch.empty((B, Hq), dtype=torch.float32)
    sm = torch.empty((B, Hq), dtype=torch.float32)
    fn = lib().wh_attn_triple_f32 if dt == torch.float32 else lib().wh_attn_triple
    _check(fn(_p(q), _p(k_pages), _p(v_pages), _p(table), _p(lens), B, Hq, Hkv, Dk, Dv, ps,
              table.shape[1], num_pages, ctypes.c_float(scale), int(bool(normalize)), _p(out),
              _p(mx), _p(sm), int(threads)))
    return out, mx, sm


def mla_triple_dense(q_nope: torch.Tensor, q_pe: torch.Tensor, c: torch.Tensor,
                     pe: torch.Tensor, lens, scale: float, normalize: bool, threads: int = 0):
    """The reference's MLA triple (wh_mla_triple) over the dense host arrays
    c [B, cap, 512], pe [B, cap, 64]: fp32 (out [B*H, 512], row_max [B*H],
    row_sum [B*H]), out unnormalised unless `normalize`."""
    B, cap, Dc = c.shape
    _cpu(c, torch.bfloat16, "c")
    _cpu(pe, torch.bfloat16, "pe")
    _cpu(q_nope, torch.bfloat16, "q_nope")
    _cpu(q_pe, torch.bfloat16, "q_pe")
    rows = q_nope.shape[0]
    if Dc != MLA_C or tuple(pe.shape) != (B, cap, MLA_PE) or B == 0 or \
            rows % (B * MLA_HEADS) or tuple(q_nope.shape) != (rows, MLA_C) or \
            tuple(q_pe.shape) != (rows, MLA_PE):
        raise ValueError(f"q_nope [B*H, 512], q_pe [B*H, 64], c [B, cap, 512], pe "
                         f"[B, cap, 64] with H a multiple of 16; got {tuple(q_nope.shape)}, "
                         f"{tuple(q_pe.shape)}, {tuple(c.shape)}, {tuple(pe.shape)}")
    table = torch.arange(B, dtype=torch.int32).view(B, 1)
    lens = _lens(lens, B)
    out = torch.empty((rows, MLA_C), dtype=torch.float32)
    mx = torch.empty((rows,), dtype=torch.float32)
    sm = torch.empty((rows,), dtype=torch.float32)
    _check(lib().wh_mla_triple(_p(q_nope), _p(q_pe), _p(c), MLA_C, _p(pe), MLA_PE, _p(table),
                               _p(lens), B, rows // B, max(cap, 1), 1, B,
                               ctypes.c_float(scale), int(bool(normalize)), _p(out), _p(mx),
                               _p(sm), int(threads)))
    return out, mx, sm


def gqa_partial_dense(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, lens, scale: float,
                      threads: int = 0, out=None, lse=None):
    """gqa_partial over the reference's dense host rows k, v [B*Hkv, cap, D]
    (row b*Hkv + kvh): one page of cap tokens per sequence."""
    B = q.shape[0]
    R, cap, D = k.shape
    if B == 0 or R % B != 0 or v.shape != k.shape:
        raise ValueError(f"shape mismatch q {tuple(q.shape)} k {tuple(k.shape)} "
                         f"v {tuple(v.shape)}")
    Hkv = R // B
    table = torch.arange(B, dtype=torch.int32).view(B, 1)
    return gqa_partial(q, k.view(B, Hkv, cap, D), v.view(B, Hkv, cap, D), table, lens, scale,
                       threads, out, lse)


def mla_partial(q_nope: torch.Tensor, q_pe: torch.Tensor, latent_pages: torch.Tensor,
                page_table, lens, scale: float, threads: int = 0, out=None, lse=None,
                prepare: bool = False, out_dtype=torch.float32):
    """(out [B*H, 512], lse fp32 [B*H]) over a paged host latent pool
    latent_pages [num_pages, page_size, 576] (the GPU pool layout: 512 latent
    then 64 rope per token); out fp32, or bf16 (wh_mla_partial_bf16) when
    out / out_dtype is bf16.  prepare=True returns a Prepared call."""
    _cpu(latent_pages, torch.bfloat16, "latent_pages")
    if latent_pages.dim() != 3 or latent_pages.shape[2] != MLA_C + MLA_PE:
        raise ValueError(f"latent_pages must be [num_pages, page_size, 576], got "
                         f"{tuple(latent_pages.shape)}")
    num_pages, ps, W = latent_pages.shape
    pe_view = latent_pages.view(-1)[MLA_C:]
    return _mla_call(q_nope, q_pe, latent_pages, W, pe_view, W, page_table, lens, ps,
                     num_pages, scale, threads, out, lse, prepare, out_dtype)


def mla_partial_dense(q_nope: torch.Tensor, q_pe: torch.Tensor, c: torch.Tensor,
                      pe: torch.Tensor, lens, scale: float, threads: int = 0, out=None,
                      lse=None):
    """mla_partial over the reference's separate dense host arrays
    c [B, cap, 512], pe [B, cap, 64] (system/deepseek.py:161-166): one page of
    cap tokens per sequence."""
    B, cap, Dc = c.shape
    _cpu(c, torch.bfloat16, "c")
    _cpu(pe, torch.bfloat16, "pe")
    if Dc != MLA_C or tuple(pe.shape) != (B, cap, MLA_PE):
        raise ValueError(f"c must be [B, cap, 512] and pe [B, cap, 64], got "
                         f"{tuple(c.shape)} / {tuple(pe.shape)}")
    table = torch.arange(B, dtype=torch.int32).view(B, 1)
    return _mla_call(q_nope, q_pe, c, MLA_C, pe, MLA_PE, table, lens, max(cap, 1), B, scale,
                     threads, out, lse)


def _mla_call(q_nope, q_pe, c, c_stride, pe, pe_stride, page_table, lens, page_size,
              num_pages, scale, threads, out, lse, prepare=False, out_dtype=torch.float32):
    _cpu(q_nope, torch.bfloat16, "q_nope")
    _cpu(q_pe, torch.bfloat16, "q_pe")
    rows = q_nope.shape[0]
    table = torch.as_tensor(page_table, dtype=torch.int32)
    B = table.shape[0] if table.dim() == 2 else 0
    # H = q rows / B, any multiple of 16 (kernel/cpu_attn.cpp:860 takes nH the same way)
    if B == 0 or rows % (B * MLA_HEADS) or q_nope.shape != (rows, MLA_C) or \
            q_pe.shape != (rows, MLA_PE):
        raise ValueError(f"q_nope must be [B*H, 512] and q_pe [B*H, 64] with H a multiple "
                         f"of 16 and B = page_table rows, got {tuple(q_nope.shape)} / "
                         f"{tuple(q_pe.shape)}, {B} sequences")
    H = rows // B
    table = _table(page_table, B)
    lens = _lens(lens, B)
    out, lse = _outputs(out, lse, (rows, MLA_C), (rows,), out_dtype)
    fn = lib().wh_mla_partial_bf16 if out.dtype == torch.bfloat16 else lib().wh_mla_partial
    call = Prepared(fn,
                    (_p(q_nope), _p(q_pe), _p(c), int(c_stride), _p(pe), int(pe_stride),
                     _p(table), _p(lens), B, H, int(page_size), table.shape[1], int(num_pages),
                     ctypes.c_float(scale), _p(out), _p(lse), int(threads)),
                    (q_nope, q_pe, c, pe, table, lens, out, lse))
    if prepare:
        return call
    call()
    return out, lse
