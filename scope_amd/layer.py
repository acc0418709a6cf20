"""The two-sided decode layer in one native call (scope_amd/lib/libwslayer.so,
include/wslayer.h).

wl_mla_layer / wl_gqa_layer run, without Python in between and with the GIL
released: the query to pinned host memory (ws_copy), the GPU split step with
the fused append, the wait for the query, the host partial over the host pages
(bf16 out) and the merge that reads it in place (or the W_UV epilogue).  The
paged caches (scope_amd/paged.py) drive their decode steps through it; the
structures below mirror the C ones field for field (checked against the
library's own sizeof at load).
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libwslayer.so")

EXPORTS = ("wl_mla_layer", "wl_gqa_layer", "wl_last_error", "wl_struct_size")

vp, i32, i64, f32, f64, sz = (ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float,
                              ctypes.c_double, ctypes.c_size_t)


class WlMlaLayer(ctypes.Structure):
    _fields_ = [
        ("q_nope", vp), ("q_pe", vp), ("c_new", vp), ("c_stride", i64), ("pe_new", vp),
        ("pe_stride", i64), ("latent_pages", vp), ("page_table", vp), ("len_in", vp),
        ("len_out", vp), ("B", i32), ("H", i32), ("page_size", i32), ("max_pages", i32),
        ("num_pages", i32), ("max_len", i32), ("n_splits", i32), ("scale", f32),
        ("out_g", vp), ("lse_g", vp), ("workspace", vp), ("workspace_bytes", sz),
        ("ev_step_begin", vp), ("ev_step_end", vp),
        ("q_nope_h", vp), ("q_pe_h", vp), ("host_latent", vp), ("host_table", vp),
        ("host_lens", vp), ("host_page_size", i32), ("host_max_pages", i32),
        ("host_num_pages", i32), ("host_threads", i32), ("out_h", vp), ("lse_h", vp),
        ("out", vp), ("lse_out", vp), ("w_uv", vp), ("Dout", i32), ("out_v", vp),
        ("host_seconds", f64), ("stage", i32),
    ]


class WlGqaLayer(ctypes.Structure):
    _fields_ = [
        ("q", vp), ("k_new", vp), ("v_new", vp), ("k_pages", vp), ("v_pages", vp),
        ("page_table", vp), ("len_in", vp), ("len_out", vp), ("B", i32), ("Hq", i32),
        ("Hkv", i32), ("D", i32), ("page_size", i32), ("max_pages", i32), ("num_pages", i32),
        ("max_len", i32), ("n_splits", i32), ("scale", f32), ("out_g", vp), ("lse_g", vp),
        ("workspace", vp), ("workspace_bytes", sz), ("ev_step_begin", vp),
        ("ev_step_end", vp), ("q_h", vp), ("host_k", vp), ("host_v", vp), ("host_table", vp),
        ("host_lens", vp), ("host_page_size", i32), ("host_max_pages", i32),
        ("host_num_pages", i32), ("host_threads", i32), ("out_h", vp), ("lse_h", vp),
        ("out", vp), ("lse_out", vp), ("host_seconds", f64), ("stage", i32),
    ]


class WlError(RuntimeError):
    """A libwslayer entry point returned an error."""

    def __init__(self, msg, stage):
        super().__init__(msg)
        self.stage = stage  # 0 nothing launched, 1 split step launched, 2 merge launched


_lib = None


def lib() -> ctypes.CDLL:
    """Load libwslayer.so (after libwsgpu.so and libwshost.so, which it links;
    torch is imported first so that the process keeps a single HIP runtime)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is not built; run `python -m scope_amd._build` "
                "(or __graft_entry__.build())")
        import torch  # noqa: F401
        from . import host, ops

        ops.lib()
        host.lib()
        L = ctypes.CDLL(LIB_PATH)
        L.wl_last_error.restype = ctypes.c_char_p
        L.wl_last_error.argtypes = []
        L.wl_struct_size.restype = sz
        L.wl_struct_size.argtypes = [i32]
        L.wl_mla_layer.restype = i32
        L.wl_mla_layer.argtypes = [ctypes.POINTER(WlMlaLayer), vp]
        L.wl_gqa_layer.restype = i32
        L.wl_gqa_layer.argtypes = [ctypes.POINTER(WlGqaLayer), vp]
        for which, st in ((0, WlMlaLayer), (1, WlGqaLayer)):
            if L.wl_struct_size(which) != ctypes.sizeof(st):
                raise RuntimeError(f"{st.__name__}: {ctypes.sizeof(st)} bytes here, "
                                   f"{L.wl_struct_size(which)} in the library")
        _lib = L
    return _lib


def run(fn, args, stream) -> None:
    """Runs wl_mla_layer / wl_gqa_layer on a filled structure; raises WlError
    (with the stage the call reached) on failure."""
    rc = fn(ctypes.byref(args), stream)
    if rc != 0:
        raise WlError(f"{lib().wl_last_error().decode()} (rc={rc})", args.stage)
