"""ctypes binding of the oracle's C restatement (tests / CPU baseline only).

Functions mirror the reference CPU entry points' contracts
(kernel/cpu_attn.cpp:572-672, 852-1022) on numpy arrays; bf16 is uint16.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "libwsoracle.so")
_lib = None


def build() -> str:
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        vp, i32, i64, f32 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float
        L.ws_oracle_gqa.argtypes = [vp, vp, vp, i32, i32, i32, i32, i32, i32,
                                    i64, i64, i64, i64, f32, i32, i32, vp, vp, vp]
        L.ws_oracle_gqa.restype = None
        L.ws_oracle_mla_compressed.argtypes = [vp, vp, vp, vp, i32, i32, i32, f32,
                                               i32, vp, vp, vp]
        L.ws_oracle_mla_compressed.restype = None
        _lib = L
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def cpu_attn(q, k, v, scale, normalize=True, n_threads=0):
    """fused_cpu_attn (normalize=True) / fused_cpu_attn_mla (False) contract.

    q [B_kv, G, Dk] contiguous; k [B_kv, S, Dk], v [B_kv, S, Dv] with a
    contiguous last dim (row strides honoured, kernel/cpu_attn.cpp:598-601).
    Dtype uint16 (bf16 bits) or float32, all equal.  Returns fp32
    (out [B_kv, G, Dv], max [B_kv, G, 1], sum [B_kv, G, 1]).
    """
    q = np.ascontiguousarray(q)
    if not (q.dtype == k.dtype == v.dtype) or q.dtype not in (np.uint16, np.float32):
        raise TypeError("q, k, v must share dtype uint16 (bf16) or float32")
    if k.strides[2] != k.itemsize or v.strides[2] != v.itemsize:
        raise ValueError("k/v last dim must be contiguous")
    B, G, Dk = q.shape
    S, Dv = k.shape[1], v.shape[2]
    out = np.zeros((B, G, Dv), np.float32)
    mx = np.zeros((B, G, 1), np.float32)
    sm = np.zeros((B, G, 1), np.float32)
    it = k.itemsize
    lib().ws_oracle_gqa(_p(q), _p(k), _p(v), int(q.dtype == np.uint16), B, G, Dk, Dv, S,
                        k.strides[0] // it, k.strides[1] // it,
                        v.strides[0] // it, v.strides[1] // it,
                        float(scale), int(normalize), int(n_threads),
                        _p(out), _p(mx), _p(sm))
    return out, mx, sm


def cpu_attn_mla_compressed(q_proj, q_pe, c_kv, k_pe, scale, n_threads=0):
    """fused_cpu_attn_mla_compressed contract: returns fp32 unnormalised
    out [B*H, 512], max [B*H], sum [B*H] (kernel/cpu_attn.cpp:852-1022)."""
    q_proj = np.ascontiguousarray(q_proj, np.uint16)
    q_pe = np.ascontiguousarray(q_pe, np.uint16)
    c_kv = np.ascontiguousarray(c_kv, np.uint16)
    k_pe = np.ascontiguousarray(k_pe, np.uint16)
    B, S = c_kv.shape[0], c_kv.shape[1]
    H = q_proj.shape[0] // B
    if q_proj.shape[1] != 512 or q_pe.shape[1] != 64 or c_kv.shape[2] != 512 or k_pe.shape[2] != 64:
        raise ValueError("MLA compressed layout is 512 latent + 64 rope")
    out = np.zeros((B * H, 512), np.float32)
    mx = np.zeros((B * H,), np.float32)
    sm = np.zeros((B * H,), np.float32)
    lib().ws_oracle_mla_compressed(_p(q_proj), _p(q_pe), _p(c_kv), _p(k_pe), B, H, S,
                                   float(scale), int(n_threads), _p(out), _p(mx), _p(sm))
    return out, mx, sm
