"""Seeded inputs shared by the CPU and GPU tests.

Inputs are drawn as fp32 normal * sigma from torch.Generator('cpu') and
rounded to bf16, so the oracle (numpy, uint16 bit patterns) and the GPU see
bit-identical data.
"""
from __future__ import annotations

import numpy as np
import torch

# Tolerances of the parity bar: bf16 outputs 2e-2 abs/rel, fp32 LSE 1e-3.
OUT_ATOL = OUT_RTOL = 2e-2
LSE_ATOL = LSE_RTOL = 1e-3


def bf16_randn(shape, seed, sigma=1.0):
    g = torch.Generator(device="cpu").manual_seed(seed)
    return (torch.randn(shape, generator=g, dtype=torch.float32) * sigma).to(torch.bfloat16)


def bits(t: torch.Tensor) -> np.ndarray:
    """bf16 tensor -> numpy uint16 bit patterns (CPU copy)."""
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def assert_close(got, want, atol, rtol, what=""):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, (what, got.shape, want.shape)
    same_inf = np.isinf(got) & np.isinf(want) & (np.sign(got) == np.sign(want))
    with np.errstate(invalid="ignore"):
        err = np.abs(got - want)
    bad = ~same_inf & ~(err <= atol + rtol * np.abs(want))
    if bad.any():
        idx = np.argwhere(bad)[0]
        raise AssertionError(
            f"{what}: {bad.sum()} / {bad.size} elements out of tolerance; first at "
            f"{tuple(idx)}: got {got[tuple(idx)]!r} want {want[tuple(idx)]!r}; "
            f"max err {np.nanmax(np.where(same_inf, 0, err)):.3g}")
