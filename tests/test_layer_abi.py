"""The two-sided layer driver's C ABI (include/wslayer.h, libwslayer.so) on
the CPU: every declared entry point is exported, the ctypes structures have
the C layout, and arguments are refused before anything is launched."""
import ctypes
import os
import re

import torch  # noqa: F401  (loads the HIP runtime before the libraries)

from scope_amd import layer

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "wslayer.h")


def test_every_declared_entry_point_is_exported():
    names = sorted(set(re.findall(r"\b(wl_\w+)\s*\(", open(HEADER).read())))
    assert set(names) == set(layer.EXPORTS), names
    L = layer.lib()
    for n in names:
        assert hasattr(L, n), n


def test_structures_match_the_library():
    L = layer.lib()
    assert L.wl_struct_size(0) == ctypes.sizeof(layer.WlMlaLayer)
    assert L.wl_struct_size(1) == ctypes.sizeof(layer.WlGqaLayer)
    # the output fields sit where the header puts them: last in the struct
    assert layer.WlMlaLayer.stage.offset > layer.WlMlaLayer.host_seconds.offset
    assert layer.WlGqaLayer.stage.offset > layer.WlGqaLayer.host_seconds.offset


def test_bad_arguments_are_refused_before_any_launch():
    L = layer.lib()
    a = layer.WlMlaLayer()
    a.B, a.H = 0, 16
    assert L.wl_mla_layer(ctypes.byref(a), None) == -1
    assert b"bad batch" in L.wl_last_error() and a.stage == 0
    lens = (ctypes.c_int32 * 2)(0, 0)
    a.B, a.host_lens = 2, ctypes.cast(lens, ctypes.c_void_p)
    assert L.wl_mla_layer(ctypes.byref(a), None) == -1  # neither out nor w_uv
    assert b"no output" in L.wl_last_error() and a.stage == 0
    lens[1] = 64  # host tokens but no pinned host buffers
    a.out = 0x1000
    assert L.wl_mla_layer(ctypes.byref(a), None) == -1
    assert b"host buffers" in L.wl_last_error() and a.stage == 0
    g = layer.WlGqaLayer()
    g.B, g.Hq, g.Hkv = 1, 30, 8
    assert L.wl_gqa_layer(ctypes.byref(g), None) == -1
    assert b"bad shape" in L.wl_last_error() and g.stage == 0
