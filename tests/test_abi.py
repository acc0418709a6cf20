"""The C-ABI library loads on a machine without a GPU, exports every entry
point include/wsgpu.h declares, and rejects bad arguments on the host (no
kernel is launched by these tests)."""
import ctypes
import os
import re

import pytest
import torch  # noqa: F401  (loads the HIP runtime before libwsgpu)

from scope_amd import ops

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "wsgpu.h")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ws_\w+)\s*\(", text)))


def test_library_built():
    assert os.path.exists(ops.LIB_PATH), "run __graft_entry__.build() first"


def test_every_declared_symbol_is_exported():
    L = ctypes.CDLL(ops.LIB_PATH)
    names = declared()
    assert set(names) == set(ops.EXPORTS), (names, ops.EXPORTS)
    for n in names:
        assert hasattr(L, n), f"{n} not exported"


def test_version_and_plan():
    L = ops.lib()
    assert L.ws_version().decode().startswith("wsgpu")
    tps, ns = ops.decode_plan(0, 16, 32768, 256)
    assert (tps, ns) == (256, 128)
    tps, ns = ops.decode_plan(0, 16, 0, 0)
    assert ns == 1 and tps % 32 == 0
    tps, ns = ops.decode_plan(1, 8, 8192, 0)
    assert tps % 32 == 0 and ns == -(-8192 // tps)
    with pytest.raises(ops.WsError):
        ops.decode_plan(0, 16, 100, 48)  # not a multiple of 32
    assert L.ws_decode_workspace_bytes(10, 128, 3) == 3 * 10 * 129 * 4


def test_host_side_argument_checks():
    L = ops.lib()
    rc = L.ws_kv_append(None, None, None, None, None, None, 1, 1, 128, 1, 64, 1, 1, 1, None)
    assert rc == -1 and b"null" in L.ws_last_error()
    fake = ctypes.c_void_p(0x1000)  # never dereferenced: rejected before launch
    rc = L.ws_gqa_decode_partial(fake, fake, fake, fake, fake, 1, 24, 8, 128, 64, 4, 4,
                                 100, 0, 1.0, fake, fake, None, 0, None)
    assert rc == -1 and b"group size" in L.ws_last_error()
    rc = L.ws_gqa_decode_partial(fake, fake, fake, fake, fake, 1, 32, 8, 96, 64, 4, 4,
                                 100, 0, 1.0, fake, fake, None, 0, None)
    assert rc == -1 and b"head_dim" in L.ws_last_error()
    rc = L.ws_gqa_decode_partial(fake, fake, fake, fake, fake, 1, 32, 8, 128, 48, 4, 4,
                                 100, 0, 1.0, fake, fake, None, 0, None)
    assert rc == -1 and b"paging" in L.ws_last_error()
    # workspace too small for a multi-split call
    rc = L.ws_gqa_decode_partial(fake, fake, fake, fake, fake, 1, 32, 8, 128, 64, 64, 64,
                                 4096, 256, 1.0, fake, fake, None, 0, None)
    assert rc == -3 and b"workspace" in L.ws_last_error()
    rc = L.ws_mla_decode_partial(fake, fake, fake, fake, fake, 1, 8, 64, 4, 4, 100, 0, 1.0,
                                 fake, fake, None, 0, None)
    assert rc == -1 and b"H=8" in L.ws_last_error()
    rc = L.ws_lse_merge(fake, fake, fake, fake, None, 1, None, fake, None, 4, 128, None)
    assert rc == -1 and b"b_aux1" in L.ws_last_error()
    rc = L.ws_lse_merge(fake, fake, fake, fake, None, 9, None, fake, None, 4, 128, None)
    assert rc == -1 and b"format" in L.ws_last_error()
