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
    pad = lambda n: -(-n // 256) * 256
    # explicit split counts are kept; workspace = lse slots + bf16 piece slots
    n, wsb = ops.decode_plan(0, 16, 8, 32768, 100)
    assert n == 100 and wsb == pad((100 + 16) * 8 * 4) + (100 + 16) * 8 * 128 * 2
    n, wsb = ops.decode_plan(1, 8, 16, 16384, 64)
    assert n == 64 and wsb == pad((64 + 8) * 16 * 4) + (64 + 8) * 16 * 512 * 2
    # the library's choice never exceeds the blocks available (2 per GQA
    # split, i.e. per wave) nor the merge's 4096 splits
    for rows, G, L in ((128, 4, 15773), (16, 8, 131072), (4, 8, 4096), (1, 1, 1), (2, 16, 1 << 20)):
        n, _ = ops.decode_plan(0, rows, G, L, 0)
        assert 1 <= n <= max(1, -(-rows * -(-L // 32) // 2)) and n <= 4096
    n, _ = ops.decode_plan(1, 8, 16, 8192, 0)
    assert 1 <= n <= 8 * 256 // 4
    with pytest.raises(ops.WsError):
        ops.decode_plan(0, 16, 0, 100, 0)  # no heads
    with pytest.raises(ops.WsError):
        ops.decode_plan(0, 16, 8, 100, -1)


def test_width_plan():
    """The plan at other head widths: the piece slots scale with the value
    width, 128/128 matches kind 0, and widths without a kernel are refused."""
    pad = lambda n: -(-n // 256) * 256
    for Dk, Dv in ((64, 64), (128, 128), (256, 256), (192, 128), (16, 16), (80, 80),
                   (192, 192), (240, 240)):
        n, wsb = ops.gqa_plan(16, 8 if Dk != 192 else 1, Dk, Dv, 32768, 100)
        G = 8 if Dk != 192 else 1
        assert n == 100 and wsb == pad((100 + 16) * G * 4) + (100 + 16) * G * Dv * 2
    n_w, wsb_w = ops.gqa_plan(16, 8, 128, 128, 32768, 100)
    assert (n_w, wsb_w) == ops.decode_plan(0, 16, 8, 32768, 100)
    for Dk, Dv in ((40, 40), (8, 8), (272, 272), (128, 64), (256, 128)):
        with pytest.raises(ops.WsError, match="unsupported"):
            ops.gqa_plan(16, 1, Dk, Dv, 100, 10)
    # the 192/128 kernel exists for group size 1 only, as the launch checks
    with pytest.raises(ops.WsError, match="group size 1"):
        ops.gqa_plan(16, 8, 192, 128, 100, 10)


def test_host_side_argument_checks():
    L = ops.lib()
    rc = L.ws_kv_append(None, None, None, None, None, None, 1, 1, 128, 1, 64, 1, 1, 1, None)
    assert rc == -1 and b"null" in L.ws_last_error()
    fake = ctypes.c_void_p(0x1000)  # never dereferenced: rejected before launch
    rc = L.ws_gqa_decode_partial(fake, fake, fake, fake, fake, 1, 136, 8, 128, 64, 4, 4,
                                 100, 0, 1.0, fake, fake, None, 0, None)
    assert rc == -1 and b"group size" in L.ws_last_error()
    rc = L.ws_gqa_decode_partial(fake, fake, fake, fake, fake, 1, 32, 8, 40, 64, 4, 4,
                                 100, 0, 1.0, fake, fake, None, 0, None)
    assert rc == -1 and b"head_dim" in L.ws_last_error()
    rc = L.ws_gqa_decode_partial(fake, fake, fake, fake, fake, 1, 32, 8, 128, 48, 4, 4,
                                 100, 0, 1.0, fake, fake, None, 0, None)
    assert rc == -1 and b"paging" in L.ws_last_error()
    # workspace too small
    rc = L.ws_gqa_decode_partial(fake, fake, fake, fake, fake, 1, 32, 8, 128, 64, 64, 64,
                                 4096, 16, 1.0, fake, fake, None, 0, None)
    assert rc == -3 and b"workspace" in L.ws_last_error()
    rc = L.ws_mla_decode_partial(fake, fake, fake, fake, fake, 1, 8, 64, 4, 4, 100, 0, 1.0,
                                 fake, fake, None, 0, None)
    assert rc == -1 and b"H=8" in L.ws_last_error()
    # fused append: len_out must not alias len_in; k_new required
    rc = L.ws_gqa_append_decode_partial(fake, fake, fake, fake, fake, fake, fake, fake, 1, 32,
                                        8, 128, 64, 4, 4, 100, 0, 1.0, fake, fake, None, 0,
                                        None)
    assert rc == -1 and b"alias" in L.ws_last_error()
    rc = L.ws_gqa_append_decode_partial(fake, None, fake, fake, fake, fake, fake, None, 1, 32,
                                        8, 128, 64, 4, 4, 100, 0, 1.0, fake, fake, None, 0,
                                        None)
    assert rc == -1 and b"k_new" in L.ws_last_error()
    rc = L.ws_mla_append_decode_partial(fake, fake, fake, 100, fake, 576, fake, fake, fake,
                                        None, 1, 16, 64, 4, 4, 100, 0, 1.0, fake, fake, None,
                                        0, None)
    assert rc == -1 and b"new-latent" in L.ws_last_error()
    # misaligned workspace
    rc = L.ws_gqa_decode_partial(fake, fake, fake, fake, fake, 1, 32, 8, 128, 64, 64, 64,
                                 4096, 16, 1.0, fake, fake, ctypes.c_void_p(0x1010),
                                 1 << 30, None)
    assert rc == -1 and b"256-byte" in L.ws_last_error()
    rc = L.ws_lse_merge(fake, fake, fake, fake, None, 1, None, fake, None, 4, 128, None)
    assert rc == -1 and b"b_aux1" in L.ws_last_error()
    rc = L.ws_lse_merge(fake, fake, fake, fake, None, 9, None, fake, None, 4, 128, None)
    assert rc == -1 and b"format" in L.ws_last_error()
    # ws_copy: alignment, size and overlap are checked before any launch
    rc = L.ws_copy(fake, ctypes.c_void_p(0x2008), 64, None)
    assert rc == -1 and b"aligned" in L.ws_last_error()
    rc = L.ws_copy(fake, ctypes.c_void_p(0x2000), 66, None)
    assert rc == -1 and b"multiple of 4" in L.ws_last_error()
    rc = L.ws_copy(fake, ctypes.c_void_p(0x1010), 64, None)
    assert rc == -1 and b"overlap" in L.ws_last_error()
    assert L.ws_copy(None, None, 0, None) == 0  # nothing to copy
    rc = L.ws_copy(None, fake, 16, None)
    assert rc == -1 and b"null" in L.ws_last_error()
    with pytest.raises(ValueError, match="one side must be on a GPU"):
        ops.copy_(torch.zeros(4), torch.zeros(4))
    # ws_copy_pages: sizes and alignment are checked before any launch
    rc = L.ws_copy_pages(fake, 0, fake, 4, fake, 0, fake, 4, 1, 1, 72, 0, None)
    assert rc == -1 and b"bad sizes" in L.ws_last_error()
    rc = L.ws_copy_pages(fake, 8, fake, 4, fake, 0, fake, 4, 1, 1, 64, 0, None)
    assert rc == -1 and b"aligned" in L.ws_last_error()
    rc = L.ws_copy_pages(None, 0, fake, 4, fake, 0, fake, 4, 1, 1, 64, 0, None)
    assert rc == -1 and b"null" in L.ws_last_error()
    assert L.ws_copy_pages(None, 0, None, 0, None, 0, None, 0, 0, 1, 64, 0, None) == 0
    rc = L.ws_copy_pages(fake, 0, fake, 4, fake, 0, fake, 4, 1, 1, 64, -1, None)
    assert rc == -1 and b"max_workgroups" in L.ws_last_error()
