"""Transfers of the two-sided decode step on the GPU: ws_copy between HBM and
pinned host memory (bit-exact, any multiple of 4 bytes), and the merges
reading their host operand from pinned host memory in place, call after call
with new host data (no stale copy of the operand is ever read)."""
import pytest
import torch

from scope_amd import ops

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _say(msg):
    print(msg, flush=True)


@pytest.mark.parametrize("nbytes", [4, 16, 20, 1152 * 512, 1 << 22, (1 << 22) + 12])
def test_copy_both_directions_bit_exact(nbytes):
    _say(f"ws_copy {nbytes} bytes")
    n = nbytes // 4
    src = torch.randint(-2**31, 2**31 - 1, (n,), dtype=torch.int32, device=DEV)
    host = torch.zeros(n, dtype=torch.int32, pin_memory=True)
    back = torch.zeros(n, dtype=torch.int32, device=DEV)
    dev2 = torch.zeros(n, dtype=torch.int32, device=DEV)
    for rep in range(3):  # the same buffers, new contents each time
        src.random_(-2**31, 2**31 - 1)
        ops.copy_(host, src)
        ops.copy_(back, host)
        ops.copy_(dev2, src)
        torch.cuda.synchronize()
        assert torch.equal(host, src.cpu()), rep
        assert torch.equal(back, src), rep
        assert torch.equal(dev2, src), rep


def test_copy_rejects_bad_arguments():
    a = torch.zeros(64, dtype=torch.float32, device=DEV)
    with pytest.raises(ValueError, match="pinned"):
        ops.copy_(torch.zeros(64, dtype=torch.float32), a)  # pageable host memory
    with pytest.raises(ValueError, match="same dtype"):
        ops.copy_(torch.zeros(64, dtype=torch.int32, device=DEV), a)
    with pytest.raises(ops.WsError, match="overlap"):
        ops.copy_(a[4:36], a[0:32])


@pytest.mark.parametrize("fmt", [ops.PARTIAL_LSE_F32, ops.TRIPLE_NORM_BF16,
                                 ops.PARTIAL_LSE_BF16])
def test_merges_read_pinned_host_operands_in_place(fmt):
    _say(f"lse_merge with a pinned host operand fmt={fmt}")
    rows, Dv = 300, 128
    g = torch.Generator().manual_seed(5)
    out_g = torch.randn((rows, Dv), generator=g).to(DEV)
    lse_g = (torch.randn(rows, generator=g) + 3).to(DEV)
    dt = torch.float32 if fmt == ops.PARTIAL_LSE_F32 else torch.bfloat16
    hb = [torch.empty((rows, Dv), dtype=dt, pin_memory=True),
          torch.empty(rows, dtype=torch.float32 if fmt == ops.PARTIAL_LSE_BF16 else dt,
                      pin_memory=True)]
    if fmt == ops.TRIPLE_NORM_BF16:
        hb.append(torch.empty(rows, dtype=dt, pin_memory=True))
    for rep in range(4):  # the host rewrites the same pinned buffers each call
        hb[0].copy_(torch.randn((rows, Dv), generator=g))
        hb[1].copy_(torch.randn(rows, generator=g) + rep)
        if len(hb) == 3:
            hb[2].copy_(torch.rand(rows, generator=g) * 20 + 1)
        got, gl = ops.lse_merge(out_g, lse_g, tuple(hb), fmt, out_dtype=torch.float32)
        want, wl = ops.lse_merge(out_g, lse_g, tuple(x.to(DEV) for x in hb), fmt,
                                 out_dtype=torch.float32)
        torch.cuda.synchronize()
        assert torch.equal(got, want) and torch.equal(gl, wl), rep


@pytest.mark.parametrize("page_shape,wg", [((64, 576), 0), ((8, 64, 128), 0), ((3, 16), 0),
                                           ((64, 576), 5), ((8, 64, 128), 1)])
def test_copy_pages_both_directions_every_layer(page_shape, wg):
    # wg: a bounded grid that strides over the (layer, page, chunk) units
    _say(f"ws_copy_pages page {page_shape} max_workgroups {wg}")
    layers, n_host, n_gpu = 3, 40, 33
    g = torch.Generator().manual_seed(11)
    host = torch.randn((layers, n_host, *page_shape), generator=g).to(torch.bfloat16)
    host = host.pin_memory()
    gpu = torch.randn((layers, n_gpu, *page_shape), generator=g).to(torch.bfloat16).to(DEV)
    rng = torch.Generator().manual_seed(12)
    src = torch.randperm(n_host, generator=rng)[:17].tolist()
    dst = torch.randperm(n_gpu, generator=rng)[:17].tolist()
    want = gpu.clone()
    want[:, dst] = host[:, src].to(DEV)
    ops.copy_pages(gpu, dst, host, src, wg)  # host -> HBM
    torch.cuda.synchronize()
    assert torch.equal(gpu, want)
    back_src = torch.randperm(n_gpu, generator=rng)[:9].tolist()
    back_dst = torch.randperm(n_host, generator=rng)[:9].tolist()
    want_h = host.clone()
    want_h[:, back_dst] = gpu[:, back_src].cpu()
    ops.copy_pages(host, back_dst, gpu, back_src, wg)  # HBM -> host
    torch.cuda.synchronize()
    assert torch.equal(host, want_h)


def test_copy_pages_rejects_ids_outside_the_pools():
    host = torch.zeros((1, 4, 64, 576), dtype=torch.bfloat16).pin_memory()
    gpu = torch.zeros((1, 3, 64, 576), dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError, match="dst_ids"):
        ops.copy_pages(gpu, [3], host, [0])
    with pytest.raises(ValueError, match="src_ids"):
        ops.copy_pages(gpu, [0], host, [-1])
    with pytest.raises(ValueError, match="pinned"):
        ops.copy_pages(gpu, [0], torch.zeros((1, 4, 64, 576), dtype=torch.bfloat16), [0])
