"""GPU: Spyre tensors (SpyreTensor) -- round trips, D2H of views, device to
device copies, H2D into views, restickify -- mirroring the reference's
tests/test_spyre.py:384-662, plus bit-exact checks of the device bytes
against the oracle's DMA restatement.  Values are exact (raw copies)."""

import numpy as np
import pytest
import torch

from oracle import layout as OL
from oracle import relayout as OR
from tests.conftest import SEED

pytestmark = pytest.mark.gpu


def _bits(shape, seed, device):
    b = OR.random_finite_f16_bits(shape, seed)
    return b, torch.from_numpy(b.view(np.int16)).to(device).view(torch.float16)


def _raw(t):
    import torch_spyre_amd as tsa

    if isinstance(t, tsa.SpyreTensor):
        t = tsa.device_buffer(t)
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def test_round_trip(cuda):
    """tests/test_spyre.py:395-407."""
    import torch_spyre_amd as tsa

    x = torch.tensor([1, 2], dtype=torch.float16)
    d = tsa.to_device_layout(x)
    assert isinstance(d, tsa.SpyreTensor) and d.device.type == "cuda"
    assert d.untyped_storage().nbytes() == 128
    torch.testing.assert_close(d.cpu(), x)


def test_device_to_device(cuda):
    """tests/test_spyre.py:571-580: dst.copy_(src) between two device tensors."""
    import torch_spyre_amd as tsa

    src = tsa.to_device_layout(torch.randn(3, generator=torch.Generator().manual_seed(SEED)).half())
    dst = tsa.spyre_empty_with_layout([3], [1], torch.float16, tsa.SpyreTensorLayout([3], torch.float16))
    dst.copy_(src)
    assert torch.equal(src.cpu(), dst.cpu())
    assert src.data_ptr() != dst.data_ptr()


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_device_to_device_with_view(cuda, dtype):
    """tests/test_spyre.py:582-589: copy into a base tensor, read it back
    through a reshaping view."""
    import torch_spyre_amd as tsa

    a_host = torch.randn(512, 512, generator=torch.Generator().manual_seed(SEED + 1)).to(dtype)
    a = tsa.to_device_layout(a_host)
    b = tsa.to_device_layout(torch.zeros((512, 512), dtype=dtype))
    c = b.view((64, 8, 512))
    b.copy_(a)
    assert torch.equal(a.cpu(), b.cpu())
    assert torch.equal(a.cpu().view(64, 8, 512), c.cpu())
    assert torch.equal(c.cpu(), a_host.view(64, 8, 512))


def test_d2h_copy_of_expanded_view(cuda):
    """tests/test_spyre.py:591-626: stride-0 dims read the broadcast values;
    a slice's storage offset is applied on the host side."""
    import torch_spyre_amd as tsa

    src = tsa.to_device_layout(torch.tensor([1.0, 2.0, 3.0, 4.0], dtype=torch.float16))
    expected = torch.tensor([[1, 2, 3, 4]] * 3, dtype=torch.float16)
    expanded = src.unsqueeze(0).expand(3, 4)
    assert not expanded.is_contiguous() and expanded.stride() == (0, 1)
    assert torch.equal(expanded.cpu(), expected)
    assert torch.equal(src.broadcast_to(3, 4).cpu(), expected)
    col = tsa.to_device_layout(torch.tensor([10.0, 20.0], dtype=torch.float16))
    assert torch.equal(col.unsqueeze(1).expand(2, 5).cpu(),
                       torch.tensor([[10] * 5, [20] * 5], dtype=torch.float16))
    base = tsa.to_device_layout(torch.tensor([float(i) for i in range(20)], dtype=torch.float16))
    sliced_expanded = base[5:9].unsqueeze(0).expand(3, 4)
    assert sliced_expanded.storage_offset() == 5
    assert torch.equal(sliced_expanded.cpu(), torch.tensor([[5, 6, 7, 8]] * 3, dtype=torch.float16))


def test_d2h_copy_of_strided_slice(cuda):
    """tests/test_spyre.py:628-641."""
    import torch_spyre_amd as tsa

    t = tsa.to_device_layout(torch.tensor([float(i) for i in range(10)], dtype=torch.float16))
    sliced = t[::2]
    assert sliced.size() == (5,) and sliced.stride() == (2,)
    assert torch.equal(sliced.cpu(), torch.tensor([0.0, 2.0, 4.0, 6.0, 8.0], dtype=torch.float16))


def test_d2h_copy_of_transposed_view(cuda):
    """tests/test_spyre.py:643-662."""
    import torch_spyre_amd as tsa

    m = tsa.to_device_layout(torch.tensor([[1.0, 2.0, 3.0, 4.0], [5.0, 6.0, 7.0, 8.0], [9.0, 10.0, 11.0, 12.0]],
                                          dtype=torch.float16))
    mt = m.t()
    assert not mt.is_contiguous() and mt.stride() == (1, 4)
    assert torch.equal(mt.cpu(), torch.tensor([[1, 5, 9], [2, 6, 10], [3, 7, 11], [4, 8, 12]], dtype=torch.float16))
    # from_device_layout keeps the transposed (dense) strides
    h = tsa.from_device_layout(mt)
    assert h.is_cuda and h.stride() == (1, 4)


def test_views_of_a_large_tensor_vs_oracle(cuda):
    """Views of a [200, 300] fp16 tensor (two partial stick tiles) read back
    bit-exact against the oracle's D2H of the whole allocation plus the view."""
    import torch_spyre_amd as tsa

    bits, x = _bits((200, 300), SEED + 2, cuda)
    d = tsa.to_device_layout(x)
    lay = OL.stl_default([200, 300])
    host = OL.d2h(OL.h2d(bits.reshape(-1), [200, 300], [300, 1], 0, lay), [200, 300], lay)
    assert np.array_equal(_raw(d).reshape(-1), OL.h2d(bits.reshape(-1), [200, 300], [300, 1], 0, lay))
    for view, ref in ((d[3:150:7, 65:250], host[3:150:7, 65:250]), (d.t()[10:20], host.T[10:20]),
                      (d[17].unsqueeze(0).expand(4, 300), np.broadcast_to(host[17], (4, 300))),
                      (d.view(600, 100)[::3], host.reshape(600, 100)[::3])):
        assert np.array_equal(_raw(view.cpu()), np.ascontiguousarray(ref))


def test_h2d_into_views(cuda):
    """copy_ into a view writes only the view's elements; the rest of the
    allocation keeps its values."""
    import torch_spyre_amd as tsa

    bits, x = _bits((130, 70), SEED + 3, cuda)
    d = tsa.to_device_layout(x)
    nb, new = _bits((20, 10), SEED + 4, cuda)
    d[100:120, 5:15].copy_(new)
    want = bits.copy()
    want[100:120, 5:15] = nb
    assert np.array_equal(_raw(d.cpu()), want)
    # broadcast source and a transposed destination
    d.t()[3].copy_(torch.full((130,), 2.0, dtype=torch.float16))
    want[:, 3] = np.float16(2.0).view(np.uint16)
    assert np.array_equal(_raw(tsa.from_device_layout(d)), want)


def test_d2d_between_layouts_and_copy_tensor(cuda):
    """D2D copy_ from the default layout into a transpose-restick layout is
    the restickify (bit-exact device bytes); copy_tensor blocks unless
    non_blocking."""
    import torch_spyre_amd as tsa

    bits, x = _bits((256, 192), SEED + 5, cuda)
    a = tsa.to_device_layout(x)
    b = tsa.spyre_empty_with_layout([256, 192], [192, 1], torch.float16, tsa.transpose_restick_layout(256, 192))
    b.copy_(a)
    assert np.array_equal(_raw(b).reshape(-1), OR.transpose_restick(bits).reshape(-1))
    c = tsa.to_device_layout(torch.zeros((256, 192), dtype=torch.float16))
    tsa.copy_tensor(b, c)
    assert np.array_equal(_raw(c).reshape(-1), OR.to_sticks(bits).reshape(-1))
    h = torch.empty((256, 192), dtype=torch.float16, device=cuda)
    tsa.copy_tensor(c, h, non_blocking=True)
    torch.cuda.synchronize()
    assert np.array_equal(_raw(h), bits)
    # spyre::copy_from_d2d, the reference's D2D op
    e = tsa.to_device_layout(torch.zeros((256, 192), dtype=torch.float16), tsa.transpose_restick_layout(256, 192))
    torch.ops.spyre.copy_from_d2d(a, e)
    assert np.array_equal(_raw(e).reshape(-1), OR.transpose_restick(bits).reshape(-1))


def test_restickify_op_default_target(cuda):
    """torch.ops.spyre.restickify(x) with the reference's one-tensor schema:
    for x = a.t() the stick moves to a's dim 0, so the new allocation holds
    the sticks of a^T (transpose-restick, bit-exact) and the result reads as
    a.t()."""
    import torch_spyre_amd as tsa

    bits, x = _bits((256, 192), SEED + 6, cuda)
    a = tsa.to_device_layout(x)
    r = torch.ops.spyre.restickify(a.t())
    assert isinstance(r, tsa.SpyreTensor) and r.shape == (192, 256) and r.stride() == (1, 192)
    assert r.device_tensor_layout() == tsa.transpose_restick_layout(256, 192)
    assert np.array_equal(_raw(r).reshape(-1), OR.transpose_restick(bits).reshape(-1))
    assert np.array_equal(_raw(r.cpu()), bits.T)
    # a tensor whose stick is already innermost keeps its layout
    same = torch.ops.spyre.restickify(a)
    assert same.device_tensor_layout() == a.device_tensor_layout()
    assert np.array_equal(_raw(same), _raw(a))


def test_restickify_op_out_of_band_target(cuda):
    """A target recorded for the allocation (the reference's plan carries it
    in the compiler's layout) wins over the default, for every view."""
    import torch_spyre_amd as tsa

    size = [3, 100, 130]
    bits, x = _bits(tuple(size), SEED + 7, cuda)
    a = tsa.to_device_layout(x)
    target = tsa.SpyreTensorLayout(size, OL.contiguous_strides(size), torch.float16, [2, 0, 1])
    tsa.set_restickify_target(a, target)
    r = torch.ops.spyre.restickify(a[1:])
    want = OL.h2d(bits.reshape(-1), size, OL.contiguous_strides(size), 0,
                  OL.stl_init(size, OL.contiguous_strides(size), "float16", [2, 0, 1]))
    assert r.device_tensor_layout() == target
    assert np.array_equal(_raw(r).reshape(-1)[: want.size], want)
    assert np.array_equal(_raw(r.cpu()), bits[1:])
    tsa.set_restickify_target(a, None)


def test_to_device_layout_of_a_device_tensor(cuda):
    """Tensor.to(device_layout=) on a device tensor (torch_spyre/_monkey_patch.py:135-155):
    a D2D relayout, or the tensor itself when the layout matches."""
    import torch_spyre_amd as tsa

    bits, x = _bits((128, 256), SEED + 8, cuda)
    a = tsa.to_device_layout(x)
    assert tsa.to_device_layout(a, a.device_tensor_layout()) is a
    t = tsa.to_device_layout(a, tsa.transpose_restick_layout(128, 256))
    assert np.array_equal(_raw(t).reshape(-1), OR.transpose_restick(bits).reshape(-1))
    assert np.array_equal(_raw(t.clone().cpu()), bits)
    assert np.array_equal(_raw(a.t().clone().cpu()), bits.T)


def test_strided_host_source_round_trip(cuda):
    """A device tensor written from a transposed host view keeps that view's
    strides as its DMA geometry; restickify and D2H go through it."""
    import torch_spyre_amd as tsa

    bits, x = _bits((192, 256), SEED + 9, cuda)
    xt = x.t()  # [256, 192], strides (1, 256)
    d = tsa.to_device_layout(xt)
    assert d.stride() == (1, 256)
    assert np.array_equal(_raw(d.cpu()), bits.T)
    r = tsa.restickify(d, tsa.SpyreTensorLayout([256, 192], [1, 256], torch.float16, [1, 0]))
    assert np.array_equal(_raw(r.cpu()), bits.T)


# ------------------------------------------------- KV-cache writes (boxes) --

def _cache(cuda, seed):
    """A [1, 8, 2048, 128] fp16 KV cache in its default stick layout
    (tests/inductor/test_inductor_ops.py:5688-5739), and its host bits."""
    import torch_spyre_amd as tsa

    bits, x = _bits((1, 8, 2048, 128), seed, cuda)
    return bits, tsa.to_device_layout(x, tsa.SpyreTensorLayout([1, 8, 2048, 128], torch.float16))


def _device_want(host_bits):
    size = list(host_bits.shape)
    return OL.h2d(host_bits.reshape(-1), size, OL.contiguous_strides(size), 0, OL.stl_default(size))


def test_token_write_by_slice_select_and_index_copy(cuda):
    """Decode writes into a stick-layout cache: a token by slice copy_, one by
    select copy_, one by index_copy_ (the reference's decode pattern,
    tests/inductor/test_inductor_ops.py:5715-5739) and a 14-token prefill
    by index_copy_ (:5688-5713): the device bytes equal the oracle's layout of
    the cache with the tokens written, and every write moved only its own
    elements."""
    from torch_spyre_amd import device_tensor as DT

    bits, cache = _cache(cuda, SEED + 200)
    want = bits.copy()
    t1b, t1 = _bits((1, 8, 1, 128), SEED + 201, cuda)
    cache[:, :, 14:15, :].copy_(t1)
    want[:, :, 14:15, :] = t1b
    t2b, t2 = _bits((1, 8, 128), SEED + 202, cuda)
    cache[:, :, 15, :].copy_(t2)
    want[:, :, 15, :] = t2b
    t3b, t3 = _bits((1, 8, 1, 128), SEED + 203, cuda)
    res = cache.index_copy_(2, torch.tensor([16], dtype=torch.int64), t3)
    assert res is cache
    want[:, :, 16:17, :] = t3b
    pb, p = _bits((1, 8, 14, 128), SEED + 204, cuda)
    cache.index_copy_(2, torch.arange(100, 114, dtype=torch.int64, device=cuda), p)
    want[:, :, 100:114, :] = pb
    assert np.array_equal(_raw(cache).reshape(-1), _device_want(want))
    # the writes' loop nests move exactly the token's elements
    v = cache[:, :, 14:15, :]
    infos = DT._box_infos(v, t1, host2device=True)
    assert sum(int(np.prod(i.size[:i.rank])) for i in infos) == t1.numel()
    # reading a token back moves only its elements too, and equals the oracle
    assert np.array_equal(_raw(cache[:, :, 100:114, :].cpu()), pb)


def test_index_copy_out_of_place_and_errors(cuda):
    """index_copy (out of place) leaves self unchanged; indices out of range
    and shape mismatches raise."""
    bits, cache = _cache(cuda, SEED + 210)
    tb, t = _bits((1, 8, 2, 128), SEED + 211, cuda)
    out = torch.index_copy(cache, 2, torch.tensor([5, 2047]), t)
    want = bits.copy()
    want[:, :, 5], want[:, :, 2047] = tb[:, :, 0], tb[:, :, 1]
    assert np.array_equal(_raw(out).reshape(-1), _device_want(want))
    assert np.array_equal(_raw(cache).reshape(-1), _device_want(bits))
    with pytest.raises(IndexError):
        cache.index_copy_(2, torch.tensor([2048]), t[:, :, :1])
    with pytest.raises(IndexError):
        cache.index_copy_(2, torch.tensor([1, 2, 3]), t)


def test_box_writes_across_sticks(cuda):
    """Writes into boxes that start and end inside sticks, of the default and
    the transposed ([1, 0]) layouts, and through a transposed view: bit-exact
    against the oracle."""
    import torch_spyre_amd as tsa

    size = [130, 200]
    for k, order in enumerate(([0, 1], [1, 0])):
        bits, x = _bits(tuple(size), SEED + 220 + k, cuda)
        stl = tsa.SpyreTensorLayout(size, [200, 1], torch.float16, order)
        d = tsa.to_device_layout(x, stl)
        want = bits.copy()
        ab, a = _bits((97, 145), SEED + 230 + k, cuda)
        d[3:100, 5:150].copy_(a)
        want[3:100, 5:150] = ab
        bb, b = _bits((100, 40), SEED + 240 + k, cuda)
        d.t()[20:120, 10:50].copy_(b)
        want.T[20:120, 10:50] = bb
        ol = OL.Layout(list(stl.device_size), list(stl.stride_map), "float16")
        assert np.array_equal(_raw(d).reshape(-1), OL.h2d(want.reshape(-1), size, [200, 1], 0, ol))
        assert np.array_equal(_raw(d[7:90, 33:180].cpu()), want[7:90, 33:180])


# --------------------------------------------------- views carrying layouts --

def test_views_with_layout(cuda):
    """as_strided_with_layout / reinterpret_tensor[_with_layout]
    (torch_spyre/csrc/spyre_views.cpp:123-181): with the tensor's own layout
    a view keeps the DMA geometry (reads equal the host view); with another
    layout the allocation's bytes are read through the new layout and the
    view's own geometry (bit-exact against the oracle's D2H of the raw
    bytes)."""
    import torch_spyre_amd as tsa

    bits, x = _bits((256, 192), SEED + 250, cuda)
    d = tsa.to_device_layout(x, tsa.SpyreTensorLayout([256, 192], torch.float16))
    v = tsa.as_strided_with_layout(d, [64, 192], [192, 1], 192 * 10, d.device_tensor_layout())
    assert np.array_equal(_raw(v.cpu()), bits[10:74])
    r = tsa.reinterpret_tensor(d, [32, 192], [192, 1], 192 * 100)
    assert np.array_equal(_raw(r.cpu()), bits[100:132])
    raw = _raw(d).reshape(-1)
    # the 96 KiB allocation as [128, 384] in its default layout
    stl2 = tsa.SpyreTensorLayout([128, 384], torch.float16)
    w = tsa.reinterpret_tensor_with_layout(d, [128, 384], [384, 1], 0, stl2)
    assert w.device_tensor_layout() == stl2 and w.data_ptr() == d.data_ptr()
    assert np.array_equal(_raw(w.cpu()), OL.d2h(raw, [128, 384], OL.stl_default([128, 384])))
    a = tsa.as_strided_with_layout(d, [128, 384], [384, 1], 0, stl2)
    assert np.array_equal(_raw(a.cpu()), OL.d2h(raw, [128, 384], OL.stl_default([128, 384])))
    with pytest.raises(ValueError):  # more than the allocation holds
        tsa.reinterpret_tensor_with_layout(d, [512, 192], [192, 1], 0, tsa.SpyreTensorLayout([512, 192],
                                                                                            torch.float16))


def test_tensor_to_device_layout_and_empty(cuda):
    """The reference's method forms (torch_spyre/_monkey_patch.py:63-196):
    x.to(device_layout=) from CPU and GPU host order and between layouts,
    torch.empty(..., device_layout=), Tensor.device_tensor_layout()."""
    import torch_spyre_amd as tsa

    bits, x = _bits((256, 192), SEED + 260, cuda)
    stl = tsa.SpyreTensorLayout([256, 192], torch.float16)
    tr = tsa.SpyreTensorLayout([256, 192], [192, 1], torch.float16, [1, 0])
    d = x.cpu().to(device_layout=stl)
    assert isinstance(d, tsa.SpyreTensor) and d.device_tensor_layout() == stl
    assert np.array_equal(_raw(d).reshape(-1), OR.to_sticks(bits).reshape(-1))
    d2 = x.to(device_layout=stl)
    assert np.array_equal(_raw(d2).reshape(-1), OR.to_sticks(bits).reshape(-1))
    assert d2.to(device_layout=stl) is d2 and d2.to(device_layout=stl, copy=True) is not d2
    t = d2.to(device_layout=tr)
    assert t.device_tensor_layout() == tr and np.array_equal(_raw(t).reshape(-1), OR.transpose_restick(bits).reshape(-1))
    assert np.array_equal(_raw(t.cpu()), bits)
    assert x.device_tensor_layout() is None
    e = torch.empty(256, 192, dtype=torch.float16, device_layout=stl)
    assert isinstance(e, tsa.SpyreTensor) and e.device_tensor_layout() == stl and list(e.shape) == [256, 192]
    e.copy_(x)
    assert np.array_equal(_raw(e).reshape(-1), OR.to_sticks(bits).reshape(-1))
    assert torch.empty(3, 4).device_tensor_layout() is None  # torch's own otherwise
    f = x.to(torch.float32, device_layout=tsa.SpyreTensorLayout([256, 192], torch.float32))
    assert f.dtype == torch.float32 and torch.equal(f.cpu(), x.float().cpu())
