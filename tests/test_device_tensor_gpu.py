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
