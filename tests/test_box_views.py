"""CPU: loop nests of views that are boxes of a Spyre tensor's allocation
(device_tensor._box_infos, used by view writes, view reads and index_copy_)
against the oracle.

The nests are executed by the oracle's model of the DMA engine
(oracle.layout.execute_infos) on a device buffer the oracle built; the
result must equal the oracle's relayout of the host tensor with the view
written (or, for reads, the host tensor's view).  The planner must also move
exactly the view's elements (bytes in proportion to the write).  No GPU is
used: the tensors' buffers live in host memory."""

import numpy as np
import pytest
import torch

from oracle import layout as OL
from oracle import relayout as OR


@pytest.fixture(scope="module")
def tsa():
    import torch_spyre_amd

    return torch_spyre_amd


def _olayout(stl):
    return OL.Layout(list(stl.device_size), list(stl.stride_map), "float16")


def _spyre(tsa, bits, stl):
    """A SpyreTensor whose host-memory buffer is the oracle's H2D of bits."""
    size = list(bits.shape)
    stride = OL.contiguous_strides(size)
    dev = OL.h2d(bits.reshape(-1), size, stride, 0, _olayout(stl))
    data = torch.from_numpy(dev.view(np.int16).copy()).view(torch.float16)
    return tsa.SpyreTensor(data, stl, size, stride), dev


def _oracle_infos(infos):
    return [OL.StrideInfo(*[list(v) if isinstance(v, tuple) else v for v in i.as_tuple()]) for i in infos]


def _write(tsa, x, dev, view_fn, seed):
    """Writes random bits through view_fn(x) with the planner's nests (run by
    the oracle's DMA model); returns (new device bits, host bits written,
    elements moved)."""
    from torch_spyre_amd import device_tensor as DT

    v = view_fn(x)
    src_bits = OR.random_finite_f16_bits(tuple(v.shape), seed)
    src = torch.from_numpy(src_bits.view(np.int16).copy()).view(torch.float16)
    infos = DT._box_infos(v, src, host2device=True)
    assert infos is not None
    out = dev.copy()
    OL.execute_infos(src_bits.reshape(-1), out, _oracle_infos(infos))
    moved = sum(int(np.prod(i.size[:i.rank])) for i in infos)
    return out, src_bits, moved


CASES = [
    # host size, layout kind, view (as a function of a tensor or array), name
    ([130, 200], "default", lambda t: t[3:100, 5:150], "crosses sticks at both ends"),
    ([130, 200], "default", lambda t: t[7:9, 64:128], "one whole stick per row"),
    ([130, 200], "default", lambda t: t[0:130, 190:200], "the padded last stick"),
    ([130, 200], "default", lambda t: t[5, 10:190], "a select and a slice"),
    ([130, 200], "transpose", lambda t: t[3:100, 5:150], "the stick on dim 0"),
    ([1, 8, 2048, 128], "default", lambda t: t[:, :, 14:15, :], "a token of a KV cache"),
    ([1, 8, 2048, 128], "default", lambda t: t[:, :, 100:114, :], "a 14-token prefill"),
    ([1, 8, 2048, 128], "default", lambda t: t[:, 2:5, 7, 30:100], "select + slices"),
]


def _layout(tsa, size, kind):
    if kind == "default":
        return tsa.SpyreTensorLayout(list(size), torch.float16)
    st = OL.contiguous_strides(list(size))
    return tsa.SpyreTensorLayout(list(size), st, torch.float16, [1, 0])


@pytest.mark.parametrize("size,kind,view,name", CASES, ids=[c[3] for c in CASES])
def test_box_write_equals_oracle(tsa, size, kind, view, name):
    stl = _layout(tsa, size, kind)
    bits = OR.random_finite_f16_bits(tuple(size), 7)
    x, dev = _spyre(tsa, bits, stl)
    got, src_bits, moved = _write(tsa, x, dev, view, 11)
    want_host = bits.copy()
    view(want_host)[...] = src_bits
    want = OL.h2d(want_host.reshape(-1), size, OL.contiguous_strides(size), 0, _olayout(stl))
    assert np.array_equal(got, want)
    assert moved == src_bits.size  # only the view's elements


@pytest.mark.parametrize("size,kind,view,name", CASES, ids=[c[3] for c in CASES])
def test_box_read_equals_oracle(tsa, size, kind, view, name):
    from torch_spyre_amd import device_tensor as DT

    stl = _layout(tsa, size, kind)
    bits = OR.random_finite_f16_bits(tuple(size), 8)
    x, dev = _spyre(tsa, bits, stl)
    v = view(x)
    out = torch.empty(v.shape, dtype=torch.float16)
    infos = DT._box_infos(v, out, host2device=False)
    assert infos is not None
    got = np.zeros(out.numel(), dtype=np.uint16)
    OL.execute_infos(dev, got, _oracle_infos(infos))
    assert np.array_equal(got.reshape(v.shape), view(bits))


def test_transposed_view_write(tsa):
    """A permuted view: view dim 0 steps host dim 1 (the stick dim)."""
    size = [130, 200]
    stl = _layout(tsa, size, "default")
    bits = OR.random_finite_f16_bits(tuple(size), 9)
    x, dev = _spyre(tsa, bits, stl)
    got, src_bits, moved = _write(tsa, x, dev, lambda t: t.t()[20:120, 10:50], 12)
    want_host = bits.copy()
    want_host.T[20:120, 10:50] = src_bits
    want = OL.h2d(want_host.reshape(-1), size, OL.contiguous_strides(size), 0, _olayout(stl))
    assert np.array_equal(got, want) and moved == src_bits.size


def test_non_box_views_are_not_planned(tsa):
    """Step-2 slices and broadcast writes are no boxes: the caller takes the
    round trip."""
    from torch_spyre_amd import device_tensor as DT

    size = [130, 200]
    x, _ = _spyre(tsa, OR.random_finite_f16_bits(tuple(size), 10), _layout(tsa, size, "default"))
    v = x[::2, 5:20]
    assert DT._box_infos(v, torch.empty(v.shape, dtype=torch.float16), True) is None
    e = x[3:4, :].expand(5, 200)
    assert DT._box_infos(e, torch.empty(e.shape, dtype=torch.float16), True) is None
    # a broadcast read is planned (device stride 0)
    out = torch.empty(e.shape, dtype=torch.float16)
    assert DT._box_infos(e, out, False) is not None
