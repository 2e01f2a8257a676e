"""CPU: the Spyre tensor's host-side logic -- allocation sizes, the geometry of
views, the restickify target rule -- against the reference's golden vectors.
No kernel runs here: the buffers of these tensors live in host memory and
only their geometry is examined."""

import json
import math
import os

import pytest
import torch

G = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "stl_golden.json")))


@pytest.fixture(scope="module")
def tsa():
    import torch_spyre_amd

    return torch_spyre_amd


def _empty(tsa, size, dtype=torch.float16, layout=None):
    stride = tsa.relayout._contiguous_strides(size)
    layout = layout or tsa.SpyreTensorLayout(list(size), dtype)
    return tsa.spyre_empty_with_layout(size, stride, dtype, layout, device="cpu")


def test_allocation_size_reference_case(tsa):
    """tests/test_spyre.py:384-393: a [2] fp16 tensor's device storage is one
    128-byte stick, unlike its 4 host bytes."""
    x = _empty(tsa, [2])
    assert x.untyped_storage().nbytes() == 128
    assert torch.tensor([1, 2], dtype=torch.float16).untyped_storage().nbytes() == 4


def _golden_layouts():
    for c in G["default_layout"]:
        if c["host_size"]:
            yield c["host_size"], c["device_size"], c["stride_map"]
    for c in G["dim_order"]:
        yield c["host_size"], c["device_size"], c["stride_map"]
    for c in G["explicit_roundtrip"]:
        yield c["sizes"], c["device_size"], c["stride_map"]


@pytest.mark.parametrize("host_size,device_size,stride_map", list(_golden_layouts()))
def test_allocation_rule_on_goldens(tsa, host_size, device_size, stride_map):
    """Storage = max(128 x prod(device_size[:-1]), host bytes)
    (torch_spyre/csrc/spyre_mem.cpp:468-473), for every golden layout: the
    device part from the native get_device_size_in_bytes, the host part
    from the element count."""
    from torch_spyre_amd import _lib

    lay = tsa.SpyreTensorLayout(device_size, stride_map, tsa.DataFormats.SEN169_FP16)
    x = _empty(tsa, host_size, layout=lay)
    dev = int(_lib.lib().spyre_device_size_in_bytes(_lib.i64_array(device_size), len(device_size)))
    assert dev == 128 * math.prod(device_size[:-1])
    assert x.untyped_storage().nbytes() == max(dev, 2 * math.prod(host_size))
    assert x.shape == tuple(host_size) and x.is_base()


def test_allocation_host_bytes_win(tsa):
    """A layout smaller than the host tensor (a sparse stick over [4, 64]
    holds one row) still gets the host bytes."""
    lay = tsa.SpyreTensorLayout([1, 64], [-1, 1], tsa.DataFormats.SEN169_FP16)
    x = _empty(tsa, [4, 64], layout=lay)
    assert lay.device_size_in_bytes() == 128
    assert x.untyped_storage().nbytes() == 4 * 64 * 2


def _swap_of_identity(order):
    r = len(order)
    diff = [i for i in range(r) if order[i] != i]
    return diff[0] if len(diff) == 2 and diff[1] == r - 1 else None


@pytest.mark.parametrize("case", [c for c in G["dim_order"] if _swap_of_identity(c["dim_order"]) is not None],
                         ids=lambda c: f"{c['host_size']}-{c['dim_order']}")
def test_restickify_target_matches_golden_dim_orders(tsa, case):
    """Moving the stick of the default layout to host dim d
    (pass_utils.py:749-781) gives the reference's golden layout for the
    dim order that swaps d with the last dim (tests/tensor/test_tensor_layout.py:39-104)."""
    size, strides = case["host_size"], case["host_strides"]
    d = _swap_of_identity(case["dim_order"])
    src = tsa.SpyreTensorLayout(size, torch.float16)
    got = tsa.restickify_target_layout(src, size, strides, d)
    assert (got.device_size, got.stride_map) == (case["device_size"], case["stride_map"])
    # and back again
    back = tsa.restickify_target_layout(got, size, strides, len(size) - 1)
    assert back == src


def test_restickify_target_same_dim_is_identity(tsa):
    src = tsa.SpyreTensorLayout([512, 256], torch.float16)
    assert tsa.restickify_target_layout(src, [512, 256], [256, 1], 1) == src


def test_view_geometry(tsa):
    """Views share the buffer and layout and change only the logical
    geometry (the cases of tests/test_spyre.py:589-662)."""
    t = _empty(tsa, [20])
    s = t[5:9].unsqueeze(0).expand(3, 4)
    assert s.shape == (3, 4) and s.stride() == (0, 1) and s.storage_offset() == 5
    assert tsa.device_buffer(s) is tsa.device_buffer(t) and s.untyped_storage().nbytes() == 128
    assert not s.is_base() and t.is_base()
    e = t[::2]
    assert e.shape == (10,) and e.stride() == (2,)
    m = _empty(tsa, [3, 4])
    assert m.t().stride() == (1, 4) and not m.t().is_contiguous()
    assert m.view(4, 3).stride() == (3, 1)
    assert m.device_tensor_layout() == tsa.SpyreTensorLayout([3, 4], torch.float16)
    assert tsa.device_tensor_layout(m[1]) == m.device_tensor_layout()
    assert m.detach().is_base()
    assert isinstance(m.unbind(0)[2], tsa.SpyreTensor) and m.unbind(0)[2].storage_offset() == 8


def test_other_ops_raise(tsa):
    m = _empty(tsa, [3, 4])
    with pytest.raises(NotImplementedError, match="not available on SpyreTensor"):
        m + 1
    with pytest.raises(NotImplementedError):
        m.view(torch.int16)


def test_repr_names_layout(tsa):
    r = repr(_empty(tsa, [3, 4]))
    assert "SpyreTensor(size=[3, 4]" in r and "SpyreTensorLayout(device_size=[1, 3, 64]" in r
