"""CPU: pin the oracle's layout + DMA restatement to the reference's golden
vectors and to what the layout definition fixes."""

import itertools
import json
import os

import numpy as np
import pytest

from oracle import layout as L
from oracle import relayout as R

G = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "stl_golden.json")))


@pytest.mark.parametrize("case", G["default_layout"], ids=lambda c: str(c["host_size"]))
def test_default_layout_golden(case):
    s = L.stl_default(case["host_size"])
    assert s.device_size == case["device_size"]
    assert s.stride_map == case["stride_map"]


@pytest.mark.parametrize("case", G["doc_default_layout"] + G["dim_order"] + G["sparse_dim_order"],
                         ids=lambda c: f"{c['host_size']}-{c['dim_order']}")
def test_dim_order_golden(case):
    strides = case.get("host_strides") or L.contiguous_strides(case["host_size"])
    s = L.stl_init(case["host_size"], strides, "float16", case["dim_order"])
    assert (s.device_size, s.stride_map) == (case["device_size"], case["stride_map"])


def test_str_golden():
    assert str(L.stl_default(G["str"]["host_size"])) == G["str"]["expected"]


def test_dma_known_answer():
    """tensors_and_layouts.md:305-318: ((4,1024,64),(65536,64,1),(64,256,1))."""
    ka = G["dma_known_answer"]
    lay = L.stl_default(ka["host_size"])
    infos = L.device_stride_infos(ka["host_size"], [256, 1], 0, lay.device_size, lay.stride_map, True, [256, 1])
    assert len(infos) == 1
    i = infos[0]
    assert list(reversed(i.size)) == ka["loop_ranges"]
    assert list(reversed(i.stride_dst)) == ka["device_strides"]
    assert list(reversed(i.stride_src)) == ka["host_strides"]


def _host_case(case, rng):
    sizes, strides = list(case["sizes"]), list(case["strides"])
    span = 1 + sum((s - 1) * st for s, st in zip(sizes, strides))
    store = rng.integers(0, 1 << 15, size=span).astype(np.int16)
    off = 0
    if case["kind"] == "sliced_batch":
        off = sizes[0] // 2
        sizes = [sizes[0] - off]
    return sizes, strides, store, off


@pytest.mark.parametrize("case", G["explicit_roundtrip"], ids=lambda c: f"{c['kind']}-{c['sizes']}-{c['device_size']}")
def test_explicit_roundtrip_golden(case):
    """Every explicit-layout case of tests/tensor/test_tensor_layout.py:193-405:
    x == D2H(H2D(x))."""
    rng = np.random.default_rng(7)
    sizes, strides, store, off = _host_case(case, rng)
    lay = L.Layout(case["device_size"], case["stride_map"])
    dev = L.h2d(store, sizes, strides, off, lay)
    back = L.d2h(dev, sizes, lay, strides)
    ref = np.lib.stride_tricks.as_strided(store[off:], shape=sizes, strides=[s * 2 for s in strides])
    assert np.array_equal(back, ref)


@pytest.mark.parametrize("case", [c for c in G["explicit_roundtrip"] if 0 not in c["stride_map"]],
                         ids=lambda c: f"{c['kind']}-{c['sizes']}-{c['device_size']}")
def test_stride_map_identity_brute_force(case):
    """tensors_and_layouts.md:210-217: for every written device position,
    host offset = dot(device coords, stride_map)."""
    sizes, strides = list(case["sizes"]), list(case["strides"])
    if case["kind"] == "sliced_batch":
        sizes = [sizes[0] - sizes[0] // 2]
    lay = L.Layout(case["device_size"], case["stride_map"])
    m = L.valid_device_coords(lay, sizes, strides)
    assert m, "layout writes nothing"
    for dev_off, host_off in m.items():
        assert L.stride_map_offset(lay, L.device_coords_of_offset(lay, dev_off)) == host_off


def test_h2d_is_injective_and_covers_host():
    """Every host element lands on exactly one device position (no element is
    dropped or duplicated) for padded, tiled and permuted layouts."""
    for case in G["explicit_roundtrip"]:
        if case["kind"] in ("expanding", "sliced_batch"):
            continue
        sizes, strides = case["sizes"], case["strides"]
        lay = L.Layout(case["device_size"], case["stride_map"])
        m = L.valid_device_coords(lay, sizes, strides)
        n = int(np.prod(sizes))
        assert sorted(m.values()) == sorted(
            int(np.dot(idx, strides)) for idx in itertools.product(*[range(s) for s in sizes])), case
        assert len(m) == n


def test_planted_mistake_is_caught():
    """A transposed stride in the oracle's plan breaks the documented known
    answer -- the pin is not vacuous."""
    lay = L.stl_default([1024, 256])
    info = L.device_stride_infos([1024, 256], [256, 1], 0, lay.device_size, lay.stride_map, True, [256, 1])[0]
    info.stride_src[1], info.stride_src[2] = info.stride_src[2], info.stride_src[1]
    assert list(reversed(info.stride_src)) != G["dma_known_answer"]["host_strides"]


@pytest.mark.parametrize("R_,C_", [(64, 64), (128, 192), (256, 64), (192, 320)])
def test_closed_forms_equal_dma_nests(R_, C_):
    """The three closed forms equal the generic loop-nest execution."""
    bits = R.random_finite_f16_bits((R_, C_), R_ + C_)
    st = [C_, 1]
    default = L.stl_default([R_, C_])
    assert np.array_equal(L.h2d(bits.reshape(-1), [R_, C_], st, 0, default), R.to_sticks(bits).reshape(-1))
    assert np.array_equal(R.from_sticks(R.to_sticks(bits)), bits)
    assert np.array_equal(L.d2h(R.to_sticks(bits).reshape(-1), [R_, C_], default), bits)
    tr = L.stl_init([R_, C_], st, "float16", [1, 0])
    assert np.array_equal(L.h2d(bits.reshape(-1), [R_, C_], st, 0, tr), R.transpose_restick(bits).reshape(-1))
    # transpose-restick equals the default sticks of X^T
    assert np.array_equal(R.transpose_restick(bits), R.to_sticks(np.ascontiguousarray(bits.T)))


def test_random_bits_are_finite():
    u = R.random_finite_f16_bits((1000,), 1)
    assert not ((u & 0x7C00) == 0x7C00).any()
    assert np.isfinite(u.view(np.float16)).all()
