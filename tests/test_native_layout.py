"""CPU: the native descriptor and DMA planner (libspyre_hip.so host code,
called through the C ABI) against the golden vectors and the oracle.  No GPU
kernel is launched here."""

import copy
import itertools
import json
import os
import pickle
import re

import numpy as np
import pytest
import torch

from oracle import layout as OL

G = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "stl_golden.json")))
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def tsa():
    import torch_spyre_amd

    return torch_spyre_amd


def test_library_exports_every_declared_symbol(tsa):
    """Every function include/spyre_hip.h declares is exported and bound."""
    hdr = open(os.path.join(ROOT, "include", "spyre_hip.h")).read()
    declared = set(re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\*?\s+\*?(spyre_[a-z_0-9]+)\(", hdr, re.M))
    assert len(declared) >= 12
    from torch_spyre_amd import _lib

    L = _lib.lib()
    for name in declared:
        assert hasattr(L, name), name
        assert name in _lib.SIGNATURES, name
    assert L.spyre_abi_version() == _lib.ABI_VERSION


def test_default_layout_golden(tsa):
    for c in G["default_layout"]:
        s = tsa.SpyreTensorLayout(c["host_size"], torch.float16)
        assert (s.device_size, s.stride_map) == (c["device_size"], c["stride_map"]), c


def test_dim_order_golden(tsa):
    for c in G["doc_default_layout"] + G["dim_order"] + G["sparse_dim_order"]:
        strides = c.get("host_strides") or OL.contiguous_strides(c["host_size"])
        s = tsa.SpyreTensorLayout(c["host_size"], strides, torch.float16, c["dim_order"])
        assert (s.device_size, s.stride_map) == (c["device_size"], c["stride_map"]), c


def test_str_eq_hash_pickle(tsa):
    """tests/tensor/test_tensor_layout.py:106-150."""
    s = tsa.SpyreTensorLayout([512, 256], torch.float16)
    assert str(s) == G["str"]["expected"]
    x = tsa.SpyreTensorLayout([512, 256], torch.float16)
    y = tsa.SpyreTensorLayout([512, 256], [256, 1], torch.float16, [0, 1])
    z = tsa.SpyreTensorLayout([512, 256], [256, 1], torch.float16, [1, 0])
    z2 = tsa.SpyreTensorLayout([512, 256], torch.float32)
    assert x == y and hash(x) == hash(y)
    assert y != z and hash(y) != hash(z)
    assert x != z2 and hash(x) != hash(z2)
    assert {x: "value"}[y] == "value"
    assert len({x, y, z}) == 2
    assert pickle.loads(pickle.dumps(z)) == z
    assert copy.deepcopy(z) == z
    # explicit constructor equals the default one (test_tensor_layout.py:93-99)
    e = tsa.SpyreTensorLayout([4, 512, 64], [64, 256, 1], tsa.get_device_dtype(torch.float16))
    assert e == x
    # older pickle versions load
    st = z.__getstate__()
    v2 = tsa.layout._from_state((2, st[1], st[2], st[3]))
    v1 = tsa.layout._from_state((1, st[1], [0, 0, 0], st[2], st[3]))
    assert v2 == z and v1 == z
    with pytest.raises(ValueError):
        tsa.layout._from_state((9, [], [], 1, 0))
    assert z.elems_per_stick() == 64 and z2.elems_per_stick() == 32
    assert s.device_size_in_bytes() == 4 * 512 * 128


def _plans_equal(native, oracle):
    a = [i.as_tuple() for i in native]
    b = [(tuple(i.size), tuple(i.stride_src), tuple(i.stride_dst), i.offset_src, i.offset_dst) for i in oracle]
    return a == b


@pytest.mark.parametrize("case", G["explicit_roundtrip"], ids=lambda c: f"{c['kind']}-{c['sizes']}-{c['device_size']}")
@pytest.mark.parametrize("h2d", [True, False])
def test_dma_plans_equal_oracle_on_golden_layouts(tsa, case, h2d):
    sizes, strides = list(case["sizes"]), list(case["strides"])
    off = 0
    if case["kind"] == "sliced_batch":
        off = sizes[0] // 2
        sizes = [sizes[0] - off]
    lay = tsa.SpyreTensorLayout(case["device_size"], case["stride_map"], tsa.DataFormats.SEN169_FP16)
    native = tsa.dma_plan(sizes, strides, strides, off, lay, h2d)
    oracle = OL.device_stride_infos(sizes, strides, off, case["device_size"], case["stride_map"], h2d, strides)
    assert _plans_equal(native, oracle)


def test_dma_known_answer_native(tsa):
    lay = tsa.SpyreTensorLayout([1024, 256], torch.float16)
    (info,) = tsa.dma_plan([1024, 256], [256, 1], [256, 1], 0, lay, True)
    size, ss, sd, _, _ = info.as_tuple()
    ka = G["dma_known_answer"]
    assert list(reversed(size)) == ka["loop_ranges"]
    assert list(reversed(sd)) == ka["device_strides"]
    assert list(reversed(ss)) == ka["host_strides"]


def test_random_layouts_native_equals_oracle(tsa):
    rng = np.random.default_rng(5)
    for _ in range(300):
        rank = int(rng.integers(1, 6))
        sizes = [int(rng.choice([1, 2, 3, 40, 64, 65, 100, 128, 300])) for _ in range(rank)]
        order = list(rng.permutation(rank))
        if rng.random() < 0.2:
            order = order + [-1]
        strides = OL.contiguous_strides(sizes)
        s = tsa.SpyreTensorLayout(sizes, strides, torch.float16, order)
        o = OL.stl_init(sizes, strides, "float16", order)
        assert (s.device_size, s.stride_map) == (o.device_size, o.stride_map), (sizes, order)
        for h2d in (True, False):
            try:
                oracle = OL.device_stride_infos(sizes, strides, 0, o.device_size, o.stride_map, h2d, strides)
            except RuntimeError:
                with pytest.raises(Exception):
                    tsa.dma_plan(sizes, strides, strides, 0, s, h2d)
                continue
            assert _plans_equal(tsa.dma_plan(sizes, strides, strides, 0, s, h2d), oracle), (sizes, order)


def test_restick_plan_config2(tsa):
    src = tsa.SpyreTensorLayout([4096, 4096], torch.float16)
    dst = tsa.transpose_restick_layout(4096, 4096)
    info = tsa.restick_plan([4096, 4096], src, dst)
    size, ss, sd, _, _ = info.as_tuple()
    # per host element (r, c): src offset and dst offset from the two plans
    # must agree with the closed forms on a sample of elements
    rng = np.random.default_rng(0)
    for _ in range(200):
        idx = [int(rng.integers(s)) for s in size]
        so = sum(i * x for i, x in zip(idx, ss))
        do = sum(i * x for i, x in zip(idx, sd))
        # decode src offset (default sticks [C/64, R, 64]) -> (r, c)
        t, rem = divmod(so, 4096 * 64)
        r, k = divmod(rem, 64)
        c = 64 * t + k
        # dst (transposed sticks [R/64, C, 64]): dst[r // 64][c][r % 64]
        assert do == (r // 64) * 4096 * 64 + c * 64 + r % 64


def test_restick_plan_unsupported_returns_none(tsa):
    # a layout with remainder splitting (folding) has no single-pass plan
    a = tsa.SpyreTensorLayout([38, 64], [64, 1], tsa.DataFormats.SEN169_FP16)
    b = tsa.SpyreTensorLayout([40, 60], torch.float16)
    assert tsa.restick_plan([40, 60], a, b) is None


def test_invalid_arguments_raise(tsa):
    from torch_spyre_amd._lib import SpyreHipError

    with pytest.raises(SpyreHipError):
        tsa.SpyreTensorLayout([1, 2, 3, 4, 5, 6, 7], torch.float16)  # rank 7
    with pytest.raises(SpyreHipError):
        tsa.SpyreTensorLayout([4, 4], [4, 1], torch.float16, [0])  # dim_order length
    with pytest.raises(TypeError):
        tsa.SpyreTensorLayout([4, 4], torch.float64)
    assert tsa.get_device_dtype(torch.float64) == tsa.DataFormats.INVALID
    assert tsa.get_device_dtype(torch.bfloat16) == tsa.DataFormats.SEN169_FP16


def test_sdpa_call_workspace_routes(tsa):
    """The per-call SDPA workspace size (host code): none without a mask or
    for fp16 / bool masks whose slices are whole 16-byte units; a copy with
    16-byte rows of the non-broadcast extent for other fp16 / bool masks;
    V's token-stick relayout for fp32 masks."""
    from torch_spyre_amd import _lib

    L = _lib.lib()
    B, Hq, Hkv, Sq, D = 2, 8, 2, 100, 128

    def need(kind, strides, Skv, ptr=0x10000):
        return L.spyre_sdpa_fwd_call_workspace_bytes(ptr, kind, _lib.i64_array(strides), B, Hq, Hkv, Sq, Skv, D)

    vt = L.spyre_sdpa_fwd_workspace_bytes(B, Hkv, 160, D)
    assert vt == B * Hkv * D * 192 * 2
    # no mask, a grid that fills the device (64 blocks x 8 >= 256 units): nothing
    assert L.spyre_sdpa_fwd_call_workspace_bytes(None, 0, None, 16, Hq, Hkv, Sq, 160, D) == 0
    # no mask, one row tile (g q heads x Sq <= 32 rows): the short-decode kernel takes up to
    # 8 x 64 keys per block at D 64 (batch-1 decode, 512 keys: one block per head, no
    # partials) and 8 x 32 at D 128; longer runs split into such blocks while they fit one
    # round of the device, in blocks of 4 wavefronts (half the keys) when the 8-wavefront
    # split would use at most half the compute units: 4096 keys at D 128 -> 32 splits of
    # [32 rows, 128 + 2] fp32, then a 4-byte arrival flag per (sequence, KV head, split) (the
    # splits merge in the kernel); 513 keys at D 64 -> 3 splits of 256
    assert L.spyre_sdpa_fwd_call_workspace_bytes(None, 0, None, 1, 8, 8, 1, 512, 64) == 0
    assert L.spyre_sdpa_fwd_call_workspace_bytes(None, 0, None, 1, 8, 8, 1, 513, 64) == 8 * 3 * 66 * 4 + 8 * 3 * 4
    assert L.spyre_sdpa_fwd_call_workspace_bytes(None, 0, None, 1, 32, 8, 1, 4096, 128) == \
        32 * 32 * 130 * 4 + 8 * 32 * 4
    # 16 (sequence, KV head) pairs x 9 splits of 256 keys at 8 wavefronts fill more than half
    # the units: 8-wavefront blocks
    assert L.spyre_sdpa_fwd_call_workspace_bytes(None, 0, None, 2, 64, 8, 1, 2200, 128) == \
        2 * 64 * 9 * 130 * 4 + 16 * 9 * 4
    # 64 splits of 8 (sequence, KV head) blocks pass one round, so the call leaves the short
    # kernel; the decode route then takes 32 chunks per (sequence, KV head): their partials
    # [8, 32, 4, 128 + 2] fp32 and flags [8, 32] (above the LDS kernel's split of 32 x [32, 130])
    assert L.spyre_sdpa_fwd_call_workspace_bytes(None, 0, None, 1, 32, 8, 1, 16384, 128) == \
        8 * 32 * (4 * 130 + 1) * 4
    assert L.spyre_sdpa_fwd_call_workspace_bytes(None, 0, None, 1, 8, 8, 40, 127, 64) == 0  # one step
    # decode grids of at least half the device take the split-KV decode kernels on dense K / V:
    # batch 32 x 4096 tokens is one chunk per (sequence, KV head), no partials; batch 2 x 20037
    # tokens, 16 chunks of 20 pages each: [B, Hkv, 16, g, 128 + 2] fp32, then a 4-byte arrival
    # flag per (sequence, KV head, chunk) (the chunks merge in the kernel)
    assert L.spyre_sdpa_fwd_call_workspace_bytes(None, 0, None, 32, 32, 8, 1, 4096, 128) == 0
    assert L.spyre_sdpa_fwd_call_workspace_bytes(None, 0, None, 2, 16, 8, 1, 20037, 128) == \
        2 * 8 * 16 * 2 * 130 * 4 + 2 * 8 * 16 * 4
    # D 64: batch 32 x 16 heads x 2048 tokens, one chunk; batch 8 x 16384 tokens, 4 chunks of 64 + 2
    assert L.spyre_sdpa_fwd_call_workspace_bytes(None, 0, None, 32, 16, 16, 1, 2048, 64) == 0
    assert L.spyre_sdpa_fwd_call_workspace_bytes(None, 0, None, 8, 32, 8, 1, 16384, 64) == \
        8 * 8 * 4 * 4 * 66 * 4 + 8 * 8 * 4 * 4
    # staged as they lie: fp16 rows of 160 keys (320 B), bool rows of 160 B, broadcasts, wider rows
    assert need(1, [0, 0, 160, 1], 160) == 0
    assert need(3, [0, 0, 160, 1], 160) == 0
    assert need(1, [8 * 100 * 168, 100 * 168, 168, 1], 160) == 0
    assert need(1, [0, 160, 0, 1], 160) == 0
    # a misaligned pointer, or a slice that ends inside a 16-byte unit: copied
    assert need(1, [0, 0, 160, 1], 160, ptr=0x10002) == 100 * 320
    assert need(1, [0, 0, 168, 1], 164) == 100 * 336  # 164 keys = 328 B -> rows of 336
    # odd rows: [Sq, 77] fp16 -> 160-B rows; [B, 1, Sq, 77] bool -> 80-B rows, per sequence
    assert need(1, [0, 0, 77, 1], 77) == 100 * 160
    assert need(3, [100 * 77, 0, 77, 1], 77) == B * 100 * 80
    # a padding row [1, Hq, 1, 77] and a transposed view (key stride Sq)
    assert need(1, [0, 77, 0, 1], 77) == Hq * 160
    assert need(1, [0, 0, 1, 100], 77) == 100 * 160
    # fp32 masks take V's relayout
    assert need(2, [0, 0, 160, 1], 160) == vt


def test_paged_decode_workspace_and_kernel_count(tsa):
    """The paged decode's workspace (host code): fp32 chunk partials
    [B, Hkv, chunks, g, D + 2], then a 4-byte arrival flag per (sequence, KV
    head, chunk); chunks = ceil(max_context_len / (8 split_tokens)).  The
    kernel count of one call: 1 whenever every context fits one chunk (no
    device is asked), a negative error code for bad sizes."""
    from torch_spyre_amd import _lib

    L = _lib.lib()

    def ws(B, Hq, Hkv, D, ctx, split):
        return L.spyre_paged_decode_attn_workspace_bytes(B, Hq, Hkv, D, ctx, split)

    # Llama-3-8B decode (B 32, 32 / 8 heads, ctx 4096, split 512): one chunk
    assert ws(32, 32, 8, 128, 4096, 512) == 32 * 8 * 1 * (4 * 130 + 1) * 4
    # 64 sequences up to 32768 tokens: 8 chunks
    assert ws(64, 32, 8, 128, 32768, 512) == 64 * 8 * 8 * (4 * 130 + 1) * 4
    # B 4, 64 / 8 heads, 131073 tokens: 33 chunks of g 8
    assert ws(4, 64, 8, 128, 131073, 512) == 4 * 8 * 33 * (8 * 130 + 1) * 4
    # D 64, MHA, split 64: chunks of 512 tokens
    assert ws(3, 16, 16, 64, 1025, 64) == 3 * 16 * 3 * (1 * 66 + 1) * 4
    assert ws(0, 32, 8, 128, 4096, 512) == 0 and ws(2, 30, 8, 128, 4096, 512) == 0
    for args in [(32, 32, 8, 128, 4096, 512), (1, 8, 8, 64, 0, 512), (6, 32, 8, 128, 2048, 256)]:
        assert L.spyre_paged_decode_attn_kernels(*args) == 1
    for bad in [(0, 32, 8, 128, 4096, 512), (2, 30, 8, 128, 4096, 512), (2, 32, 8, 96, 4096, 512),
                (2, 32, 8, 128, 4096, 100), (2, 32, 8, 128, -1, 512)]:
        assert L.spyre_paged_decode_attn_kernels(*bad) == _lib.SPYRE_EINVAL
