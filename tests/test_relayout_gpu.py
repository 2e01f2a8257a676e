"""GPU parity of the stick relayouts against the oracle (bit-exact).

Inputs are raw 16-bit patterns (finite fp16) compared as int16, so nothing
goes through a float conversion.
"""

import itertools
import json
import os

import numpy as np
import pytest
import torch

from oracle import layout as OL
from oracle import relayout as OR
from oracle import kv as OK
from tests.conftest import SEED

pytestmark = pytest.mark.gpu

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "stl_golden.json")))


def _bits_tensor(bits: np.ndarray, device) -> torch.Tensor:
    return torch.from_numpy(bits.view(np.int16)).to(device).view(torch.float16)


def _as_bits(t: torch.Tensor) -> np.ndarray:
    """Raw 16-bit patterns; a SpyreTensor gives its buffer in stick order."""
    import torch_spyre_amd as tsa

    if isinstance(t, tsa.SpyreTensor):
        t = tsa.device_buffer(t)
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def test_config2_to_sticks_full(cuda):
    import torch_spyre_amd as tsa

    bits = OR.random_finite_f16_bits((4096, 4096), SEED)
    x = _bits_tensor(bits, cuda)
    stl = tsa.SpyreTensorLayout([4096, 4096], torch.float16)
    assert stl.device_size == [64, 4096, 64] and stl.stride_map == [64, 4096, 1]
    dev = tsa.to_device_layout(x, stl)
    torch.cuda.synchronize()
    assert np.array_equal(_as_bits(dev), OR.to_sticks(bits))


def test_config2_from_sticks_full(cuda):
    import torch_spyre_amd as tsa

    bits = OR.random_finite_f16_bits((4096, 4096), SEED + 1)
    stl = tsa.SpyreTensorLayout([4096, 4096], torch.float16)
    dev = _bits_tensor(OR.to_sticks(bits), cuda)
    host = tsa.from_device_layout(dev, stl, [4096, 4096])
    torch.cuda.synchronize()
    assert np.array_equal(_as_bits(host), bits)


def test_config2_transpose_restick_full(cuda):
    import torch_spyre_amd as tsa

    bits = OR.random_finite_f16_bits((4096, 4096), SEED + 2)
    x = _bits_tensor(bits, cuda)
    src = tsa.SpyreTensorLayout([4096, 4096], torch.float16)
    dst = tsa.transpose_restick_layout(4096, 4096)
    assert dst.device_size == [64, 4096, 64] and dst.stride_map == [262144, 1, 4096]
    want = OR.transpose_restick(bits)
    # device -> device restickify (single pass)
    dev = tsa.to_device_layout(x, src)
    out = tsa.restickify(dev, dst)
    # host order -> transposed sticks directly
    out2 = tsa.to_device_layout(x, dst)
    torch.cuda.synchronize()
    assert np.array_equal(_as_bits(out), want)
    assert np.array_equal(_as_bits(out2), want)
    # and back
    back = tsa.from_device_layout(out)
    assert np.array_equal(_as_bits(back), bits)


@pytest.mark.parametrize("case", GOLDEN["explicit_roundtrip"], ids=lambda c: f"{c['kind']}-{c['sizes']}-{c['device_size']}")
def test_golden_explicit_layouts(cuda, case):
    """Every explicit layout of tests/tensor/test_tensor_layout.py:193-405:
    device bytes equal the oracle's H2D, and D2H restores the tensor."""
    import torch_spyre_amd as tsa

    sizes, strides = list(case["sizes"]), list(case["strides"])
    span = 1 + sum((s - 1) * st for s, st in zip(sizes, strides))
    store = OR.random_finite_f16_bits((span,), SEED + span)
    off = 0
    if case["kind"] == "sliced_batch":
        off = sizes[0] // 2
        sizes = [sizes[0] - off]
    stl = tsa.SpyreTensorLayout(case["device_size"], case["stride_map"], tsa.DataFormats.SEN169_FP16)
    base = _bits_tensor(store, cuda)
    x = base.as_strided(sizes, strides, off)
    dev = tsa.to_device_layout(x, stl)
    want = OL.h2d(store, sizes, strides, off, OL.Layout(case["device_size"], case["stride_map"]))
    got = _as_bits(dev).reshape(-1)
    assert np.array_equal(got[: want.size], want)
    back = tsa.from_device_layout(dev)
    ref = np.lib.stride_tricks.as_strided(store[off:], shape=sizes, strides=[s * 2 for s in strides])
    assert np.array_equal(_as_bits(back).reshape(sizes), ref)


def _random_cases(n, seed):
    rng = np.random.default_rng(seed)
    for _ in range(n):
        rank = int(rng.integers(1, 5))
        sizes = [int(rng.choice([1, 3, 40, 64, 65, 127, 128, 200])) for _ in range(rank)]
        while np.prod(sizes) > 300_000:
            sizes[int(rng.integers(rank))] = 3
        orders = list(itertools.permutations(range(rank)))
        order = list(orders[int(rng.integers(len(orders)))])
        yield sizes, order


@pytest.mark.parametrize("sizes,order", list(_random_cases(40, SEED)))
def test_random_dim_orders_vs_oracle(cuda, sizes, order):
    """Default/dim_order layouts of random shapes (padding, unit dims) vs the oracle."""
    import torch_spyre_amd as tsa

    strides = OL.contiguous_strides(sizes)
    stl = tsa.SpyreTensorLayout(sizes, strides, torch.float16, order)
    o = OL.stl_init(sizes, strides, "float16", order)
    assert (stl.device_size, stl.stride_map) == (o.device_size, o.stride_map)
    bits = OR.random_finite_f16_bits((int(np.prod(sizes)),), SEED + len(sizes))
    x = _bits_tensor(bits, cuda).view(sizes)
    dev = tsa.to_device_layout(x, stl)
    want = OL.h2d(bits, sizes, strides, 0, o)
    assert np.array_equal(_as_bits(dev).reshape(-1)[: want.size], want)
    back = tsa.from_device_layout(dev)
    assert np.array_equal(_as_bits(back).reshape(-1), bits)


@pytest.mark.parametrize("sizes,order", list(_random_cases(24, SEED + 7)))
def test_restickify_random_vs_oracle(cuda, sizes, order):
    """D2D restickify from the default layout to a dim_order layout equals the
    oracle's H2D(dst) of D2H(src), padding included."""
    import torch_spyre_amd as tsa

    strides = OL.contiguous_strides(sizes)
    src = tsa.SpyreTensorLayout(sizes, torch.float16)
    dst = tsa.SpyreTensorLayout(sizes, strides, torch.float16, order)
    bits = OR.random_finite_f16_bits((int(np.prod(sizes)),), SEED + 3 * len(sizes))
    x = _bits_tensor(bits, cuda).view(sizes)
    out = tsa.restickify(tsa.to_device_layout(x, src), dst)
    want = OL.h2d(bits, sizes, strides, 0, OL.stl_init(sizes, strides, "float16", order))
    assert np.array_equal(_as_bits(out).reshape(-1)[: want.size], want)


# Shapes whose nests take the 32 x 32-stick tile kernel: partial tiles along
# both stick loops, and one or two outer loops.
def test_prepared_dma_copy_matches(cuda):
    """DmaCopy (validated once, launched repeatedly) == dma_copy."""
    import torch_spyre_amd as tsa

    sizes = [100, 2112]
    bits = OR.random_finite_f16_bits(tuple(sizes), SEED + 17)
    x = _bits_tensor(bits, cuda)
    stl = tsa.SpyreTensorLayout(sizes, torch.float16)
    want = tsa.device_buffer(tsa.to_device_layout(x, stl))
    out = torch.zeros_like(want)
    call = tsa.DmaCopy(x, out, tsa.dma_plan(sizes, [2112, 1], [2112, 1], 0, stl, True))
    for _ in range(3):
        call()
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), want.view(torch.int16))


TILE_CASES = [([100, 2112], [0, 1]), ([33, 4096], [0, 1]), ([100, 40, 2112], [0, 1, 2]),
              ([40, 100, 2112], [1, 0, 2]), ([2, 3, 100, 2112], [2, 1, 0, 3])]


@pytest.mark.parametrize("sizes,order", TILE_CASES, ids=lambda v: str(v))
def test_stick_tile_layouts_vs_oracle(cuda, sizes, order):
    import torch_spyre_amd as tsa

    strides = OL.contiguous_strides(sizes)
    stl = tsa.SpyreTensorLayout(sizes, strides, torch.float16, order)
    o = OL.stl_init(sizes, strides, "float16", order)
    bits = OR.random_finite_f16_bits((int(np.prod(sizes)),), SEED + sum(sizes))
    x = _bits_tensor(bits, cuda).view(sizes)
    dev = tsa.to_device_layout(x, stl)
    want = OL.h2d(bits, sizes, strides, 0, o)
    assert np.array_equal(_as_bits(dev).reshape(-1)[: want.size], want)
    back = tsa.from_device_layout(dev)
    assert np.array_equal(_as_bits(back).reshape(-1), bits)


@pytest.mark.parametrize("sizes", [[104, 2112], [3, 136, 4160], [8, 4096]], ids=str)
def test_transpose_restick_partial_tiles_vs_oracle(cuda, sizes):
    """Transpose-restick nests whose 64 x 64 tile counts are not multiples of
    the four tiles a wavefront takes."""
    import torch_spyre_amd as tsa

    order = list(range(len(sizes)))
    order[-2], order[-1] = order[-1], order[-2]
    strides = OL.contiguous_strides(sizes)
    src = tsa.SpyreTensorLayout(sizes, torch.float16)
    dst = tsa.SpyreTensorLayout(sizes, strides, torch.float16, order)
    bits = OR.random_finite_f16_bits((int(np.prod(sizes)),), SEED + 11 * len(sizes))
    x = _bits_tensor(bits, cuda).view(sizes)
    out = tsa.restickify(tsa.to_device_layout(x, src), dst)
    want = OL.h2d(bits, sizes, strides, 0, OL.stl_init(sizes, strides, "float16", order))
    assert np.array_equal(_as_bits(out).reshape(-1)[: want.size], want)


@pytest.mark.parametrize("sizes", [[64, 1024], [192, 2048], [2, 128, 1024], [4, 64, 3072]], ids=str)
def test_transpose_whole_tile_rows_vs_oracle(cuda, sizes):
    """Transpose nests of whole rows of 64 x 64 tiles with outer loops:
    device restickify and host -> transposed sticks directly, bit-exact, and
    back."""
    import torch_spyre_amd as tsa

    order = list(range(len(sizes)))
    order[-2], order[-1] = order[-1], order[-2]
    strides = OL.contiguous_strides(sizes)
    src = tsa.SpyreTensorLayout(sizes, torch.float16)
    dst = tsa.SpyreTensorLayout(sizes, strides, torch.float16, order)
    bits = OR.random_finite_f16_bits((int(np.prod(sizes)),), SEED + 13 * sum(sizes))
    x = _bits_tensor(bits, cuda).view(sizes)
    want = OL.h2d(bits, sizes, strides, 0, OL.stl_init(sizes, strides, "float16", order))
    out = tsa.restickify(tsa.to_device_layout(x, src), dst)
    out2 = tsa.to_device_layout(x, dst)
    torch.cuda.synchronize()
    assert np.array_equal(_as_bits(out).reshape(-1)[: want.size], want)
    assert np.array_equal(_as_bits(out2).reshape(-1)[: want.size], want)
    back = tsa.from_device_layout(out)
    assert np.array_equal(_as_bits(back).reshape(-1), bits)


def test_page_layouts_vs_oracle(cuda):
    """The paged K/V cache layouts built by the relayout engine equal the
    oracle's H2D of the same logical pages."""
    import torch_spyre_amd as tsa
    from oracle import attention as OA

    P, Hkv, D = 6, 2, 128
    bits_k = OR.random_finite_f16_bits((P, Hkv, 64, D), SEED + 11)
    bits_v = OR.random_finite_f16_bits((P, Hkv, 64, D), SEED + 12)
    cache = tsa.PagedKVCache.from_pages(_bits_tensor(bits_k, cuda), _bits_tensor(bits_v, cuda))
    wk, wv = OA.logical_to_pages(bits_k, bits_v)
    assert np.array_equal(_as_bits(cache.k).reshape(-1), wk)
    assert np.array_equal(_as_bits(cache.v).reshape(-1), wv)


@pytest.mark.parametrize("shape,dims,offsets", [
    ((1, 8, 64, 128), [2], [5]),
    ((4, 8, 64, 128), [0, 2], [3, 63]),
    ((3, 5, 7), [1], [2]),
    ((64,), [0], [17]),
])
def test_overwrite_vs_oracle(cuda, shape, dims, offsets):
    import torch_spyre_amd as tsa

    out_bits = OR.random_finite_f16_bits(shape, SEED + 5)
    in_shape = list(shape)
    for d in dims:
        in_shape[d] = 1 if shape[d] > 1 else shape[d]
    if shape == (64,):
        in_shape = [9]
    in_bits = OR.random_finite_f16_bits(tuple(in_shape), SEED + 6)
    out = _bits_tensor(out_bits, cuda)
    inp = _bits_tensor(in_bits, cuda)
    torch.ops.spyre.overwrite(inp, out, dims, offsets)
    want = out_bits.copy()
    OK.overwrite(in_bits, want, dims, offsets)
    assert np.array_equal(_as_bits(out), want)


def test_overwrite_sequential_kv_pattern(cuda):
    """tests/inductor/test_overwrite.py:166-187: ten single-token writes into a
    [1, 8, 64, 128] cache at dim 2, each at its own offset."""
    import torch_spyre_amd as tsa

    cache = torch.zeros((1, 8, 64, 128), dtype=torch.float16, device=cuda)
    want = np.zeros((1, 8, 64, 128), dtype=np.uint16)
    for i in range(10):
        tok_bits = OR.random_finite_f16_bits((1, 8, 1, 128), SEED + 100 + i)
        tsa.overwrite(_bits_tensor(tok_bits, cuda), cache, [2], [i])
        OK.overwrite(tok_bits, want, [2], [i])
    assert np.array_equal(_as_bits(cache), want)


def test_empty_and_errors(cuda):
    import torch_spyre_amd as tsa
    from torch_spyre_amd._lib import SpyreHipError

    x = torch.empty((0, 64), dtype=torch.float16, device=cuda)
    stl = tsa.SpyreTensorLayout([0, 64], torch.float16)
    dev = tsa.to_device_layout(x, stl)
    assert tsa.from_device_layout(dev).shape == (0, 64)
    # a loop nest past the end of the destination is refused on the host
    src = torch.zeros(128, dtype=torch.float16, device=cuda)
    dst = torch.zeros(64, dtype=torch.float16, device=cuda)
    info = tsa._lib.StrideInfo()
    info.rank, info.size[0], info.stride_src[0], info.stride_dst[0] = 1, 128, 1, 1
    with pytest.raises(SpyreHipError):
        tsa.relayout.dma_copy(src, dst, [info])
    with pytest.raises(RuntimeError):  # CPU buffers: no CPU path
        tsa.relayout.h2d_buffer(torch.zeros(64, 64, dtype=torch.float16), stl)


# Row-major <-> default sticks through the stepped stick-tile kernel.  The
# stick loop (host dim 0 in the default layout) and the last dim's sticks
# form the tiles; the remaining loops step whole tiles.  Loops that are
# dense on both sides merge (the B tiles with the next host dim when host
# rows are dense), so [96, 3, 16, 4096] steps two loops and the view
# [96, 3, 8, 4096] of a [96, 3, 8, 4160] buffer three; in the view of a
# [96, 3, 10, 4160] buffer nothing merges: four.
STICK_STEP_CASES = [([64, 2048], None), ([96, 4096], None), ([96, 3, 16, 4096], None),
                    ([96, 3, 8, 4096], {3: 4160}), ([96, 3, 8, 4096], {2: 10, 3: 4160})]


def _host_view(sizes, pad, seed, cuda):
    """Random bit patterns as a CUDA tensor of `sizes`: contiguous, or with
    pad = {dim: n, ...} the view [..., :sizes[dim], ...] of a buffer whose
    dims are n long.  Returns the tensor, the flat store, its strides and
    offset."""
    pad = pad or {}
    full = [pad.get(d, s) for d, s in enumerate(sizes)]
    store = OR.random_finite_f16_bits((int(np.prod(full)),), seed)
    x = _bits_tensor(store, cuda).view(full)
    for d in pad:
        x = x.narrow(d, 0, sizes[d])
    return x, store, list(x.stride()), x.storage_offset()


@pytest.mark.parametrize("sizes,pad", STICK_STEP_CASES, ids=str)
def test_stepped_stick_tiles_vs_oracle(cuda, sizes, pad):
    """Host order (contiguous or a strided view) -> default sticks -> host
    order: device bytes equal the oracle's H2D, and D2H restores every
    element.  The layout's stride_map refers to the host tensor's own
    strides, as x.to(device_layout=...) records them."""
    import torch_spyre_amd as tsa

    x, store, strides, off = _host_view(sizes, pad, SEED + 400 + sum(sizes) + len(pad or {}), cuda)
    order = list(range(len(sizes)))
    stl = tsa.SpyreTensorLayout(list(sizes), strides, torch.float16, order)
    dev = tsa.to_device_layout(x, stl)
    want = OL.h2d(store, list(sizes), strides, off, OL.stl_init(list(sizes), strides, "float16", order))
    assert np.array_equal(_as_bits(dev).reshape(-1)[: want.size], want)
    back = tsa.from_device_layout(dev)
    torch.cuda.synchronize()
    assert torch.equal(back.contiguous().view(torch.int16), x.contiguous().view(torch.int16))


# Transposes (the stick moves from the last dim to the one before it):
# device restickify of 64 x 64-element tiles, four consecutive ones to a
# wavefront, so the first stepped loop's count is a multiple of 4:
# [768, 1024] and [4, 512, 256] step both ways; in [768, 640] one
# direction's first loop has 10 tiles, in [3, 256, 320] both directions'
# is dim 0 (3), and those take the LDS-staged transpose.  The host view
# [3, 5, 128, 256] of a [3, 6, 128, 256] buffer goes straight to transposed
# sticks (tile loops 4, 2, then 5 and 3) and back.
@pytest.mark.parametrize("sizes", [[768, 640], [768, 1024], [3, 256, 320], [4, 512, 256]], ids=str)
def test_stepped_restickify_vs_oracle(cuda, sizes):
    import torch_spyre_amd as tsa

    order = list(range(len(sizes)))
    order[-2], order[-1] = order[-1], order[-2]
    strides = OL.contiguous_strides(sizes)
    src = tsa.SpyreTensorLayout(sizes, torch.float16)
    dst = tsa.SpyreTensorLayout(sizes, strides, torch.float16, order)
    bits = OR.random_finite_f16_bits((int(np.prod(sizes)),), SEED + 410 + sum(sizes))
    x = _bits_tensor(bits, cuda).view(sizes)
    out = tsa.restickify(tsa.to_device_layout(x, src), dst)
    want = OL.h2d(bits, sizes, strides, 0, OL.stl_init(sizes, strides, "float16", order))
    assert np.array_equal(_as_bits(out).reshape(-1)[: want.size], want)
    back = tsa.restickify(out, src)
    assert np.array_equal(_as_bits(back).reshape(-1), _as_bits(tsa.to_device_layout(x, src)).reshape(-1))


def test_stepped_transpose_from_strided_host_vs_oracle(cuda):
    import torch_spyre_amd as tsa

    sizes = [3, 5, 128, 256]
    x, store, strides, off = _host_view(sizes, {1: 6}, SEED + 420, cuda)
    order = [0, 1, 3, 2]
    dst = tsa.SpyreTensorLayout(sizes, strides, torch.float16, order)
    dev = tsa.to_device_layout(x, dst)
    want = OL.h2d(store, sizes, strides, off, OL.stl_init(sizes, strides, "float16", order))
    assert np.array_equal(_as_bits(dev).reshape(-1)[: want.size], want)
    back = tsa.from_device_layout(dev)
    torch.cuda.synchronize()
    assert torch.equal(back.contiguous().view(torch.int16), x.contiguous().view(torch.int16))


# Narrow stick tiles: a loop of 8, 16 or 24 sticks beside the stick (host
# dim 0 of a default layout: a batch of 8, a KV cache of 8 sequences) moves
# in 8 x 128 / 16 x 64 tiles one way and 128 x 8 / 64 x 16 the other.
NARROW_CASES = [([8, 1024, 4096], None), ([16, 256, 2048], None), ([24, 128, 1024], None),
                ([8, 8, 2048, 128], None), ([8, 3, 64, 4096], {2: 72})]


@pytest.mark.parametrize("sizes,pad", NARROW_CASES, ids=str)
def test_narrow_stick_tiles_vs_oracle(cuda, sizes, pad):
    import torch_spyre_amd as tsa

    x, store, strides, off = _host_view(sizes, pad, SEED + 450 + sum(sizes), cuda)
    order = list(range(len(sizes)))
    stl = tsa.SpyreTensorLayout(list(sizes), strides, torch.float16, order)
    dev = tsa.to_device_layout(x, stl)
    want = OL.h2d(store, list(sizes), strides, off, OL.stl_init(list(sizes), strides, "float16", order))
    assert np.array_equal(_as_bits(dev).reshape(-1)[: want.size], want)
    back = tsa.from_device_layout(dev)
    torch.cuda.synchronize()
    assert torch.equal(back.contiguous().view(torch.int16), x.contiguous().view(torch.int16))


@pytest.mark.parametrize("sizes", [[64, 64], [1, 64, 64], [2, 64, 64]], ids=str)
def test_single_tile_restickify_vs_oracle(cuda, sizes):
    """A transpose that is one 64 x 64 tile (or one per outer index): no
    tile loop longer than one."""
    import torch_spyre_amd as tsa

    order = list(range(len(sizes)))
    order[-2], order[-1] = order[-1], order[-2]
    strides = OL.contiguous_strides(sizes)
    src = tsa.SpyreTensorLayout(sizes, torch.float16)
    dst = tsa.SpyreTensorLayout(sizes, strides, torch.float16, order)
    bits = OR.random_finite_f16_bits((int(np.prod(sizes)),), SEED + 470 + sum(sizes))
    x = _bits_tensor(bits, cuda).view(sizes)
    out = tsa.restickify(tsa.to_device_layout(x, src), dst)
    want = OL.h2d(bits, sizes, strides, 0, OL.stl_init(sizes, strides, "float16", order))
    assert np.array_equal(_as_bits(out).reshape(-1)[: want.size], want)
    back = tsa.from_device_layout(tsa.to_device_layout(x, dst))
    torch.cuda.synchronize()
    assert torch.equal(back.contiguous().view(torch.int16), x.view(torch.int16))


# A small side (2 .. 31 sticks, no multiple of 8) beside the stick, its
# other side dense: n rows of T sticks against one dense run per tile, both
# ways (the dma_stick_small_kernel route).
SMALL_CASES = [([3, 2048, 4096], None), ([5, 64, 4096], None), ([2, 1024, 2048], None), ([12, 256, 1024], None),
               ([31, 64, 2048], None), ([4, 8, 2048, 128], None), ([3, 5, 64, 4096], {2: 72})]


@pytest.mark.parametrize("sizes,pad", SMALL_CASES, ids=str)
def test_small_side_stick_tiles_vs_oracle(cuda, sizes, pad):
    import torch_spyre_amd as tsa

    x, store, strides, off = _host_view(sizes, pad, SEED + 480 + sum(sizes), cuda)
    order = list(range(len(sizes)))
    stl = tsa.SpyreTensorLayout(list(sizes), strides, torch.float16, order)
    dev = tsa.to_device_layout(x, stl)
    want = OL.h2d(store, list(sizes), strides, off, OL.stl_init(list(sizes), strides, "float16", order))
    assert np.array_equal(_as_bits(dev).reshape(-1)[: want.size], want)
    back = tsa.from_device_layout(dev)
    torch.cuda.synchronize()
    assert torch.equal(back.contiguous().view(torch.int16), x.contiguous().view(torch.int16))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [[1000, 1000], [3, 64, 4100], [8, 1024, 512], [4096, 2048]], ids=str)
def test_relayout_other_dtypes_vs_oracle(cuda, dtype, shape):
    """fp32 tensors (32 elements a stick) and bf16 tensors (16-bit patterns
    in the fp16 device format) to their default device layout and back: the
    device bytes equal the oracle's DMA execution, the round trip is
    bit-exact."""
    import math

    import torch_spyre_amd as tsa

    gen = torch.Generator().manual_seed(SEED + 170 + len(shape))
    n = math.prod(shape)
    if dtype == torch.float32:
        raw = torch.randint(-(2 ** 31), 2 ** 31 - 1, (n,), generator=gen, dtype=torch.int64).to(torch.int32)
        name, npt = "float32", np.uint32
    else:
        raw = torch.randint(-(2 ** 15), 2 ** 15 - 1, (n,), generator=gen, dtype=torch.int32).to(torch.int16)
        name, npt = "float16", np.uint16
    x = raw.view(dtype).view(shape)
    stl = tsa.SpyreTensorLayout(shape, dtype)
    o = OL.stl_default(shape, name)
    assert (stl.device_size, stl.stride_map) == (o.device_size, o.stride_map)
    dev = tsa.to_device_layout(x.to(cuda), stl)
    torch.cuda.synchronize()
    got = tsa.device_buffer(dev).contiguous().view(raw.dtype).cpu().numpy().view(npt).reshape(-1)
    want = OL.h2d(raw.numpy().view(npt), shape, OL.contiguous_strides(shape), 0, o)
    assert got.size >= want.size
    assert np.array_equal(got[:want.size], want)
    back = dev.cpu()
    assert torch.equal(back.view(raw.dtype).reshape(-1), raw)


@pytest.mark.parametrize("nbytes,off_s,off_d", [(32 << 20, 0, 0), ((5 << 17) + 48, 0, 0), ((3 << 17) + 16, 64, 16),
                                                (1 << 17, 8, 8), ((1 << 17) - 16, 0, 0), (48, 0, 0)])
def test_contiguous_copy_blocks(cuda, nbytes, off_s, off_d):
    """One contiguous nest (the byte-for-byte copy of an allocation): whole
    128 KiB blocks through LDS, the tail by the vector kernel; offsets that
    keep 16-byte alignment; shorter copies wholly by the vector kernel.
    Bit-exact, and nothing outside the copy is written."""
    import torch_spyre_amd as tsa

    n = nbytes // 2
    bits = OR.random_finite_f16_bits((n + off_s // 2,), SEED + 500 + nbytes % 997)
    src = _bits_tensor(bits, cuda)
    dst = torch.full((n + off_d // 2 + 64,), -1.0, dtype=torch.float16, device=cuda)
    info = tsa._lib.StrideInfo()
    info.rank, info.size[0], info.stride_src[0], info.stride_dst[0] = 1, n, 1, 1
    info.offset_src, info.offset_dst = off_s // 2, off_d // 2
    tsa.relayout.dma_copy(src, dst, [info])
    got = _as_bits(dst)
    assert np.array_equal(got[off_d // 2:off_d // 2 + n], bits[off_s // 2:])
    minus_one = np.array([-1.0], dtype=np.float16).view(np.uint16)[0]
    assert (got[:off_d // 2] == minus_one).all() and (got[off_d // 2 + n:] == minus_one).all()
