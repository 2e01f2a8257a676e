"""The prepared calls captured into HIP graphs (torch.cuda.CUDAGraph).

A serving loop replays one captured decode step: the KV append plus the
decode call.  The library allocates and clears nothing and launches on the
caller's current stream, so both can be captured.  Each test replays its
graph several times, with eager work that changes the inputs in between, and
checks every replay bit for bit against the same calls made eagerly.
"""

import numpy as np
import pytest
import torch

from oracle import relayout as OR
from tests.conftest import SEED
from tests.test_attention_gpu import make_case

pytestmark = pytest.mark.gpu


def _capture(cuda, fn):
    side = torch.cuda.Stream(device=cuda)
    side.wait_stream(torch.cuda.current_stream(cuda))
    with torch.cuda.stream(side):  # warm-up outside the capture
        fn()
    torch.cuda.current_stream(cuda).wait_stream(side)
    torch.cuda.synchronize(cuda)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    return g


def test_decode_step_graph_replays_match_eager(cuda):
    """kv_append + PagedDecode with contexts up to 5000 tokens at split 512
    (two chunks, merged inside the split kernel by arrival flags that each
    replay sets and clears) in one graph; each replay follows new q / new
    token values written eagerly."""
    import torch_spyre_amd as tsa

    B, Hq, Hkv, D = 6, 32, 8, 128
    lens = [700, 64, 1999, 5000, 1, 4097]
    cache, table, lens_t, q = make_case(cuda, B, Hq, Hkv, D, lens, SEED + 91)
    t, l = table.to(cuda), lens_t.to(cuda)
    pos = (l - 1).contiguous()  # rewrite each sequence's last token
    gg = torch.Generator(device=cuda).manual_seed(SEED + 92)
    k_new = torch.randn((B, Hkv, D), generator=gg, device=cuda).half()
    v_new = torch.randn((B, Hkv, D), generator=gg, device=cuda).half()
    q_static = q.clone()
    call = tsa.PagedDecode(q_static, cache.k, cache.v, t, l, max_context_len=max(lens))
    ref = tsa.PagedDecode(q_static, cache.k, cache.v, t, l, max_context_len=max(lens))
    assert call.passes == 1

    def step():
        tsa.kv_append(k_new, v_new, cache.k, cache.v, t, pos)
        call()

    g = _capture(cuda, step)
    for i in range(3):
        q_static.copy_(torch.randn(q.shape, generator=gg, device=cuda).half())
        k_new.copy_(torch.randn(k_new.shape, generator=gg, device=cuda).half())
        v_new.copy_(torch.randn(v_new.shape, generator=gg, device=cuda).half())
        torch.cuda.synchronize(cuda)
        g.replay()
        torch.cuda.synchronize(cuda)
        got = call.out.clone()
        tsa.kv_append(k_new, v_new, cache.k, cache.v, t, pos)
        want = ref()
        torch.cuda.synchronize(cuda)
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), i


def test_relayout_graph_replays_match_oracle(cuda):
    """A prepared to-sticks copy and a transpose-restick in one graph, fed new
    bit patterns before each replay; every replay bit-exact to the oracle."""
    import torch_spyre_amd as tsa

    R, C = 256, 192
    x = torch.empty((R, C), dtype=torch.float16, device=cuda)
    stl = tsa.SpyreTensorLayout([R, C], torch.float16)
    trl = tsa.transpose_restick_layout(R, C)
    dev = tsa.device_buffer(tsa.spyre_empty_with_layout([R, C], [C, 1], torch.float16, stl, cuda))
    tr = tsa.device_buffer(tsa.spyre_empty_with_layout([R, C], [C, 1], torch.float16, trl, cuda))
    to_sticks = tsa.DmaCopy(x, dev, tsa.dma_plan([R, C], [C, 1], [C, 1], 0, stl, True))
    restick = tsa.DmaCopy(dev, tr, [tsa.restick_plan([R, C], stl, trl)])

    def fn():
        to_sticks()
        restick()

    g = _capture(cuda, fn)
    for i in range(3):
        bits = OR.random_finite_f16_bits((R, C), SEED + 200 + i)
        x.copy_(torch.from_numpy(bits.view(np.int16)).to(cuda).view(torch.float16))
        torch.cuda.synchronize(cuda)
        g.replay()
        torch.cuda.synchronize(cuda)
        got_s = dev.view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1)
        got_t = tr.view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1)
        assert np.array_equal(got_s, OR.to_sticks(bits).reshape(-1)), i
        assert np.array_equal(got_t, OR.transpose_restick(bits).reshape(-1)), i


@pytest.mark.parametrize("B,S", [(1, 4096), (4, 8192)])
def test_dense_decode_graph_replays_match_eager(cuda, B, S):
    """A prepared dense decode in a graph -- batch 1 (short-decode kernel,
    key splits + merge) and batch 4 x 8192 tokens (the split-KV decode
    kernel, chunks merged in it); q and the newest key/value row rewritten
    eagerly before each replay; every replay bit-equal to the eager call."""
    import torch_spyre_amd as tsa

    gg = torch.Generator(device=cuda).manual_seed(SEED + 95)
    q = torch.randn((B, 32, 1, 128), generator=gg, device=cuda).half()
    k = torch.randn((B, 8, S, 128), generator=gg, device=cuda).half()
    v = torch.randn((B, 8, S, 128), generator=gg, device=cuda).half()
    call = tsa.SdpaCall(q, k, v, enable_gqa=True, return_lse=True)
    g = _capture(cuda, call)
    for i in range(3):
        q.copy_(torch.randn(q.shape, generator=gg, device=cuda).half())
        k[:, :, S - 1].copy_(torch.randn((B, 8, 128), generator=gg, device=cuda).half())
        v[:, :, S - 1].copy_(torch.randn((B, 8, 128), generator=gg, device=cuda).half())
        g.replay()
        want, want_lse = tsa.scaled_dot_product_attention(q, k, v, enable_gqa=True, return_lse=True)
        torch.cuda.synchronize()
        assert torch.equal(call.out.view(torch.int16), want.view(torch.int16)), f"replay {i}"
        assert torch.equal(call.lse, want_lse), f"replay {i}"
