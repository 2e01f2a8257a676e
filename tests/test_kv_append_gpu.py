"""GPU parity of the batched paged KV append (bit-exact) and of
append-then-attend (the long-context decode step)."""

import math

import numpy as np
import pytest
import torch

from oracle import attention as OA
from oracle import kv as OK
from oracle import relayout as OR
from tests.conftest import SEED
from tests.test_attention_gpu import (assert_close, assert_token_count_exact, make_case, mean_v64, oracle_lse64,
                                     oracle_rows, run)

pytestmark = pytest.mark.gpu


def _bits(shape, seed):
    return OR.random_finite_f16_bits(shape, seed)


def _t(bits, dev):
    return torch.from_numpy(bits.view(np.int16)).to(dev).view(torch.float16)


@pytest.mark.parametrize("D", [64, 128])
def test_kv_append_bitexact(cuda, D):
    import torch_spyre_amd as tsa

    P, Hkv, B = 9, 4, 5
    k_log = _bits((P, Hkv, 64, D), SEED + 1)
    v_log = _bits((P, Hkv, 64, D), SEED + 2)
    cache = tsa.PagedKVCache.from_pages(_t(k_log, cuda), _t(v_log, cuda))
    table = np.array([[3, 1], [0, 8], [2, 5], [6, 7], [4, 4]], dtype=np.int32)
    positions = np.array([5, 64, 127, -1, 0], dtype=np.int32)
    k_new = _bits((B, Hkv, D), SEED + 3)
    v_new = _bits((B, Hkv, D), SEED + 4)
    tsa.kv_append(_t(k_new, cuda), _t(v_new, cuda), cache.k, cache.v,
                  torch.from_numpy(table).to(cuda), torch.from_numpy(positions).to(cuda))
    OK.append_token(k_log, v_log, k_new, v_new, table, positions)
    wk, wv = OA.logical_to_pages(k_log, v_log)
    assert np.array_equal(cache.k.view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1), wk)
    assert np.array_equal(cache.v.view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1), wv)


def test_kv_append_out_of_range_page_dropped(cuda):
    import torch_spyre_amd as tsa

    cache = tsa.PagedKVCache(2, 1, 64, device=cuda)
    table = torch.tensor([[5]], dtype=torch.int32, device=cuda)  # no page 5
    tsa.kv_append(torch.ones((1, 1, 64), dtype=torch.float16, device=cuda),
                  torch.ones((1, 1, 64), dtype=torch.float16, device=cuda), cache.k, cache.v,
                  table, torch.tensor([3], dtype=torch.int32, device=cuda))
    torch.cuda.synchronize()
    assert torch.count_nonzero(cache.k) == 0 and torch.count_nonzero(cache.v) == 0


def test_append_then_attend_matches_oracle(cuda):
    """Append one token per sequence at position ctx, then attend over ctx+1
    (the long-context step, at a reduced context)."""
    import torch_spyre_amd as tsa

    B, Hq, Hkv, D = 4, 64, 8, 128
    ctx = [4095, 4096, 100, 63]
    cache, table, lens, q = make_case(cuda, B, Hq, Hkv, D, [c + 1 for c in ctx], SEED + 31)
    gg = torch.Generator(device=cuda).manual_seed(SEED + 32)
    k_new = torch.randn((B, Hkv, D), generator=gg, device=cuda).half()
    v_new = torch.randn((B, Hkv, D), generator=gg, device=cuda).half()
    pos = torch.tensor(ctx, dtype=torch.int32, device=cuda)
    tsa.kv_append(k_new, v_new, cache.k, cache.v, table.to(cuda), pos)
    out = run(cache, table, lens, q, cuda)
    ref = oracle_rows(cache, table, lens, q, list(range(B)), 1 / math.sqrt(D))
    assert_close(out, ref)
    # the appended token is the one the oracle saw
    tab = table.numpy()
    for b, p in enumerate(ctx):
        page = int(tab[b][p // 64])
        kd = cache.k[page].cpu().numpy()
        k_log, _ = OA.pages_to_logical(kd[None], cache.v[page].cpu().numpy()[None], 1, Hkv, D)
        assert np.array_equal(k_log[0][:, p % 64, :], k_new[b].cpu().numpy())


def test_config5_long_context_append_full_shape(cuda):
    """Batch 4, 64 q / 8 KV heads (g = 8), D 128: append the token at position
    131072 into its stick-layout page, then attend over 131073 tokens (2049
    pages, several chunks and the merge pass); every row against the oracle,
    LSE against fp64, and the token count exact (q = 0)."""
    import torch_spyre_amd as tsa

    B, Hq, Hkv, D, ctx = 4, 64, 8, 128, 131072
    cache, table, lens, q = make_case(cuda, B, Hq, Hkv, D, [ctx + 1] * B, SEED + 33, extra_pages=0)
    gg = torch.Generator(device=cuda).manual_seed(SEED + 34)
    k_new = torch.randn((B, Hkv, D), generator=gg, device=cuda).half()
    v_new = torch.randn((B, Hkv, D), generator=gg, device=cuda).half()
    pos = torch.full((B,), ctx, dtype=torch.int32, device=cuda)
    tsa.kv_append(k_new, v_new, cache.k, cache.v, table.to(cuda), pos)
    out, lse = run(cache, table, lens, q, cuda, max_context_len=ctx + 1, return_lse=True)
    rows = list(range(B))
    assert_close(out, oracle_rows(cache, table, lens, q, rows, 1 / math.sqrt(D)))
    lse64 = oracle_lse64(cache, table, lens, q, rows, 1 / math.sqrt(D))
    assert np.abs(lse.cpu().numpy() - lse64).max() <= 1e-4
    # q = 0 (closed form): every one of the 131073 tokens, the appended one
    # included, counted exactly once
    out0, lse0 = run(cache, table, lens, torch.zeros_like(q), cuda, max_context_len=ctx + 1, return_lse=True)
    assert_token_count_exact(out0, lse0, mean_v64(cache, table, lens, Hq, rows), lens, rows)
