"""GPU: the op layer as a caller of the reference's interface sees it -- every
``torch.ops.spyre.*`` op and ``aten::_scaled_dot_product_fused_attention_overrideable``
called through the dispatcher and checked against the oracle (bit-exact for
relayout, overwrite and kv_append; attention within |gpu - ref| <= 2e-3 +
1e-2 |ref| of CPU fp32 SDPA and LSE within 2e-3 of fp64), torch.library.opcheck
on each op, the F.scaled_dot_product_attention override, and a
torch.compile(fullgraph=True) decode step (append, then paged attention)."""

import math

import numpy as np
import pytest
import torch

from oracle import attention as OA
from oracle import kv as OK
from oracle import layout as OL
from oracle import relayout as OR
from tests.conftest import SEED

pytestmark = pytest.mark.gpu

ATOL, RTOL, LSE_ATOL = 2e-3, 1e-2, 2e-3


def assert_close(got, ref):
    got, ref = got.float().cpu(), torch.as_tensor(ref).float().cpu()
    assert got.shape == ref.shape and not torch.isnan(got).any()
    assert not torch.isnan(ref).any(), "NaN in the reference"
    err = (got - ref).abs()
    assert not (err > ATOL + RTOL * ref.abs()).any(), f"max abs err {err.max():.3e}"


def _bits(shape, seed, device):
    b = OR.random_finite_f16_bits(shape, seed)
    return b, torch.from_numpy(b.view(np.int16)).to(device).view(torch.float16)


def _raw(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _paged_case(cuda, B, Hq, Hkv, D, ctx, seed):
    import torch_spyre_amd as tsa

    n = [max(1, (c + 64) // 64) for c in ctx]  # room for one more token
    pool = sum(n) + 2
    perm = torch.randperm(pool, generator=torch.Generator().manual_seed(seed)).to(torch.int32)
    table = torch.full((B, max(n)), -1, dtype=torch.int32)
    k = 0
    for b, nb in enumerate(n):
        table[b, :nb] = perm[k:k + nb]
        k += nb
    g = torch.Generator(device=cuda).manual_seed(seed)
    cache = tsa.PagedKVCache(pool, Hkv, D, device=cuda, zero=False)
    cache.k.normal_(generator=g)
    cache.v.normal_(generator=g)
    q = torch.randn((B, Hq, D), generator=g, device=cuda).half()
    kn = torch.randn((B, Hkv, D), generator=g, device=cuda).half()
    vn = torch.randn((B, Hkv, D), generator=g, device=cuda).half()
    return cache, table.to(cuda), q, kn, vn


# --------------------------------------------------- every op vs the oracle --

def test_relayout_and_host_ops_vs_oracle(cuda):
    """spyre::to_device_layout, spyre::relayout (the explicit restickify) and
    spyre::from_device_layout on [200, 300] fp16, bit-exact."""
    size, st = [200, 300], [300, 1]
    bits, x = _bits(tuple(size), SEED, cuda)
    src = OL.stl_default(size)
    dst = OL.stl_init(size, st, "float16", [1, 0])
    dev = torch.ops.spyre.to_device_layout(x, src.device_size, src.stride_map)
    assert np.array_equal(_raw(dev).reshape(-1), OL.h2d(bits.reshape(-1), size, st, 0, src))
    moved = torch.ops.spyre.relayout(dev, size, st, src.device_size, src.stride_map, dst.device_size, dst.stride_map)
    want = OL.h2d(bits.reshape(-1), size, st, 0, dst)
    assert np.array_equal(_raw(moved).reshape(-1)[: want.size], want)
    back = torch.ops.spyre.from_device_layout(moved, dst.device_size, dst.stride_map, size)
    assert back.is_contiguous() and np.array_equal(_raw(back), bits)


def test_overwrite_ops_vs_oracle(cuda):
    """spyre::overwrite (in place) and spyre::overwrite_f (functional)."""
    ob, out = _bits((2, 8, 64, 128), SEED + 1, cuda)
    ib, inp = _bits((2, 8, 3, 128), SEED + 2, cuda)
    want = ob.copy()
    OK.overwrite(ib, want, [2], [61])
    res = torch.ops.spyre.overwrite_f(inp, out, [2], [61])
    assert np.array_equal(_raw(res), want) and np.array_equal(_raw(out), ob)
    torch.ops.spyre.overwrite(inp, out, [2], [61])
    assert np.array_equal(_raw(out), want)


def test_overwrite_f_in_compiled_loop(cuda):
    """tests/inductor/test_overwrite.py:208-241: a torch.compile'd loop of
    spyre::overwrite_f, one token per slot.  The result equals the oracle's
    overwrites bit for bit; inductor's reinplace pass (the registration of
    torch_spyre/_inductor/customops.py:333-335) turns every overwrite_f after
    the first (which reads the graph input, not mutated) into an in-place
    overwrite of that one copy, so the generated code copies the cache once
    instead of once per token."""
    from torch._inductor.utils import run_and_get_code

    slots = [3, 11, 7, 19]

    def scatter(cache, tokens):
        for i in range(len(slots)):
            cache = torch.ops.spyre.overwrite_f(tokens[i:i + 1], cache, [0], [slots[i]])
        return cache

    torch._dynamo.reset()
    cb, cache = _bits((32, 4, 64), SEED + 20, cuda)
    tb, tokens = _bits((4, 4, 64), SEED + 21, cuda)
    result, codes = run_and_get_code(torch.compile(scatter), cache, tokens)
    want = cb.copy()
    for i, s in enumerate(slots):
        OK.overwrite(tb[i:i + 1], want, [0], [s])
    assert np.array_equal(_raw(result), want)
    assert np.array_equal(_raw(cache), cb)  # the input is unchanged
    code = "\n".join(codes)
    # the first write reads the graph input, which is not mutated: one
    # overwrite_f (its one copy of the cache); every later one in place
    functional = code.count("torch.ops.spyre.overwrite_f.default(")
    assert functional <= 1, code
    assert code.count("torch.ops.spyre.overwrite.default(") == len(slots) - functional, code
    assert code.count("clone") + code.count(".copy_(") == 0, code


def test_kv_append_and_paged_decode_ops_vs_oracle(cuda):
    """spyre::kv_append then spyre::paged_decode_attention: the caches equal
    the oracle's append on logical pages (bit-exact), the attention its CPU
    fp32 SDPA over the gathered pages, and the LSE its fp64 logsumexp."""
    B, Hq, Hkv, D = 3, 16, 4, 128
    ctx = [700, 64, 4095]
    cache, table, q, kn, vn = _paged_case(cuda, B, Hq, Hkv, D, ctx, SEED + 3)
    P = cache.num_pages
    k_log, v_log = OA.pages_to_logical(_raw(cache.k), _raw(cache.v), P, Hkv, D)
    pos = torch.tensor(ctx, dtype=torch.int32, device=cuda)
    torch.ops.spyre.kv_append(kn, vn, cache.k, cache.v, table, pos)
    OK.append_token(k_log, v_log, _raw(kn), _raw(vn), table.cpu().numpy(), ctx)
    wk, wv = OA.logical_to_pages(k_log, v_log)
    assert np.array_equal(_raw(cache.k).reshape(-1), wk) and np.array_equal(_raw(cache.v).reshape(-1), wv)
    lens = pos + 1
    scale = 1 / math.sqrt(D)
    out, lse = torch.ops.spyre.paged_decode_attention(q, cache.k, cache.v, table, lens, scale, 512, 4096)
    kf = torch.from_numpy(k_log.view(np.float16)).float().numpy()
    vf = torch.from_numpy(v_log.view(np.float16)).float().numpy()
    ref = OA.paged_decode_reference(q.cpu().float(), kf, vf, table.cpu().numpy(), lens.cpu().numpy(), scale)
    assert_close(out, ref)
    for b in range(B):
        kb, vb = OA.gather_sequence(kf, vf, table.cpu().numpy()[b], int(lens[b]))
        _, l64 = OA.sdpa_decomposition_fp64(q[b].cpu().float().numpy()[None, :, None, :], kb[None], vb[None],
                                            scale=scale, return_lse=True)
        assert np.abs(lse[b].cpu().numpy() - l64.reshape(-1)).max() <= LSE_ATOL


def test_sdpa_fwd_op_vs_oracle(cuda):
    q = torch.randn((2, 8, 100, 64), generator=torch.Generator().manual_seed(SEED + 4)).half()
    k = torch.randn((2, 2, 150, 64), generator=torch.Generator().manual_seed(SEED + 5)).half()
    v = torch.randn((2, 2, 150, 64), generator=torch.Generator().manual_seed(SEED + 6)).half()
    out, lse = torch.ops.spyre.sdpa_fwd(q.to(cuda), k.to(cuda), v.to(cuda), None, True, None, True)
    assert out.shape == (2, 8, 100, 64) and out.stride() == (100 * 8 * 64, 64, 8 * 64, 1)
    assert_close(out, OA.sdpa_cpu_fp32(q, k, v, is_causal=True))
    _, l64 = OA.sdpa_decomposition_fp64(q, k, v, is_causal=True, return_lse=True)
    assert np.abs(lse.cpu().numpy() - l64).max() <= LSE_ATOL


@pytest.mark.parametrize("case", ["gqa_causal", "mha_bias"])
def test_aten_overrideable_op(cuda, case):
    """aten::_scaled_dot_product_fused_attention_overrideable on CUDA tensors
    runs this library's kernel and returns the reference's 9-tuple
    (torch_spyre/_inductor/decompositions.py:597-609)."""
    g = torch.Generator().manual_seed(SEED + 7)
    Hkv = 2 if case == "gqa_causal" else 8
    q = torch.randn((2, 8, 96, 128), generator=g).half()
    k = torch.randn((2, Hkv, 96, 128), generator=g).half()
    v = torch.randn((2, Hkv, 96, 128), generator=g).half()
    bias = None if case == "gqa_causal" else torch.randn((96, 96), generator=g).half()
    causal = case == "gqa_causal"
    r = torch.ops.aten._scaled_dot_product_fused_attention_overrideable(
        q.to(cuda), k.to(cuda), v.to(cuda), None if bias is None else bias.to(cuda), 0.0, causal, False,
        scale=0.1)
    assert len(r) == 9 and r[2] is None and r[3] is None and r[8] is None
    assert (r[4], r[5]) == (96, 96) and r[6].shape == (1,) and r[7].shape == (1,)
    out, lse = r[0], r[1]
    assert out.stride() == (96 * 8 * 128, 128, 8 * 128, 1)
    assert_close(out, OA.sdpa_cpu_fp32(q, k, v, attn_mask=bias, is_causal=causal, scale=0.1))
    _, l64 = OA.sdpa_decomposition_fp64(q, k, v, scale=0.1, attn_mask=None if bias is None else bias.numpy(),
                                        is_causal=causal, return_lse=True)
    assert np.abs(lse.cpu().numpy() - l64).max() <= LSE_ATOL


def test_sdpa_override_mode(cuda):
    """Inside sdpa_override, F.scaled_dot_product_attention on fp16 CUDA
    tensors runs this library's kernel (bit-identical to the direct call);
    calls it cannot serve (fp32) stay torch's."""
    import torch.nn.functional as F

    import torch_spyre_amd as tsa

    g = torch.Generator().manual_seed(SEED + 8)
    q = torch.randn((1, 8, 64, 64), generator=g).half().to(cuda)
    k = torch.randn((1, 4, 80, 64), generator=g).half().to(cuda)
    v = torch.randn((1, 4, 80, 64), generator=g).half().to(cuda)
    direct = tsa.scaled_dot_product_attention(q, k, v, is_causal=True, enable_gqa=True)
    with tsa.sdpa_override():
        got = F.scaled_dot_product_attention(q, k, v, is_causal=True, enable_gqa=True)
        f32 = F.scaled_dot_product_attention(q.float(), k.float(), v.float(), is_causal=True, enable_gqa=True)
    assert torch.equal(got.view(torch.int16), direct.view(torch.int16)) and got.stride() == direct.stride()
    assert f32.dtype == torch.float32
    assert_close(got, OA.sdpa_cpu_fp32(q.cpu(), k.cpu(), v.cpu(), is_causal=True))


def test_sdpa_override_leaves_other_shapes_to_torch(cuda):
    """Calls torch serves but this library does not -- a value head dim
    other than the query's, a key / value batch broadcast against the
    query's -- run torch's own SDPA inside sdpa_override (no error, torch's
    result)."""
    import torch.nn.functional as F

    import torch_spyre_amd as tsa

    g = torch.Generator().manual_seed(SEED + 12)
    q = torch.randn((2, 8, 16, 128), generator=g).half().to(cuda)
    k = torch.randn((2, 8, 40, 128), generator=g).half().to(cuda)
    v64 = torch.randn((2, 8, 40, 64), generator=g).half().to(cuda)
    k1 = torch.randn((1, 8, 40, 128), generator=g).half().to(cuda)
    v1 = torch.randn((1, 8, 40, 128), generator=g).half().to(cuda)
    for kk, vv in ((k, v64), (k1, v1)):
        want = F.scaled_dot_product_attention(q.float(), kk.float(), vv.float())
        with tsa.sdpa_override():
            got = F.scaled_dot_product_attention(q, kk, vv)
        assert got.shape == want.shape
        assert_close(got, want.cpu())


# ----------------------------------------------------------------- opcheck --

def _opcheck_cases(cuda):
    size = [130, 200]
    x = torch.randn(size, generator=torch.Generator().manual_seed(SEED + 9)).half().to(cuda)
    src = OL.stl_default(size)
    dst = OL.stl_init(size, [200, 1], "float16", [1, 0])
    dev = torch.ops.spyre.to_device_layout(x, src.device_size, src.stride_map)
    cache, table, q, kn, vn = _paged_case(cuda, 2, 8, 2, 64, [100, 300], SEED + 10)
    lens = torch.tensor([101, 301], dtype=torch.int32, device=cuda)
    pos = torch.tensor([100, 300], dtype=torch.int32, device=cuda)
    g = torch.Generator().manual_seed(SEED + 11)
    sq = torch.randn((1, 4, 40, 64), generator=g).half().to(cuda)
    sk = torch.randn((1, 2, 50, 64), generator=g).half().to(cuda)
    out = torch.zeros((2, 8, 64, 128), dtype=torch.float16, device=cuda)
    inp = torch.ones((2, 8, 1, 128), dtype=torch.float16, device=cuda)
    return {
        "to_device_layout": (torch.ops.spyre.to_device_layout, (x, src.device_size, src.stride_map)),
        "from_device_layout": (torch.ops.spyre.from_device_layout, (dev, src.device_size, src.stride_map, size)),
        "relayout": (torch.ops.spyre.relayout, (dev, size, [200, 1], src.device_size, src.stride_map,
                                                dst.device_size, dst.stride_map)),
        "overwrite": (torch.ops.spyre.overwrite, (inp, out, [2], [5])),
        "overwrite_f": (torch.ops.spyre.overwrite_f, (inp, out, [2], [7])),
        "copy_from_d2d": (torch.ops.spyre.copy_from_d2d, (x, torch.empty_like(x))),
        "kv_append": (torch.ops.spyre.kv_append, (kn, vn, cache.k, cache.v, table, pos)),
        "paged_decode_attention": (torch.ops.spyre.paged_decode_attention,
                                   (q, cache.k, cache.v, table, lens, 0.125, 512, 301)),
        "sdpa_fwd": (torch.ops.spyre.sdpa_fwd, (sq, sk, sk, None, False, None, True)),
    }


@pytest.mark.parametrize("name", ["to_device_layout", "from_device_layout", "relayout", "overwrite",
                                  "overwrite_f", "copy_from_d2d", "kv_append", "paged_decode_attention",
                                  "sdpa_fwd"])
def test_opcheck(cuda, name):
    op, args = _opcheck_cases(cuda)[name]
    torch.library.opcheck(op, args)


def test_opcheck_restickify(cuda):
    """spyre::restickify takes a Spyre tensor: its schema, autograd
    registration and fake kernel are checked by opcheck on a base tensor
    whose stick is on dim 0 and on a transposed view, so the default target
    moves the stick in both; the traced form (opcheck's AOT-dispatch check
    compares results with elementwise ops a Spyre tensor does not serve) is
    compiled with aot_eager here and compared bit for bit with eager.  The
    plain-tensor kernel refuses."""
    import torch_spyre_amd as tsa

    x = torch.randn((192, 256), generator=torch.Generator().manual_seed(SEED + 12)).half()
    a = tsa.to_device_layout(x, tsa.transpose_restick_layout(192, 256))
    b = tsa.to_device_layout(x).t()
    r = torch.ops.spyre.restickify(a)
    assert r.device_tensor_layout() == tsa.SpyreTensorLayout([192, 256], torch.float16)
    assert torch.equal(r.cpu(), x)
    checks = ("test_schema", "test_autograd_registration", "test_faketensor")
    for t in (a, b):
        torch.library.opcheck(torch.ops.spyre.restickify, (t,), test_utils=checks)
        traced = torch.compile(lambda v: torch.ops.spyre.restickify(v), backend="aot_eager", fullgraph=True)(t)
        eager = torch.ops.spyre.restickify(t)
        assert traced.device_tensor_layout() == eager.device_tensor_layout()
        assert traced.shape == eager.shape and traced.stride() == eager.stride()
        assert torch.equal(tsa.device_buffer(traced).view(torch.int16), tsa.device_buffer(eager).view(torch.int16))
        assert torch.equal(traced.cpu(), t.cpu())
    with pytest.raises(TypeError, match="SpyreTensor"):
        torch.ops.spyre.restickify(torch.zeros(4, 4, dtype=torch.float16, device=cuda))


# ------------------------------------------------------------ torch.compile --

def test_compiled_decode_step(cuda):
    """torch.compile(fullgraph=True) of a decode step: append one token per
    sequence into the paged cache, then attend over context + 1.  Equal to
    the eager step bit for bit (caches and output)."""
    B, Hq, Hkv, D = 4, 32, 8, 128
    ctx = [1000, 64, 3000, 129]
    scale = 1 / math.sqrt(D)

    def step(kn, vn, k_cache, v_cache, table, pos, q, lens):
        torch.ops.spyre.kv_append(kn, vn, k_cache, v_cache, table, pos)
        return torch.ops.spyre.paged_decode_attention(q, k_cache, v_cache, table, lens, scale, 512, 3001)

    compiled = torch.compile(step, fullgraph=True)
    outs = []
    for fn in (step, compiled):
        cache, table, q, kn, vn = _paged_case(cuda, B, Hq, Hkv, D, ctx, SEED + 13)
        pos = torch.tensor(ctx, dtype=torch.int32, device=cuda)
        out, lse = fn(kn, vn, cache.k, cache.v, table, pos, q, pos + 1)
        torch.cuda.synchronize()
        outs.append((_raw(out), lse.cpu(), _raw(cache.k), _raw(cache.v)))
    (o1, l1, k1, v1), (o2, l2, k2, v2) = outs
    assert np.array_equal(o1, o2) and torch.equal(l1, l2)
    assert np.array_equal(k1, k2) and np.array_equal(v1, v2)
