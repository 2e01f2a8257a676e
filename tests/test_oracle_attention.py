"""CPU: pin the attention oracle (decomposition restatement, CPU SDPA path,
page gathering) to torch's SDPA and to closed-form cases."""

import math

import numpy as np
import pytest
import torch

from oracle import attention as OA
from oracle import layout as OL
from tests.conftest import SEED


def _rand(shape, seed):
    return torch.randn(shape, generator=torch.Generator().manual_seed(seed), dtype=torch.float64)


@pytest.mark.parametrize("B,Hq,Hkv,S,D", [(1, 8, 8, 512, 64), (2, 32, 8, 100, 128), (3, 16, 2, 7, 64), (1, 4, 1, 1, 128)])
def test_decomposition_matches_torch_sdpa(B, Hq, Hkv, S, D):
    q, k, v = _rand((B, Hq, 1, D), 1), _rand((B, Hkv, S, D), 2), _rand((B, Hkv, S, D), 3)
    ref = torch.nn.functional.scaled_dot_product_attention(q, k, v, enable_gqa=Hq != Hkv)
    got = OA.sdpa_decomposition_fp64(q.numpy(), k.numpy(), v.numpy())
    assert np.allclose(got, ref.numpy(), atol=1e-12, rtol=1e-10)
    fp32 = OA.sdpa_cpu_fp32(q, k, v)
    assert np.allclose(fp32.numpy(), got, atol=1e-5, rtol=1e-4)


def test_scale_is_applied_once():
    """sqrt(scale) on q and on k equals scale on the scores; a scale applied
    to q only would not match."""
    q, k, v = _rand((1, 2, 1, 64), 4), _rand((1, 2, 9, 64), 5), _rand((1, 2, 9, 64), 6)
    ref = torch.nn.functional.scaled_dot_product_attention(q, k, v, scale=0.3)
    assert np.allclose(OA.sdpa_decomposition_fp64(q, k, v, 0.3), ref.numpy(), atol=1e-12)
    wrong = torch.nn.functional.scaled_dot_product_attention(q * math.sqrt(0.3), k, v, scale=1.0)
    assert not np.allclose(wrong.numpy(), ref.numpy(), atol=1e-3)


def test_single_key_returns_its_value():
    q, k, v = _rand((2, 4, 1, 64), 7), _rand((2, 2, 1, 64), 8), _rand((2, 2, 1, 64), 9)
    got = OA.sdpa_decomposition_fp64(q, k, v)
    assert np.allclose(got, np.repeat(v.numpy(), 2, axis=1))


def test_identical_keys_average_values():
    q, v = _rand((1, 3, 1, 64), 10), _rand((1, 3, 20, 64), 11)
    k = _rand((1, 3, 1, 64), 12).expand(1, 3, 20, 64)
    got = OA.sdpa_decomposition_fp64(q, k, v)
    assert np.allclose(got, v.numpy().mean(axis=2, keepdims=True))


def test_dominant_key_limit():
    """One key with a much larger score takes all the weight."""
    q = torch.zeros((1, 1, 1, 64), dtype=torch.float64)
    q[..., 0] = 1.0
    k = torch.zeros((1, 1, 5, 64), dtype=torch.float64)
    k[0, 0, 3, 0] = 400.0
    v = _rand((1, 1, 5, 64), 13)
    got = OA.sdpa_decomposition_fp64(q, k, v)
    assert np.allclose(got[0, 0, 0], v[0, 0, 3].numpy())


def test_gqa_head_mapping_is_h_div_g():
    """q head h reads KV head h // g (expand + flatten), not h % Hkv."""
    q, k, v = _rand((1, 8, 1, 16), 14), _rand((1, 2, 6, 16), 15), _rand((1, 2, 6, 16), 16)
    got = OA.sdpa_decomposition_fp64(q, k, v)
    kk = k.repeat_interleave(4, dim=1)
    vv = v.repeat_interleave(4, dim=1)
    ref = torch.nn.functional.scaled_dot_product_attention(q, kk, vv)
    assert np.allclose(got, ref.numpy())
    kw = k.repeat(1, 4, 1, 1)  # the planted mistake: head h -> h % Hkv
    vw = v.repeat(1, 4, 1, 1)
    wrong = torch.nn.functional.scaled_dot_product_attention(q, kw, vw)
    assert not np.allclose(got, wrong.numpy())


def test_empty_context_is_zero_like_torch():
    q = _rand((1, 4, 1, 8), 17)
    k = torch.empty((1, 2, 0, 8), dtype=torch.float64)
    ref = torch.nn.functional.scaled_dot_product_attention(q, k, k, enable_gqa=True)
    assert np.array_equal(OA.sdpa_decomposition_fp64(q, k, k), ref.numpy())
    assert not ref.abs().sum()


def test_page_layouts_round_trip_and_closed_form():
    P, Hkv, D = 3, 2, 128
    rng = np.random.default_rng(SEED)
    k_log = rng.integers(0, 1 << 15, (P, Hkv, 64, D)).astype(np.uint16)
    v_log = rng.integers(0, 1 << 15, (P, Hkv, 64, D)).astype(np.uint16)
    kd, vd = OA.logical_to_pages(k_log, v_log)
    # K: sticks along D -> [P, Hkv, D/64, 64 tok, 64]; V: sticks along tokens -> [P, Hkv, D, 64 tok]
    assert np.array_equal(kd.reshape(P, Hkv, D // 64, 64, 64),
                          k_log.reshape(P, Hkv, 64, D // 64, 64).transpose(0, 1, 3, 2, 4))
    assert np.array_equal(vd.reshape(P, Hkv, D, 64), v_log.transpose(0, 1, 3, 2))
    k2, v2 = OA.pages_to_logical(kd, vd, P, Hkv, D)
    assert np.array_equal(k2, k_log) and np.array_equal(v2, v_log)


def test_paged_reference_equals_dense_sdpa():
    """Gathering permuted pages by the block table rebuilds the dense sequence."""
    Hkv, D, ctx = 2, 64, 150
    rng = np.random.default_rng(3)
    dense_k = rng.standard_normal((Hkv, 192, D)).astype(np.float32)
    dense_v = rng.standard_normal((Hkv, 192, D)).astype(np.float32)
    perm = np.array([2, 0, 1])
    k_log = np.empty((3, Hkv, 64, D), np.float32)
    v_log = np.empty((3, Hkv, 64, D), np.float32)
    for i, p in enumerate(perm):
        k_log[p] = dense_k[:, 64 * i:64 * i + 64]
        v_log[p] = dense_v[:, 64 * i:64 * i + 64]
    q = torch.from_numpy(rng.standard_normal((1, 8, D)).astype(np.float32))
    got = OA.paged_decode_reference(q, k_log, v_log, [perm], [ctx], 0.125)
    ref = torch.nn.functional.scaled_dot_product_attention(
        q[:, :, None, :], torch.from_numpy(dense_k[None, :, :ctx]), torch.from_numpy(dense_v[None, :, :ctx]),
        scale=0.125, enable_gqa=True)
    assert torch.allclose(got, ref[:, :, 0, :], atol=1e-6)


def test_page_layout_descriptors_follow_stl_rules():
    """The oracle's page layouts are valid SpyreTensorLayouts: their DMA
    plans are single loop nests covering every element once."""
    P, Hkv, D = 2, 3, 128
    sizes = [P, Hkv, 64, D]
    st = OL.contiguous_strides(sizes)
    for lay in (OA.k_page_layout(P, Hkv, D), OA.v_page_layout(P, Hkv, D)):
        infos = OL.device_stride_infos(sizes, st, 0, lay.device_size, lay.stride_map, True, st)
        assert len(infos) == 1 and int(np.prod(infos[0].size)) == P * Hkv * 64 * D


# ---- prefill (Sq > 1): causal, masks, logsumexp ----

@pytest.mark.parametrize("B,Hq,Hkv,Sq,Sk,D", [(2, 4, 4, 9, 9, 16), (1, 8, 2, 17, 23, 32), (2, 6, 3, 5, 12, 8)])
def test_prefill_decomposition_matches_torch(B, Hq, Hkv, Sq, Sk, D):
    q, k, v = _rand((B, Hq, Sq, D), 20), _rand((B, Hkv, Sk, D), 21), _rand((B, Hkv, Sk, D), 22)
    gqa = Hq != Hkv
    for causal in (False, True):
        ref = torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=causal, enable_gqa=gqa)
        got = OA.sdpa_decomposition_fp64(q, k, v, is_causal=causal)
        assert np.allclose(got, ref.numpy(), atol=1e-12, rtol=1e-10)
    mask = _rand((Sq, Sk), 23)
    ref = torch.nn.functional.scaled_dot_product_attention(q, k, v, attn_mask=mask, enable_gqa=gqa)
    assert np.allclose(OA.sdpa_decomposition_fp64(q, k, v, attn_mask=mask.numpy()), ref.numpy(), atol=1e-12)
    assert np.allclose(OA.sdpa_cpu_fp32(q, k, v, attn_mask=mask).numpy(), ref.numpy(), atol=1e-5)


def test_causal_equals_explicit_triu_mask_and_bool_mask():
    """The reference's test pairs is_causal=True with the mask triu(-inf, 1)
    (tests/inductor/test_inductor_ops.py:2598-2626); a boolean tril mask is
    the same bias after conversion.  Excluding the diagonal (triu(-inf, 0))
    is the planted mistake and must differ."""
    q, k, v = _rand((1, 2, 12, 16), 24), _rand((1, 2, 12, 16), 25), _rand((1, 2, 12, 16), 26)
    causal = OA.sdpa_decomposition_fp64(q, k, v, is_causal=True)
    tri = np.triu(np.full((12, 12), -np.inf), 1)
    assert np.array_equal(causal, OA.sdpa_decomposition_fp64(q, k, v, attn_mask=tri))
    keep = np.tril(np.ones((12, 12), bool))
    assert np.array_equal(causal, OA.sdpa_decomposition_fp64(q, k, v, attn_mask=keep))
    wrong = np.triu(np.full((12, 12), -np.inf), 0)
    wrong[0, 0] = 0.0  # keep row 0 defined
    assert not np.allclose(causal, OA.sdpa_decomposition_fp64(q, k, v, attn_mask=wrong))


def test_causal_closed_forms():
    """Row 0 of a causal attention sees key 0 only: out = v[0], lse =
    scale * q0.k0; the last row of a square causal attention is the
    unmasked attention of that row."""
    q, k, v = _rand((1, 1, 6, 8), 27), _rand((1, 1, 6, 8), 28), _rand((1, 1, 6, 8), 29)
    out, lse = OA.sdpa_decomposition_fp64(q, k, v, scale=0.5, is_causal=True, return_lse=True)
    assert np.allclose(out[0, 0, 0], v[0, 0, 0].numpy())
    assert np.isclose(lse[0, 0, 0], 0.5 * float(q[0, 0, 0] @ k[0, 0, 0]))
    full = OA.sdpa_decomposition_fp64(q, k, v, scale=0.5)
    assert np.allclose(out[0, 0, -1], full[0, 0, -1])


def test_lse_closed_forms():
    """Identical keys: lse = s + log(n); and lse matches a direct fp64 logsumexp."""
    q = _rand((1, 1, 3, 8), 30)
    k = _rand((1, 1, 1, 8), 31).expand(1, 1, 7, 8)
    v = _rand((1, 1, 7, 8), 32)
    _, lse = OA.sdpa_decomposition_fp64(q, k, v, scale=0.25, return_lse=True)
    s = 0.25 * (q[0, 0] @ k[0, 0, 0]).numpy()
    assert np.allclose(lse[0, 0], s + np.log(7))
    mask = _rand((3, 7), 33)
    _, lse2 = OA.sdpa_decomposition_fp64(q, _rand((1, 1, 7, 8), 34), v, attn_mask=mask.numpy(), return_lse=True)
    kk = _rand((1, 1, 7, 8), 34)[0, 0].numpy()
    sc = (q[0, 0].numpy() @ kk.T) / math.sqrt(8) + mask.numpy()
    assert np.allclose(lse2[0, 0], np.log(np.exp(sc).sum(-1)))


def test_fully_masked_row_nan_in_decomposition_zero_in_cpu_sdpa():
    q, k, v = _rand((1, 1, 3, 8), 35), _rand((1, 1, 4, 8), 36), _rand((1, 1, 4, 8), 37)
    m = np.zeros((3, 4))
    m[1] = -np.inf
    assert np.isnan(OA.sdpa_decomposition_fp64(q, k, v, attn_mask=m)[0, 0, 1]).all()
    cpu = OA.sdpa_cpu_fp32(q, k, v, attn_mask=torch.from_numpy(m))
    assert not cpu[0, 0, 1].any()


@pytest.mark.parametrize("Hq,Hkv,S,D,scale", [(8, 8, 300, 64, None), (32, 8, 77, 128, 0.3), (16, 2, 1, 128, 2.0)])
def test_decode_lse_equals_decomposition_lse(Hq, Hkv, S, D, scale):
    """The lean decode LSE equals the full decomposition's logsumexp; a
    group mapping of h % Hkv (the plausible mistake) does not."""
    q, k, v = _rand((1, Hq, 1, D), 30), _rand((1, Hkv, S, D), 31), _rand((1, Hkv, S, D), 32)
    _, want = OA.sdpa_decomposition_fp64(q.numpy(), k.numpy(), v.numpy(), scale=scale, return_lse=True)
    got = OA.decode_lse_fp64(q.numpy()[0, :, 0], k.numpy()[0], scale=scale)
    assert np.allclose(got, want.reshape(-1), atol=1e-12, rtol=0)
    if Hkv not in (1, Hq):
        kk = k.numpy()[0][np.arange(Hq) % Hkv]  # [Hq, S, D], head h -> h % Hkv
        wrong = OA.decode_lse_fp64(q.numpy()[0, :, 0], kk, scale=scale)
        assert not np.allclose(wrong, want.reshape(-1), atol=1e-6)


@pytest.mark.parametrize("causal", [False, True])
def test_negative_scale_is_the_scale_on_negated_queries(causal):
    """The decomposition takes sqrt(scale), so a negative scale is pinned
    through the identity scale (q k^T) = |scale| ((-q) k^T): the fp64
    restatement on -q with |scale| equals torch's fp64 SDPA with the negative
    scale, and its logsumexp equals scipy's logsumexp of the scaled scores
    (the row max of the -q scores, not of the +q ones, is what it keeps)."""
    from scipy.special import logsumexp

    s = 0.2
    q, k, v = _rand((1, 2, 6, 64), 60), _rand((1, 2, 9, 64), 61), _rand((1, 2, 9, 64), 62)
    # torch's is_causal path gives NaN under a negative scale; its mask path
    # with the top-left lower triangle (is_causal's meaning) does not
    tril = torch.ones(6, 9, dtype=torch.bool).tril() if causal else None
    ref = torch.nn.functional.scaled_dot_product_attention(q, k, v, scale=-s, attn_mask=tril)
    got, lse = OA.sdpa_decomposition_fp64(-q.numpy(), k.numpy(), v.numpy(), scale=s, is_causal=causal,
                                          return_lse=True)
    assert np.allclose(got, ref.numpy(), atol=1e-12, rtol=1e-10)
    scores = -s * (q.numpy() @ np.swapaxes(k.numpy(), -1, -2))
    if causal:
        scores = scores + np.triu(np.full(scores.shape[-2:], -np.inf), 1)
    assert np.allclose(lse, logsumexp(scores, axis=-1), atol=1e-12, rtol=0)
    _, lse_pos = OA.sdpa_decomposition_fp64(q.numpy(), k.numpy(), v.numpy(), scale=s, is_causal=causal,
                                            return_lse=True)
    assert not np.allclose(lse_pos, lse, atol=1e-3)
    if not causal:  # the decode LSE applies the scale once, sign included
        for i in range(6):
            d = OA.decode_lse_fp64(q.numpy()[0, :, i], k.numpy()[0], scale=-s)
            assert np.allclose(d, lse[0, :, i], atol=1e-12, rtol=0)
    # the fp32 CPU path the GPU tests compare against: finite, and equal to
    # the positive scale on -q through torch's own is_causal path
    f32 = OA.sdpa_cpu_fp32(q.float(), k.float(), v.float(), scale=-s, is_causal=causal)
    want = torch.nn.functional.scaled_dot_product_attention(-q.float(), k.float(), v.float(), scale=s,
                                                            is_causal=causal)
    assert not torch.isnan(f32).any()
    assert torch.allclose(f32, want, atol=1e-6, rtol=1e-5)


def test_zero_scale_causal_averages_the_visible_values():
    """Scale 0 weighs every visible key alike: causal row i is the mean of
    v[0 .. i] (torch's own is_causal path gives NaN at scale 0)."""
    q, k, v = _rand((1, 2, 5, 64), 63), _rand((1, 2, 8, 64), 64), _rand((1, 2, 8, 64), 65)
    got = OA.sdpa_cpu_fp32(q.float(), k.float(), v.float(), scale=0.0, is_causal=True)
    want = torch.cumsum(v, dim=2)[:, :, :5] / torch.arange(1, 6, dtype=torch.float64)[:, None]
    assert torch.allclose(got.double(), want, atol=1e-6)
    _, lse = OA.sdpa_decomposition_fp64(q, k, v, scale=0.0, is_causal=True, return_lse=True)
    assert np.allclose(lse, np.log(np.arange(1, 6)), atol=1e-12)
