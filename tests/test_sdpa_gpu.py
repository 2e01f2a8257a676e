"""GPU parity of the SDPA forward kernel (prefill, causal, masks, GQA,
logsumexp) against the oracle: torch's CPU eager SDPA in fp32 (the
reference's compare path) and the fp64 restatement of the reference's
decomposition.

Bar: fp16 outputs within |gpu - ref| <= 2e-3 + 1e-2 |ref| elementwise; LSE
within 2e-3 absolute of the fp64 logsumexp.
"""

import math

import numpy as np
import pytest
import torch

from oracle import attention as OA
from tests.conftest import SEED

pytestmark = pytest.mark.gpu

ATOL = 2e-3
RTOL = 1e-2
LSE_ATOL = 2e-3


def assert_close(got, ref):
    got = got.float().cpu()
    ref = torch.as_tensor(ref).float().cpu()
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert not torch.isnan(got).any(), "NaN in output"
    assert not torch.isnan(ref).any(), "NaN in the reference"
    err = (got - ref).abs()
    bad = err > ATOL + RTOL * ref.abs()
    assert not bad.any(), f"{int(bad.sum())} elements out of tolerance; max abs err {err.max():.3e}"


def randn(shape, seed, dtype=torch.float16):
    return torch.randn(shape, generator=torch.Generator().manual_seed(seed), dtype=torch.float32).to(dtype)


def ref_case(B, Sq, Skv, Hq, Hkv, D, seed):
    """q/k/v as the reference's test builds them: [B, S, H, D] tensors viewed
    as [B, H, S, D] (tests/inductor/test_inductor_ops.py:2576-2650)."""
    q = randn((B, Sq, Hq, D), seed).transpose(1, 2)
    k = randn((B, Skv, Hkv, D), seed + 1).transpose(1, 2)
    v = randn((B, Skv, Hkv, D), seed + 2).transpose(1, 2)
    return q, k, v


def run(cuda, q, k, v, **kw):
    import torch_spyre_amd as tsa

    mask = kw.pop("attn_mask", None)
    if mask is not None:
        mask = mask.to(cuda)
    return tsa.scaled_dot_product_attention(q.to(cuda), k.to(cuda), v.to(cuda), attn_mask=mask, **kw)


# The reference's prefill parameter sets (tests/inductor/test_inductor_ops.py:2576-2650):
# q/k/v (2, 256, H, 128) fp16 transposed to (2, H, 256, 128).
REF_SETS = {
    "mha_prefill": (32, dict()),
    "mha_prefill_causal": (32, dict(is_causal=True)),
    "mha_prefill_mask": (32, dict(attn_mask=torch.triu(torch.ones((256, 256), dtype=torch.float16) * -float("inf"),
                                                      diagonal=1))),
    "gqa_prefill": (8, dict(enable_gqa=True)),
    "gqa_prefill_causal": (8, dict(is_causal=True, enable_gqa=True)),
}


@pytest.mark.parametrize("name", list(REF_SETS))
def test_reference_prefill_sets(cuda, name):
    Hkv, kw = REF_SETS[name]
    q, k, v = ref_case(2, 256, 256, 32, Hkv, 128, SEED + len(name))
    out, lse = run(cuda, q, k, v, return_lse=True, **kw)
    mask = kw.get("attn_mask")
    causal = kw.get("is_causal", False)
    ref = OA.sdpa_cpu_fp32(q, k, v, attn_mask=mask, is_causal=causal)
    assert_close(out, ref)
    ref64, lse64 = OA.sdpa_decomposition_fp64(q, k, v, attn_mask=None if mask is None else mask.numpy(),
                                              is_causal=causal, return_lse=True)
    assert_close(out, ref64)
    assert np.allclose(lse.cpu().numpy(), lse64, atol=LSE_ATOL, rtol=0)
    # the result has the strides of a contiguous [B, S, H, D] tensor (the reference's API promise)
    assert out.shape == (2, 32, 256, 128) and out.stride() == (256 * 32 * 128, 128, 32 * 128, 1)


@pytest.mark.parametrize("Sq,Skv", [(1, 1), (1, 300), (37, 100), (100, 37), (64, 64), (65, 129), (200, 513)])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("causal", [False, True])
def test_ragged_lengths(cuda, Sq, Skv, D, causal):
    q = randn((2, 4, Sq, D), SEED + Sq)
    k = randn((2, 2, Skv, D), SEED + Skv)
    v = randn((2, 2, Skv, D), SEED + Skv + 1)
    out, lse = run(cuda, q, k, v, is_causal=causal, enable_gqa=True, return_lse=True)
    assert_close(out, OA.sdpa_cpu_fp32(q, k, v, is_causal=causal))
    _, lse64 = OA.sdpa_decomposition_fp64(q, k, v, is_causal=causal, return_lse=True)
    assert np.allclose(lse.cpu().numpy(), lse64, atol=LSE_ATOL, rtol=0)


@pytest.mark.parametrize("g", [1, 2, 4, 8, 16])
def test_gqa_groups(cuda, g):
    q = randn((1, 2 * g, 70, 128), SEED + g)
    k = randn((1, 2, 90, 128), SEED + g + 1)
    v = randn((1, 2, 90, 128), SEED + g + 2)
    assert_close(run(cuda, q, k, v, enable_gqa=True), OA.sdpa_cpu_fp32(q, k, v))


@pytest.mark.parametrize("Sq,Skv,causal", [(1, 300, False), (5, 300, False), (33, 70, True), (64, 64, True)])
def test_gqa_heads_packed_into_rows(cuda, Sq, Skv, causal):
    """Short query runs without a mask on a grid of 512 (sequence, KV head)
    pairs: the 4 q heads of a KV head share one block's rows (row = query x 4
    + head), so decode reads each K / V tile once for the group."""
    q = randn((64, 32, Sq, 128), SEED + 50 + Sq)
    k, v = randn((64, 8, Skv, 128), SEED + 51), randn((64, 8, Skv, 128), SEED + 52)
    out, lse = run(cuda, q, k, v, is_causal=causal, enable_gqa=True, return_lse=True)
    assert_close(out, OA.sdpa_cpu_fp32(q, k, v, is_causal=causal))
    _, lse64 = OA.sdpa_decomposition_fp64(q, k, v, is_causal=causal, return_lse=True)
    assert np.allclose(lse.cpu().numpy(), lse64, atol=LSE_ATOL, rtol=0)


@pytest.mark.parametrize("B,Hq,Sq,Skv,causal", [(16, 64, 1, 512, False), (16, 64, 1, 512, True),
                                                (8, 64, 4, 300, False), (8, 64, 4, 300, True)])
def test_gqa_heads_partly_packed(cuda, B, Hq, Sq, Skv, causal):
    """Grids where only some of a KV head's 8 q heads share a block (on a
    256-CU device: 4 per block at B 16 / Sq 1, 2 per block at B 8 / Sq 4):
    every q head must be computed, each by the block holding its group."""
    q = randn((B, Hq, Sq, 128), SEED + 60 + B)
    k, v = randn((B, 8, Skv, 128), SEED + 61), randn((B, 8, Skv, 128), SEED + 62)
    out, lse = run(cuda, q, k, v, is_causal=causal, enable_gqa=True, return_lse=True)
    assert_close(out, OA.sdpa_cpu_fp32(q, k, v, is_causal=causal))
    _, lse64 = OA.sdpa_decomposition_fp64(q, k, v, is_causal=causal, return_lse=True)
    assert np.allclose(lse.cpu().numpy(), lse64, atol=LSE_ATOL, rtol=0)


def test_key_split_many_runs(cuda):
    """Decode over 16484 keys with 1 sequence and 8 KV heads: the key split
    runs 29 blocks per row (more than the merge pass loads at a time, the
    last group ragged); out against CPU fp32, LSE against fp64."""
    q = randn((1, 32, 1, 128), SEED + 70)
    k, v = randn((1, 8, 16484, 128), SEED + 71), randn((1, 8, 16484, 128), SEED + 72)
    out, lse = run(cuda, q, k, v, enable_gqa=True, return_lse=True)
    assert_close(out, OA.sdpa_cpu_fp32(q, k, v))
    _, lse64 = OA.sdpa_decomposition_fp64(q, k, v, return_lse=True)
    err = np.abs(lse.cpu().numpy() - lse64).max()
    assert err <= LSE_ATOL, err
    # every key counted once: q = 0 makes every score 0, so LSE = ln(Skv)
    # exactly up to fp32 rounding (a lost 356-key split moves it by 0.022,
    # one lost key by 6e-5)
    out0, lse0 = run(cuda, torch.zeros_like(q), k, v, enable_gqa=True, return_lse=True)
    assert np.abs(lse0.cpu().numpy() - math.log(16484)).max() <= 4e-6
    assert_close(out0, v.float().mean(dim=2, keepdim=True).repeat_interleave(4, dim=1))


def test_operand_views_copied(cuda):
    """Operands torch counts as contiguous but the kernel cannot read as they
    lie (an odd stride on a size-1 dim; a storage offset that is not 16-byte
    aligned) are copied, not refused."""
    q = randn((2, 4, 1, 64), SEED + 80)
    k, v = randn((2, 4, 40, 64), SEED + 81), randn((2, 4, 40, 64), SEED + 82)
    q_odd = torch.as_strided(q.to(cuda), (2, 4, 1, 64), (256, 64, 3, 1))
    assert q_odd.is_contiguous()
    flat = torch.empty(k.numel() + 1, dtype=torch.float16, device=cuda)
    k_off = flat[1:].view(k.shape)
    k_off.copy_(k.to(cuda))
    assert k_off.is_contiguous() and k_off.data_ptr() % 16 != 0
    out = run(cuda, q_odd, k_off, v)
    assert_close(out, OA.sdpa_cpu_fp32(q, k, v))


@pytest.mark.parametrize("kind", ["f16", "f32", "bool"])
@pytest.mark.parametrize("shape", ["qk", "b1qk", "1h1k"])
def test_masks_broadcast(cuda, kind, shape):
    """Additive fp16 / fp32 and boolean masks, broadcast from [Sq, Skv],
    [B, 1, Sq, Skv] and [1, Hq, 1, Skv] (a padding mask)."""
    B, Hq, Sq, Skv = 2, 4, 50, 77
    q, k, v = randn((B, Hq, Sq, 64), SEED + 1), randn((B, Hq, Skv, 64), SEED + 2), randn((B, Hq, Skv, 64), SEED + 3)
    dims = {"qk": (Sq, Skv), "b1qk": (B, 1, Sq, Skv), "1h1k": (1, Hq, 1, Skv)}[shape]
    g = torch.Generator().manual_seed(SEED + 4)
    if kind == "bool":
        mask = torch.rand(dims, generator=g) > 0.3
        mask[..., 0] = True  # no fully masked row here
    else:
        mask = (torch.randn(dims, generator=g) * 2).to(torch.float16 if kind == "f16" else torch.float32)
    out = run(cuda, q, k, v, attn_mask=mask)
    assert_close(out, OA.sdpa_cpu_fp32(q, k, v, attn_mask=mask))


def _mask(kind, dims, seed):
    g = torch.Generator().manual_seed(seed)
    if kind == "bool":
        m = torch.rand(dims, generator=g) > 0.3
        m[..., 0] = True  # no fully masked row here
        return m
    return (torch.randn(dims, generator=g) * 2).to(torch.float16)


@pytest.mark.parametrize("kind", ["f16", "bool"])
@pytest.mark.parametrize("shape", ["qk", "b1qk", "1h1k", "bhqk"])
@pytest.mark.parametrize("D", [64, 128])
def test_masks_staged_in_lds(cuda, kind, shape, D):
    """fp16 and boolean masks whose rows are whole 16-byte units (Skv a
    multiple of 16) are staged block by block beside K and V: ragged Sq,
    a last step of 32 keys, GQA, every broadcast form."""
    B, Hq, Hkv, Sq, Skv = 2, 8, 2, 100, 160
    q = randn((B, Hq, Sq, D), SEED + 11)
    k, v = randn((B, Hkv, Skv, D), SEED + 12), randn((B, Hkv, Skv, D), SEED + 13)
    dims = {"qk": (Sq, Skv), "b1qk": (B, 1, Sq, Skv), "1h1k": (1, Hq, 1, Skv), "bhqk": (B, Hq, Sq, Skv)}[shape]
    mask = _mask(kind, dims, SEED + 14)
    out = run(cuda, q, k, v, attn_mask=mask, enable_gqa=True)
    assert_close(out, OA.sdpa_cpu_fp32(q, k, v, attn_mask=mask))


@pytest.mark.parametrize("kind", ["f16", "bool"])
@pytest.mark.parametrize("Skv", [96, 100])
def test_staged_mask_ignores_bytes_past_skv(cuda, kind, Skv):
    """A mask that is a view of wider rows (112 elements): the bytes past Skv
    in each row (NaN for fp16, keep for bool) belong to no key and change
    nothing.  Skv 100: rows end inside a 16-byte unit, so the last row's
    last keys must still count (regression: staged as it lay, that unit
    arrived as zeros).  A large scale (|scale log2 e| > 1) takes the
    unscaled-score form."""
    Sq, D, W = 70, 128, 112
    q, k, v = randn((1, 4, Sq, D), SEED + 15), randn((1, 4, Skv, D), SEED + 16), randn((1, 4, Skv, D), SEED + 17)
    wide = _mask(kind, (Sq, W), SEED + 18)
    wide[:, Skv:] = True if kind == "bool" else float("nan")
    mask = wide.to(cuda)[:, :Skv]  # sliced on the device, so its rows keep their stride
    assert mask.stride() == (W, 1)
    for scale in (None, 2.0):
        out = run(cuda, q, k, v, attn_mask=mask, scale=scale)
        assert_close(out, OA.sdpa_cpu_fp32(q, k, v, attn_mask=mask.cpu().contiguous(), scale=scale))


@pytest.mark.parametrize("kind", ["f16", "bool"])
def test_staged_mask_fully_masked_rows(cuda, kind):
    """Rows with every key masked (a whole wavefront's block, and single
    rows) give zeros and a -inf logsumexp through the staged path too."""
    Sq, Skv = 80, 128
    q, k, v = randn((1, 2, Sq, 64), SEED + 19), randn((1, 2, Skv, 64), SEED + 20), randn((1, 2, Skv, 64), SEED + 21)
    mask = _mask(kind, (Sq, Skv), SEED + 22)
    dead = [3, *range(32, 64), 79]  # rows 32 .. 63: one wavefront's whole block
    mask[dead] = False if kind == "bool" else -float("inf")
    out, lse = run(cuda, q, k, v, attn_mask=mask, return_lse=True)
    assert_close(out, OA.sdpa_cpu_fp32(q, k, v, attn_mask=mask))
    assert not out[:, :, dead].float().abs().sum()
    assert torch.isinf(lse[:, :, dead]).all() and (lse[:, :, dead] < 0).all()


@pytest.mark.parametrize("kind", ["f16", "bool"])
@pytest.mark.parametrize("shape", ["qk", "b1qk", "1h1k", "bhqk", "kq_view"])
def test_unaligned_masks_are_copied(cuda, kind, shape):
    """fp16 / bool masks whose rows are not whole 16-byte units (Skv 77, a
    transposed view) are copied with 16-byte rows into the workspace and
    staged like aligned ones: the output equals, bit for bit, the call with
    the same mask stored in aligned rows, and matches the oracle."""
    import torch_spyre_amd as tsa

    B, Hq, Hkv, Sq, Skv, D = 2, 4, 2, 50, 77, 128
    q = randn((B, Hq, Sq, D), SEED + 26).to(cuda)
    k, v = randn((B, Hkv, Skv, D), SEED + 27).to(cuda), randn((B, Hkv, Skv, D), SEED + 28).to(cuda)
    dims = {"qk": (Sq, Skv), "b1qk": (B, 1, Sq, Skv), "1h1k": (1, Hq, 1, Skv), "bhqk": (B, Hq, Sq, Skv),
            "kq_view": (Skv, Sq)}[shape]
    mask = _mask(kind, dims, SEED + 29)
    mask = mask.to(cuda).t() if shape == "kq_view" else mask.to(cuda)  # kq_view: key stride Sq
    wide = torch.zeros((*mask.shape[:-1], 80), dtype=mask.dtype, device=cuda)
    wide[..., :Skv] = mask
    aligned = wide[..., :Skv]  # 160- / 80-byte rows: staged as it lies
    out = tsa.scaled_dot_product_attention(q, k, v, attn_mask=mask, enable_gqa=True)
    ref = tsa.scaled_dot_product_attention(q, k, v, attn_mask=aligned, enable_gqa=True)
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    assert_close(out, OA.sdpa_cpu_fp32(q.cpu(), k.cpu(), v.cpu(), attn_mask=mask.cpu()))


def test_unaligned_mask_with_v_sized_workspace(cuda):
    """A caller's workspace sized for V's relayout but too small for the
    mask's copy: the call runs the per-wavefront kernel, same results."""
    import torch_spyre_amd as tsa

    B, Hq, Hkv, Sq, Skv, D = 1, 8, 2, 300, 77, 128
    q = randn((B, Hq, Sq, D), SEED + 30).to(cuda)
    k, v = randn((B, Hkv, Skv, D), SEED + 31).to(cuda), randn((B, Hkv, Skv, D), SEED + 32).to(cuda)
    mask = _mask("f16", (B, Hq, Sq, Skv), SEED + 33).to(cuda)
    vt = tsa.sdpa.workspace_bytes(B, Hkv, Skv, D)
    m = mask.expand(B, Hq, Sq, Skv)
    from torch_spyre_amd import _lib

    need = _lib.lib().spyre_sdpa_fwd_call_workspace_bytes(m.data_ptr(), 1, _lib.i64_array(m.stride()), B, Hq, Hkv,
                                                          Sq, Skv, D)
    assert need == B * Hq * Sq * 160 > vt
    ws = torch.empty(vt, dtype=torch.uint8, device=cuda)
    out = tsa.scaled_dot_product_attention(q, k, v, attn_mask=mask, enable_gqa=True, workspace=ws)
    assert_close(out, OA.sdpa_cpu_fp32(q.cpu(), k.cpu(), v.cpu(), attn_mask=mask.cpu()))


@pytest.mark.parametrize("pattern", ["causal_inf", "causal_min", "window_bool", "padding_bool"])
def test_block_sparse_masks(cuda, pattern):
    """Masks that blank whole 32-query x 64-key blocks (causal as a bias of
    -inf or of fp16's minimum, a sliding window, key padding): such blocks
    add nothing and are skipped, the rest must still match."""
    Sq = Skv = 448
    q = randn((1, 4, Sq, 128), SEED + 23)
    k, v = randn((1, 2, Skv, 128), SEED + 24), randn((1, 2, Skv, 128), SEED + 25)
    i = torch.arange(Sq)[:, None]
    j = torch.arange(Skv)[None, :]
    if pattern.startswith("causal"):
        fill = -float("inf") if pattern == "causal_inf" else -65504.0
        mask = torch.zeros((Sq, Skv)).masked_fill(j > i, fill).half()
    elif pattern == "window_bool":
        mask = (j <= i) & (j > i - 100)
    else:
        mask = (j < 200).expand(Sq, Skv)
    out, lse = run(cuda, q, k, v, attn_mask=mask, enable_gqa=True, return_lse=True)
    assert_close(out, OA.sdpa_cpu_fp32(q, k, v, attn_mask=mask))
    _, lse64 = OA.sdpa_decomposition_fp64(q, k, v, attn_mask=mask.numpy(), return_lse=True)
    assert np.allclose(lse.cpu().numpy(), lse64, atol=LSE_ATOL, rtol=0)


def test_fully_masked_rows_give_zeros_and_minus_inf_lse(cuda):
    q, k, v = randn((1, 2, 40, 64), SEED + 5), randn((1, 2, 33, 64), SEED + 6), randn((1, 2, 33, 64), SEED + 7)
    mask = torch.zeros((40, 33))
    mask[3] = -float("inf")
    mask[39] = -float("inf")
    out, lse = run(cuda, q, k, v, attn_mask=mask, return_lse=True)
    ref = OA.sdpa_cpu_fp32(q, k, v, attn_mask=mask)
    assert_close(out, ref)
    assert not out[:, :, 3].float().abs().sum() and not out[:, :, 39].float().abs().sum()
    assert torch.isinf(lse[:, :, 3]).all() and (lse[:, :, 3] < 0).all()


def test_empty_keys_give_zeros(cuda):
    q = randn((1, 2, 5, 64), SEED + 8)
    k = torch.empty((1, 2, 0, 64), dtype=torch.float16)
    out = run(cuda, q, k, k)
    assert out.shape == (1, 2, 5, 64) and not out.float().abs().sum()


def test_scale_applied_once(cuda):
    q, k, v = randn((1, 4, 30, 128), SEED + 9), randn((1, 4, 45, 128), SEED + 10), randn((1, 4, 45, 128), SEED + 11)
    assert_close(run(cuda, q, k, v, scale=0.3), OA.sdpa_cpu_fp32(q, k, v, scale=0.3))


@pytest.mark.parametrize("scale", [0.0, -0.2])
@pytest.mark.parametrize("causal", [False, True])
def test_zero_and_negative_scale(cuda, scale, causal):
    """scale 0 averages the visible values (LSE = log of their count); a
    negative scale flips the scores (the kernel folds the sign into q): the
    call equals the positive scale on -q bit for bit, and its LSE is the fp64
    logsumexp of -q with |scale|."""
    q, k, v = randn((1, 4, 70, 64), SEED + 40), randn((1, 4, 90, 64), SEED + 41), randn((1, 4, 90, 64), SEED + 42)
    out, lse = run(cuda, q, k, v, scale=scale, is_causal=causal, return_lse=True)
    assert_close(out, OA.sdpa_cpu_fp32(q, k, v, scale=scale, is_causal=causal))
    if scale == 0:
        seen = torch.arange(1, 71).clamp(max=90) if causal else torch.full((70,), 90)
        want = torch.log(seen.double()).expand(1, 4, 70)
        assert np.allclose(lse.cpu().numpy(), want.numpy(), atol=LSE_ATOL, rtol=0)
        return
    out_n, lse_n = run(cuda, -q, k, v, scale=-scale, is_causal=causal, return_lse=True)
    assert torch.equal(out.cpu(), out_n.cpu()) and torch.equal(lse.cpu(), lse_n.cpu())
    _, lse64 = OA.sdpa_decomposition_fp64(-q, k, v, scale=-scale, is_causal=causal, return_lse=True)
    assert np.allclose(lse.cpu().numpy(), lse64, atol=LSE_ATOL, rtol=1e-5)


@pytest.mark.parametrize("causal", [False, True])
def test_large_scale(cuda, causal):
    """|scale log2 e| > 1 (here scale 2): Q is not prescaled (q * scale could
    leave fp16), the scale goes into the exponent instead; nearly one-hot
    rows."""
    q, k, v = randn((1, 4, 130, 128), SEED + 43), randn((1, 4, 150, 128), SEED + 44), randn((1, 4, 150, 128), SEED + 45)
    out, lse = run(cuda, q, k, v, scale=2.0, is_causal=causal, return_lse=True)
    assert_close(out, OA.sdpa_cpu_fp32(q, k, v, scale=2.0, is_causal=causal))
    _, lse64 = OA.sdpa_decomposition_fp64(q, k, v, scale=2.0, is_causal=causal, return_lse=True)
    assert np.allclose(lse.cpu().numpy(), lse64, atol=LSE_ATOL, rtol=1e-5)


def test_unaligned_views_are_accepted(cuda):
    """A head-dim slice of a wider tensor (rows not 16-byte multiples apart)
    is copied into kernel form first; the result is unchanged."""
    base = randn((1, 2, 50, 136), SEED + 12)
    q = base[..., 4:132]
    k, v = randn((1, 2, 60, 128), SEED + 13), randn((1, 2, 60, 128), SEED + 14)
    assert_close(run(cuda, q, k, v), OA.sdpa_cpu_fp32(q, k, v))


def test_overrideable_tuple_and_custom_op(cuda):
    import torch_spyre_amd as tsa

    q, k, v = ref_case(1, 100, 100, 8, 2, 64, SEED + 15)
    q, k, v = q.to(cuda), k.to(cuda), v.to(cuda)
    res = tsa.sdpa_overrideable(q, k, v, None, 0.0, True)
    assert len(res) == 9 and res[2] is None and res[3] is None and res[8] is None
    assert res[4] == 100 and res[5] == 100 and res[1].shape == (1, 8, 100) and res[1].dtype == torch.float32
    ref = OA.sdpa_cpu_fp32(q, k, v, is_causal=True)
    assert_close(res[0], ref)
    out, lse = torch.ops.spyre.sdpa_fwd(q, k, v, None, True, None, True)
    assert torch.equal(out, res[0]) and torch.equal(lse, res[1])


def test_workspace_only_for_masks(cuda):
    """Calls without a mask read V as it lies: with a caller's workspace of
    the size the call asks for (a key split's partials here: 16 blocks for
    the device) the bits equal the call that allocates its own; with none or
    a smaller one, the unsplit grid runs, within the bar.  K and V with
    different row strides; a masked call still checks its workspace."""
    import torch_spyre_amd as tsa
    from torch_spyre_amd import _lib

    q = randn((1, 8, 300, 128), SEED + 40).to(cuda)
    k = randn((1, 2, 1100, 128), SEED + 41).to(cuda)
    v = randn((1, 1100, 2, 128), SEED + 42).to(cuda).transpose(1, 2)  # row stride 256, K's is 128
    for causal in (False, True):
        need = _lib.lib().spyre_sdpa_fwd_call_workspace_bytes(None, 0, None, 1, 8, 2, 300, 1100, 128)
        assert need > 0
        a = tsa.scaled_dot_product_attention(q, k, v, is_causal=causal, enable_gqa=True)
        ws = torch.empty(max(need, 16), dtype=torch.uint8, device=cuda)
        b = tsa.scaled_dot_product_attention(q, k, v, is_causal=causal, enable_gqa=True, workspace=ws)
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))
        c = tsa.scaled_dot_product_attention(q, k, v, is_causal=causal, enable_gqa=True,
                                             workspace=torch.empty(16, dtype=torch.uint8, device=cuda))
        ref = OA.sdpa_cpu_fp32(q.cpu(), k.cpu(), v.cpu(), is_causal=causal)
        assert_close(a, ref)
        assert_close(c, ref)
    mask = torch.zeros((300, 1100), dtype=torch.float16, device=cuda)
    with pytest.raises(ValueError):
        tsa.scaled_dot_product_attention(q, k, v, attn_mask=mask, enable_gqa=True,
                                         workspace=torch.empty(16, dtype=torch.uint8, device=cuda))


# Decode with few (sequence, KV head) pairs.  One row tile (g q heads x
# Sq <= 32 rows) runs the short-decode kernel: a block takes 8 wavefront
# slices of 64 keys (D 64) or 32 (D 128), all loaded at once, and longer key
# runs split into such blocks while they all fit one round of the device
# (the Llama-3-8B batch-1 step: 16 splits of 256 keys; a ragged last split;
# D 64 without GQA); 512 keys at D 64 and 200 at D 128 are one block (a
# ragged last slice), 130 keys leave 5 slices empty.  Past one round, the
# LDS kernel splits instead (16384 keys: 32 splits of 512; 20000: 32 of
# 640, the last 160).  split: whether the call needs partials.
@pytest.mark.parametrize("B,Hq,Hkv,Skv,D,split", [(1, 32, 8, 4096, 128, True), (1, 32, 8, 1500, 128, True),
                                                  (1, 8, 8, 2048, 64, True), (2, 64, 8, 3000, 128, True),
                                                  (1, 8, 8, 512, 64, False), (1, 8, 8, 130, 64, False),
                                                  (1, 32, 8, 200, 128, False), (1, 32, 8, 16384, 128, True),
                                                  (1, 8, 8, 20000, 64, True)])
def test_key_split_for_small_grids(cuda, B, Hq, Hkv, Skv, D, split):
    from torch_spyre_amd import _lib

    assert (_lib.lib().spyre_sdpa_fwd_call_workspace_bytes(None, 0, None, B, Hq, Hkv, 1, Skv, D) > 0) == split
    q = randn((B, Hq, 1, D), SEED + 60 + Skv)
    k, v = randn((B, Hkv, Skv, D), SEED + 61), randn((B, Hkv, Skv, D), SEED + 62)
    out, lse = run(cuda, q, k, v, enable_gqa=True, return_lse=True)
    assert_close(out, OA.sdpa_cpu_fp32(q, k, v))
    _, lse64 = OA.sdpa_decomposition_fp64(q, k, v, return_lse=True)
    assert np.allclose(lse.cpu().numpy(), lse64, atol=LSE_ATOL, rtol=0)


# The short-decode kernel with several query rows per q head (Sq x g <= 32:
# speculative decode, a short chunk), an explicit scale outside the
# prescaled range (|scale log2 e| > 1) and a negative one, empty contexts,
# and q / k / v views with padded strides.
@pytest.mark.parametrize("B,Hq,Hkv,Sq,Skv,D,scale", [(2, 8, 2, 4, 700, 64, None), (1, 16, 2, 3, 300, 128, None),
                                                     (3, 4, 4, 32, 100, 128, None), (1, 8, 8, 1, 512, 64, 2.0),
                                                     (2, 32, 8, 1, 260, 128, -0.3), (1, 8, 8, 5, 0, 64, None)])
def test_short_decode_rows_and_scales(cuda, B, Hq, Hkv, Sq, Skv, D, scale):
    q = randn((B, Hq, Sq, D + 8), SEED + 70 + Skv)[..., :D]
    k = randn((B, Hkv, Skv, D + 16), SEED + 71)[..., :D]
    v = randn((B, Hkv, Skv, D), SEED + 72)
    out, lse = run(cuda, q, k, v, enable_gqa=True, return_lse=True, scale=scale)
    if Skv == 0:
        assert torch.equal(out.cpu(), torch.zeros_like(out.cpu()))
        assert bool(torch.isneginf(lse.cpu()).all())
        return
    assert_close(out, OA.sdpa_cpu_fp32(q, k, v, scale=scale))
    # the fp64 decomposition splits the scale as sqrt(scale) on q and k: a
    # negative scale is |scale| on -q
    sign = -1 if scale is not None and scale < 0 else 1
    _, lse64 = OA.sdpa_decomposition_fp64(sign * q, k, v, scale=None if scale is None else abs(scale),
                                          return_lse=True)
    # rtol: q * scale * log2(e) is rounded to fp16 (relative 2^-11 per
    # element) when |scale log2 e| <= 1, which alone moves an LSE of ~13 by
    # up to ~2.3e-3 at the scale -0.3 case
    assert np.allclose(lse.cpu().numpy(), lse64, atol=LSE_ATOL, rtol=2e-4)


def test_argument_errors(cuda):
    import torch_spyre_amd as tsa

    q, k, v = randn((1, 4, 8, 64), 1).to(cuda), randn((1, 2, 8, 64), 2).to(cuda), randn((1, 2, 8, 64), 3).to(cuda)
    with pytest.raises(ValueError):
        tsa.scaled_dot_product_attention(q, k, v)  # GQA without enable_gqa
    with pytest.raises(tsa.Unsupported):
        tsa.scaled_dot_product_attention(q, k, v, dropout_p=0.1, enable_gqa=True)
    with pytest.raises(ValueError):
        tsa.scaled_dot_product_attention(q, k, v, attn_mask=torch.zeros(8, 8, device=cuda), is_causal=True,
                                         enable_gqa=True)
    q96, k96 = randn((1, 2, 8, 96), 4).to(cuda), randn((1, 2, 8, 96), 5).to(cuda)
    with pytest.raises(tsa._lib.SpyreHipError):
        tsa.scaled_dot_product_attention(q96, k96, k96)  # head_dim 96


def test_llama3_8b_prefill_1024_causal_sampled_heads(cuda):
    """Batch 1, 32 q / 8 KV heads, D 128, 1024 tokens, causal: four heads
    (two KV groups) against the oracle."""
    q = randn((1, 32, 1024, 128), SEED + 20)
    k = randn((1, 8, 1024, 128), SEED + 21)
    v = randn((1, 8, 1024, 128), SEED + 22)
    out = run(cuda, q, k, v, is_causal=True, enable_gqa=True).cpu()
    for h in (0, 3, 17, 31):
        ref = OA.sdpa_cpu_fp32(q[:, h:h + 1], k[:, h // 4:h // 4 + 1], v[:, h // 4:h // 4 + 1], is_causal=True)
        assert_close(out[:, h:h + 1], ref)


@pytest.mark.parametrize("causal", [False, True])
def test_bench_shape_prefill_all_heads(cuda, causal):
    """The measured prefill shape (batch 1, 32 q / 8 KV heads, 4096 tokens,
    D 128): every q head against the oracle, LSE of one head per KV group
    against the fp64 logsumexp, and for causal attention the closed form of
    row 0 (it sees key 0 only: out = v[0]) on every head."""
    S = 4096
    q = randn((1, 32, S, 128), SEED + 50)
    k = randn((1, 8, S, 128), SEED + 51)
    v = randn((1, 8, S, 128), SEED + 52)
    out, lse = run(cuda, q, k, v, is_causal=causal, enable_gqa=True, return_lse=True)
    out, lse = out.cpu(), lse.cpu()
    for h in range(32):
        kv = h // 4
        ref = OA.sdpa_cpu_fp32(q[:, h:h + 1], k[:, kv:kv + 1], v[:, kv:kv + 1], is_causal=causal)
        assert_close(out[:, h:h + 1], ref)
    for h in (1, 6, 11, 13, 18, 23, 24, 31):
        kv = h // 4
        _, lse64 = OA.sdpa_decomposition_fp64(q[:, h:h + 1], k[:, kv:kv + 1], v[:, kv:kv + 1], is_causal=causal,
                                              return_lse=True)
        assert np.allclose(lse[:, h:h + 1].numpy(), lse64, atol=LSE_ATOL, rtol=1e-5), h
    if causal:
        first = out[0, :, 0].float()
        want = v[0, torch.arange(32) // 4, 0].float()
        assert torch.equal(first, want)


@pytest.mark.parametrize("kind", ["f16", "bool"])
def test_bench_shape_masked_prefill_sampled_heads(cuda, kind):
    """The measured masked prefill: batch 1, 32 q / 8 KV heads, 4096 tokens,
    D 128, one [4096, 4096] mask broadcast over heads -- an fp16 bias
    ~ N(0, 1) or a boolean keep-mask (70 % kept).  Four q heads from
    different KV groups against the oracle, LSE of two against the fp64
    logsumexp."""
    S = 4096
    q = randn((1, 32, S, 128), SEED + 53)
    k = randn((1, 8, S, 128), SEED + 54)
    v = randn((1, 8, S, 128), SEED + 55)
    gen = torch.Generator().manual_seed(SEED + 56)
    if kind == "f16":
        mask = torch.randn((S, S), generator=gen).half()
    else:
        mask = torch.rand((S, S), generator=gen) < 0.7
    out, lse = run(cuda, q, k, v, attn_mask=mask, enable_gqa=True, return_lse=True)
    out, lse = out.cpu(), lse.cpu()
    for h in (0, 13, 22, 31):
        kv = h // 4
        ref = OA.sdpa_cpu_fp32(q[:, h:h + 1], k[:, kv:kv + 1], v[:, kv:kv + 1], attn_mask=mask)
        assert_close(out[:, h:h + 1], ref)
    for h in (5, 26):
        kv = h // 4
        _, lse64 = OA.sdpa_decomposition_fp64(q[:, h:h + 1], k[:, kv:kv + 1], v[:, kv:kv + 1],
                                              attn_mask=mask.numpy(), return_lse=True)
        assert np.allclose(lse[:, h:h + 1].numpy(), lse64, atol=LSE_ATOL, rtol=1e-5), h


PREPARED_CASES = [
    # (B, Hq, Hkv, Sq, Skv, D, causal, mask kind)
    (1, 8, 8, 1, 512, 64, False, None),       # batch-1 decode: 8 key splits of one step + merge
    (1, 32, 8, 1, 4096, 128, False, None),    # Llama-3-8B batch-1 decode: 32 key splits + merge
    (4, 32, 8, 1, 700, 128, False, None),     # packed GQA decode
    (2, 8, 2, 100, 300, 128, True, None),     # causal prefill
    (1, 4, 4, 64, 200, 64, False, "f16"),     # additive fp16 mask
    (1, 4, 2, 50, 129, 128, False, "bool"),   # boolean keep-mask, GQA
]


@pytest.mark.parametrize("B,Hq,Hkv,Sq,Skv,D,causal,mk", PREPARED_CASES, ids=str)
def test_prepared_call_matches_eager(cuda, B, Hq, Hkv, Sq, Skv, D, causal, mk):
    """SdpaCall, validated once and launched three times with q, k and v
    rewritten in place before each launch: every launch bit-equal (out and
    lse) to the eager call on the same inputs, and within the bar of the
    oracle."""
    import torch_spyre_amd as tsa

    gg = torch.Generator(device=cuda).manual_seed(SEED + 300 + Skv)
    q = torch.empty((B, Hq, Sq, D), dtype=torch.float16, device=cuda)
    k = torch.empty((B, Hkv, Skv, D), dtype=torch.float16, device=cuda)
    v = torch.empty((B, Hkv, Skv, D), dtype=torch.float16, device=cuda)
    mask = None
    if mk == "f16":
        mask = torch.randn((Sq, Skv), generator=gg, device=cuda).half()
    elif mk == "bool":
        mask = torch.rand((B, 1, Sq, Skv), generator=gg, device=cuda) < 0.7
        mask[..., 0] = True
    call = tsa.SdpaCall(q, k, v, attn_mask=mask, is_causal=causal, enable_gqa=Hq != Hkv, return_lse=True)
    for _ in range(3):
        for t in (q, k, v):
            t.copy_(torch.randn(t.shape, generator=gg, device=cuda).half())
        out, lse = call()
        want, want_lse = tsa.scaled_dot_product_attention(q, k, v, attn_mask=mask, is_causal=causal,
                                                          enable_gqa=Hq != Hkv, return_lse=True)
        torch.cuda.synchronize()
        assert out.shape == want.shape and out.stride() == want.stride()
        assert torch.equal(out.view(torch.int16), want.view(torch.int16))
        assert torch.equal(lse, want_lse)
    ref = OA.sdpa_cpu_fp32(q.cpu(), k.cpu(), v.cpu(), attn_mask=None if mask is None else mask.cpu(),
                           is_causal=causal)
    assert_close(out, ref)


def test_prepared_call_refuses_copies(cuda):
    """Operands the kernel cannot read as they lie are copied by the eager
    call but refused by SdpaCall, which must read the caller's storage on
    every launch."""
    import torch_spyre_amd as tsa

    q = randn((1, 8, 1, 64), SEED + 320).to(cuda)
    kp = randn((1, 8, 512, 65), SEED + 321).to(cuda)
    k = kp[..., :64]  # row stride 65: not a multiple of 8
    v = randn((1, 8, 512, 64), SEED + 322).to(cuda)
    with pytest.raises(ValueError):
        tsa.SdpaCall(q, k, v)
    assert_close(tsa.scaled_dot_product_attention(q, k, v), OA.sdpa_cpu_fp32(q.cpu(), k.cpu(), v.cpu()))


def test_stream_pointer_follows_current_stream(cuda):
    """The launch stream is the device's current stream, inside a stream
    context too."""
    from torch_spyre_amd.relayout import _stream_ptr

    assert _stream_ptr(cuda) == torch.cuda.current_stream(cuda).cuda_stream
    s = torch.cuda.Stream(device=cuda)
    with torch.cuda.stream(s):
        assert _stream_ptr(cuda) == s.cuda_stream
        assert _stream_ptr(torch.device("cuda")) == s.cuda_stream
    assert _stream_ptr(cuda) == torch.cuda.current_stream(cuda).cuda_stream


def _short_decode_shapes(n, seed):
    """Seeded shapes in the short-decode domain (g q heads x Sq <= 32 rows
    per block): batch, KV heads, group, Sq, D, key count (0 .. 3000, most
    not a multiple of a slice) and a row padding for q and k."""
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        g = int(rng.choice([1, 2, 4, 8]))
        sq = int(rng.integers(1, 32 // g + 1))
        out.append((int(rng.integers(1, 4)), int(rng.choice([1, 2, 4, 8])), g, sq, int(rng.choice([64, 128])),
                    int(rng.integers(0, 3001)), int(rng.choice([0, 8, 32]))))
    return out


@pytest.mark.parametrize("B,Hkv,g,Sq,D,Skv,pad", _short_decode_shapes(16, SEED + 90), ids=str)
def test_short_decode_random_shapes(cuda, B, Hkv, g, Sq, D, Skv, pad):
    Hq = Hkv * g
    q = randn((B, Hq, Sq, D + pad), SEED + 91 + Skv)[..., :D]
    k = randn((B, Hkv, Skv, D + pad), SEED + 92)[..., :D]
    v = randn((B, Hkv, Skv, D), SEED + 93)
    out, lse = run(cuda, q, k, v, enable_gqa=True, return_lse=True)
    if Skv == 0:
        assert not out.float().abs().sum() and bool(torch.isneginf(lse.cpu()).all())
        return
    assert_close(out, OA.sdpa_cpu_fp32(q, k, v))
    _, lse64 = OA.sdpa_decomposition_fp64(q, k, v, return_lse=True)
    assert np.allclose(lse.cpu().numpy(), lse64, atol=LSE_ATOL, rtol=0)


@pytest.mark.parametrize("Sq,Skv,causal", [(300, 200, False), (300, 300, True), (1, 700, False), (4, 130, False)])
def test_keys_expanded_along_the_sequence(cuda, Sq, Skv, causal):
    """K and V expanded from one row ([B, Hkv, 1, D] with sequence stride 0):
    every key is the same, so each row's output is that value row and its
    LSE is scale q.k + ln(visible keys); prefill (full, causal) and the
    short-decode kernel."""
    B, Hq, Hkv, D = 2, 8, 2, 128
    q = randn((B, Hq, Sq, D), SEED + 95)
    k1, v1 = randn((B, Hkv, 1, D), SEED + 96), randn((B, Hkv, 1, D), SEED + 97)
    k, v = k1.to(cuda).expand(B, Hkv, Skv, D), v1.to(cuda).expand(B, Hkv, Skv, D)
    assert k.stride(2) == 0
    out, lse = run(cuda, q, k, v, is_causal=causal, enable_gqa=True, return_lse=True)
    g = Hq // Hkv
    want = v1.float().repeat_interleave(g, dim=1).expand(B, Hq, Sq, D)
    assert_close(out, want)
    s = (q.double() @ k1.double().repeat_interleave(g, dim=1).transpose(-1, -2))[..., 0] / math.sqrt(D)
    visible = torch.arange(Sq, dtype=torch.float64).add(1).clamp(max=Skv) if causal else torch.full((Sq,), float(Skv))
    assert np.allclose(lse.cpu().double().numpy(), (s + visible.log()).numpy(), atol=LSE_ATOL, rtol=0)


@pytest.mark.parametrize("Sq", [1, 70])
def test_key_stride_near_the_descriptor_limit(cuda, Sq):
    """K and V rows 2^29 elements (1 GiB) apart, 2 keys: the head's span
    ends just inside one 2 GiB buffer descriptor while Skv x stride passes
    it, so the tile loads' byte counts start clamped; prefill and the
    short-decode kernel."""
    D, ss = 128, 1 << 29
    q = randn((1, 2, Sq, D), SEED + 98)
    kv = []
    for s in (SEED + 99, SEED + 100):
        base = torch.zeros(ss + D, dtype=torch.float16, device=cuda)
        rows = randn((2, D), s)
        base[:D] = rows[0].to(cuda)
        base[ss:] = rows[1].to(cuda)
        kv.append(base.as_strided((1, 1, 2, D), (0, 0, ss, 1)))
    k, v = kv
    assert k.stride(2) * 2 * 2 > 0x7FFFFFF0 >= ((k.shape[2] - 1) * k.stride(2) + D) * 2
    out, lse = run(cuda, q, k, v, enable_gqa=True, return_lse=True)
    kc, vc = k.cpu(), v.cpu()
    assert_close(out, OA.sdpa_cpu_fp32(q, kc, vc))
    _, lse64 = OA.sdpa_decomposition_fp64(q, kc, vc, return_lse=True)
    assert np.allclose(lse.cpu().numpy(), lse64, atol=LSE_ATOL, rtol=0)
    del k, v, kv
    torch.cuda.empty_cache()


# Decode calls whose (sequence, KV head, chunk) grid fills at least half the
# device stream dense K / V through the split-KV decode kernels: one chunk
# per sequence, or several merged in the same kernel (the merge pass for a
# grid of more than one round); a ragged last 64-token run
# (read as the 64-token window ending with the last key); contexts shorter
# than one run; g = 1 and 16; K / V rows padded past D; D = 128 and 64.
DENSE_DECODE_CASES = [
    (32, 32, 8, 4096, 0, 128),  # Llama-3-8B decode: one chunk per (sequence, KV head)
    (4, 32, 8, 32768, 0, 128),  # long context: 8 chunks merged in the kernel
    (2, 16, 8, 20037, 0, 128),  # 16 chunks, the last run 5 tokens
    (64, 64, 64, 1000, 0, 128),  # g = 1, a ragged last run
    (16, 256, 16, 2049, 64, 128),  # g = 16, K / V rows 192 features apart
    (256, 32, 8, 70, 0, 128),  # shorter than one wavefront's share
    (3, 32, 8, 4096, 0, 128),  # 192 workgroups of one-page shares (three quarters of a 256-CU device)
    (24, 32, 8, 520, 0, 128),  # 192 single-chunk workgroups, a ragged last run
    (32, 32, 8, 4096, 0, 64),  # D = 64
    (8, 32, 8, 16384, 0, 64),  # D = 64, chunks merged in the kernel
    (32, 16, 16, 2047, 8, 64),  # D = 64, g = 1, K / V rows 72 features apart, a ragged last run
    (64, 32, 8, 40, 0, 128),  # a context shorter than one run: per-lane offsets, tokens past it out of range
    (32, 16, 16, 33, 8, 64),  # D = 64, shorter than one run, K / V rows 72 features apart
    (64, 32, 8, 65, 0, 128),  # the last run a window of 64 tokens with one of its own
    (64, 8, 8, 2048, 0, 128),  # four-wavefront items (the eight-wavefront grid takes two rounds)
    (24, 32, 8, 5000, 0, 128),  # four-wavefront items in three chunks, more than one round: the merge pass
]


def _dense_case(cuda, B, Hq, Hkv, Skv, pad, D, seed):
    q = randn((B, Hq, 1, D), seed)
    kf, vf = randn((B, Hkv, Skv, D + pad), seed + 1), randn((B, Hkv, Skv, D + pad), seed + 2)
    k, v = kf.to(cuda)[..., :D], vf.to(cuda)[..., :D]  # views with the padded token stride
    assert k.stride(2) == D + pad
    return q, k, v, kf[..., :D], vf[..., :D]


@pytest.mark.parametrize("B,Hq,Hkv,Skv,pad,D", DENSE_DECODE_CASES, ids=str)
def test_dense_decode_through_split_kernels(cuda, B, Hq, Hkv, Skv, pad, D):
    """Every sequence against CPU fp32 SDPA; LSE against the fp64
    logsumexp within 1e-4, below ln(n / (n - 1)) for these contexts' equal
    scores, the shift of one lost or doubled key."""
    q, k, v, kc, vc = _dense_case(cuda, B, Hq, Hkv, Skv, pad, D, SEED + 110 + Skv)
    out, lse = run(cuda, q, k, v, enable_gqa=True, return_lse=True)
    out = out.cpu()
    assert torch.equal(run(cuda, q, k, v, enable_gqa=True).cpu(), out)  # without the LSE: the same bits
    for b in range(B):
        assert_close(out[b:b + 1], OA.sdpa_cpu_fp32(q[b:b + 1], kc[b:b + 1], vc[b:b + 1]))
    lse64 = np.stack([OA.decode_lse_fp64(q[b, :, 0].numpy(), kc[b].numpy()) for b in range(B)])
    err = np.abs(lse.cpu().double().numpy()[..., 0] - lse64).max()
    assert err <= 1e-4, err


@pytest.mark.parametrize("B,Hq,Hkv,Skv,pad,D", [DENSE_DECODE_CASES[i] for i in (1, 2, 4, 9, 10, 11, 12, 13)],
                         ids=str)
def test_dense_decode_counts_every_key_once(cuda, B, Hq, Hkv, Skv, pad, D):
    """q = 0: every score is 0, so LSE = ln(Skv) up to the fp32 rounding of
    the log (a lost or doubled key moves it by at least 1/Skv) and out is the
    mean of V over the keys."""
    q, k, v, _, vc = _dense_case(cuda, B, Hq, Hkv, Skv, pad, D, SEED + 120 + Skv)
    out, lse = run(cuda, torch.zeros_like(q), k, v, enable_gqa=True, return_lse=True)
    assert np.abs(lse.cpu().double().numpy() - math.log(Skv)).max() <= 4e-6
    g = Hq // Hkv
    assert_close(out, vc.float().mean(dim=2, keepdim=True).repeat_interleave(g, dim=1))


def test_dense_decode_keys_expanded_along_the_sequence(cuda):
    """K and V expanded from one row (token stride 0) on a grid the
    split-KV kernels take: each row's output is that value row and its LSE
    scale q.k + ln(Skv)."""
    B, Hq, Hkv, Skv, D = 32, 32, 8, 4096, 128
    q = randn((B, Hq, 1, D), SEED + 130)
    k1, v1 = randn((B, Hkv, 1, D), SEED + 131), randn((B, Hkv, 1, D), SEED + 132)
    k, v = k1.to(cuda).expand(B, Hkv, Skv, D), v1.to(cuda).expand(B, Hkv, Skv, D)
    out, lse = run(cuda, q, k, v, enable_gqa=True, return_lse=True)
    g = Hq // Hkv
    assert_close(out, v1.float().repeat_interleave(g, dim=1))
    s = (q.double() @ k1.double().repeat_interleave(g, dim=1).transpose(-1, -2))[..., 0, 0] / math.sqrt(D)
    assert np.allclose(lse.cpu().double().numpy()[..., 0], (s + math.log(Skv)).numpy(), atol=1e-4, rtol=0)


@pytest.mark.parametrize("B,Hq,Hkv,Sq,Skv,D", [(1, 32, 8, 256, 4096, 128), (8, 32, 8, 64, 2048, 128),
                                               (16, 32, 8, 16, 4096, 128), (1, 16, 4, 512, 4100, 64)], ids=str)
def test_key_split_many_rows(cuda, B, Hq, Hkv, Sq, Skv, D):
    """Chunked-prefill shapes whose blocks would not fill the device: the
    keys are split and the partials of thousands of rows merged by the
    kernel that gives each row its own threads; out against CPU fp32, LSE
    against fp64."""
    from torch_spyre_amd import _lib

    assert _lib.lib().spyre_sdpa_fwd_call_workspace_bytes(None, 0, None, B, Hq, Hkv, Sq, Skv, D) > 0  # split
    q = randn((B, Hq, Sq, D), SEED + 140 + Sq)
    k, v = randn((B, Hkv, Skv, D), SEED + 141), randn((B, Hkv, Skv, D), SEED + 142)
    out, lse = run(cuda, q, k, v, enable_gqa=True, return_lse=True)
    assert_close(out, OA.sdpa_cpu_fp32(q, k, v))
    _, lse64 = OA.sdpa_decomposition_fp64(q, k, v, return_lse=True)
    assert np.allclose(lse.cpu().numpy(), lse64, atol=LSE_ATOL, rtol=0)


def _route_shapes(n, seed):
    """Seeded calls across the SDPA entry's routes -- short decode, the
    split-KV decode kernels on dense K / V, the LDS kernel with and without
    a key split (and its two merge kernels), causal -- with the CPU oracle's
    work bounded: batch, q heads, KV heads, Sq, Skv, D, causal."""
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        D = int(rng.choice([64, 128]))
        Hkv = int(rng.choice([1, 2, 4, 8]))
        g = int(rng.choice([1, 2, 4, 8, 16]))
        B = int(rng.choice([1, 2, 3, 5, 8, 16, 24, 32, 48]))
        Sq = 1 if rng.random() < 0.5 else int(rng.choice([2, 7, 33, 64, 100, 256, 300]))
        Skv = int(rng.integers(1, 9000))
        causal = bool(Sq > 1 and rng.random() < 0.3)
        if B * Hkv * g * Sq * Skv * D > 4e9 or B * Hkv * Skv * D > 6e7:
            continue
        out.append((B, Hkv * g, Hkv, Sq, Skv, D, causal))
    return out


@pytest.mark.parametrize("B,Hq,Hkv,Sq,Skv,D,causal", _route_shapes(24, SEED + 150), ids=str)
def test_random_calls_across_routes(cuda, B, Hq, Hkv, Sq, Skv, D, causal):
    """Out against CPU fp32 SDPA and LSE against the fp64 logsumexp for
    seeded shapes that land on every route of the entry."""
    q = randn((B, Hq, Sq, D), SEED + 151 + Skv)
    k, v = randn((B, Hkv, Skv, D), SEED + 152), randn((B, Hkv, Skv, D), SEED + 153)
    out, lse = run(cuda, q, k, v, is_causal=causal, enable_gqa=True, return_lse=True)
    out = out.cpu()
    for b in range(B):
        assert_close(out[b:b + 1], OA.sdpa_cpu_fp32(q[b:b + 1], k[b:b + 1], v[b:b + 1], is_causal=causal))
    if Sq == 1:
        lse64 = np.stack([OA.decode_lse_fp64(q[b, :, 0].numpy(), k[b].numpy()) for b in range(B)])[..., None]
    else:
        lse64 = np.concatenate([OA.sdpa_decomposition_fp64(q[b:b + 1], k[b:b + 1], v[b:b + 1], is_causal=causal,
                                                           return_lse=True)[1] for b in range(B)])
    assert np.allclose(lse.cpu().numpy(), lse64, atol=LSE_ATOL, rtol=0)


@pytest.mark.parametrize("D", [64, 128])
def test_dense_decode_ignores_rows_past_the_keys(cuda, D):
    """K / V views of the first Skv rows of a larger cache whose later rows
    hold NaN: the rows past the keys weigh nothing (finite LSE, out equal to
    the oracle's).  That no load touches them -- the last, ragged run is read
    as the 64-token window ending with the last key -- is checked for every
    lane and load on the CPU (test_decode_addresses.py); NaN there would
    show only if such a row were given weight."""
    B, Hq, Hkv, Skv, Smax = 32, 32, 8, 2000, 2048
    q = randn((B, Hq, 1, D), SEED + 160)
    kf, vf = randn((B, Hkv, Smax, D), SEED + 161), randn((B, Hkv, Smax, D), SEED + 162)
    kf[:, :, Skv:], vf[:, :, Skv:] = float("nan"), float("nan")
    k, v = kf.to(cuda)[:, :, :Skv], vf.to(cuda)[:, :, :Skv]
    out, lse = run(cuda, q, k, v, enable_gqa=True, return_lse=True)
    kc, vc = kf[:, :, :Skv], vf[:, :, :Skv]
    out = out.cpu()
    for b in range(B):
        assert_close(out[b:b + 1], OA.sdpa_cpu_fp32(q[b:b + 1], kc[b:b + 1], vc[b:b + 1]))
    assert torch.isfinite(lse.cpu()).all()


@pytest.mark.parametrize("B,Hq,Hkv,Skv,D", [(1, 32, 8, 4096, 128), (1, 8, 8, 3000, 64), (2, 16, 2, 1500, 64),
                                            (1, 4, 1, 257, 128), (1, 32, 1, 1000, 128), (3, 32, 2, 700, 64)])
def test_short_decode_split_merges_in_one_kernel(cuda, B, Hq, Hkv, Skv, D):
    """A key-split short decode (one row tile per (sequence, KV head), the
    keys over several blocks) merges inside its one kernel: the block that
    sees every split's arrival flag combines the partials.  The prepared
    call launches that one kernel; its workspace starts as random bytes and
    is shared with a call of another shape between calls; forty calls in a
    row give the same bits; outputs and LSE against the oracle."""
    import torch_spyre_amd as tsa
    from torch.profiler import ProfilerActivity, profile

    q = randn((B, Hq, 1, D), SEED + 110 + Skv)
    k, v = randn((B, Hkv, Skv, D), SEED + 111), randn((B, Hkv, Skv, D), SEED + 112)
    qo, ko, vo = randn((1, 8, 1, 128), SEED + 113), randn((1, 2, 2000, 128), SEED + 114), randn((1, 2, 2000, 128), SEED + 115)
    from torch_spyre_amd import _lib

    need = max(_lib.lib().spyre_sdpa_fwd_call_workspace_bytes(None, 0, None, B, Hq, Hkv, 1, Skv, D),
               _lib.lib().spyre_sdpa_fwd_call_workspace_bytes(None, 0, None, 1, 8, 2, 1, 2000, 128))
    assert need > 0
    ws = torch.randint(0, 256, (need,), dtype=torch.uint8, generator=torch.Generator().manual_seed(SEED + 116)).to(cuda)
    call = tsa.SdpaCall(q.to(cuda), k.to(cuda), v.to(cuda), enable_gqa=Hq != Hkv, return_lse=True, workspace=ws)
    other = tsa.SdpaCall(qo.to(cuda), ko.to(cuda), vo.to(cuda), enable_gqa=True, workspace=ws)
    first = [t.clone() for t in call()]
    with profile(activities=[ProfilerActivity.CUDA]) as prof:
        call()
        torch.cuda.synchronize(cuda)
    kernels = [e.name for e in prof.events() if e.device_type == torch.autograd.DeviceType.CUDA]
    assert len(kernels) == 1 and "sdpa_decode_short_kernel" in kernels[0], kernels
    for i in range(40):
        if i % 10 == 0:
            other()
        out, lse = call()
        assert torch.equal(out.view(torch.int16), first[0].view(torch.int16)), i
        assert torch.equal(lse, first[1]), i
    assert_close(first[0], OA.sdpa_cpu_fp32(q, k, v))
    _, lse64 = OA.sdpa_decomposition_fp64(q, k, v, return_lse=True)
    assert np.allclose(first[1].cpu().numpy(), lse64, atol=LSE_ATOL, rtol=0)
    assert_close(other(), OA.sdpa_cpu_fp32(qo, ko, vo))


@pytest.mark.parametrize("B,S", [(1, 4096), (4, 8192)], ids=str)
def test_decode_merges_in_kernel_on_two_streams(cuda, B, S):
    """Two decodes whose chunk partials merge inside the kernel -- batch 1
    (the short-decode kernel's key splits) and batch 4 x 8192 tokens (the
    split-KV decode kernel's chunks) -- in flight at once on two streams,
    each with its own workspace, twenty times over: every result bit-equal
    to the same call run alone."""
    import torch_spyre_amd as tsa

    calls, refs = [], []
    for i in range(2):
        q = randn((B, 32, 1, 128), SEED + 120 + i).to(cuda)
        k, v = randn((B, 8, S, 128), SEED + 122 + i).to(cuda), randn((B, 8, S, 128), SEED + 124 + i).to(cuda)
        c = tsa.SdpaCall(q, k, v, enable_gqa=True, return_lse=True)
        out, lse = c()
        calls.append(c)
        refs.append((out.clone(), lse.clone()))
    torch.cuda.synchronize(cuda)
    streams = [torch.cuda.Stream(device=cuda), torch.cuda.Stream(device=cuda)]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream(cuda))
    got = [[], []]
    for it in range(20):
        for i in (0, 1):
            with torch.cuda.stream(streams[i]):
                out, lse = calls[i]()
                got[i].append((out.clone(), lse.clone()))
    torch.cuda.synchronize(cuda)
    for i in (0, 1):
        for it, (out, lse) in enumerate(got[i]):
            assert torch.equal(out.view(torch.int16), refs[i][0].view(torch.int16)), (i, it)
            assert torch.equal(lse, refs[i][1]), (i, it)
