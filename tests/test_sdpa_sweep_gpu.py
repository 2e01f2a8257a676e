"""GPU: a seeded sweep of SDPA shapes against the oracle, so that every
route the planner picks -- short decode, the split-KV decode kernels on
dense K / V (eight- and four-wavefront items, one and several chunks), the
LDS kernel with and without key splits, half steps, masks staged, copied or
through the fp32-mask kernel -- meets the parity bar on shapes no
hand-written case names.

Bar: fp16 outputs within |gpu - ref| <= 2e-3 + 1e-2 |ref| of torch's CPU fp32
SDPA; LSE within 2e-3 + 2e-4 |lse| of the fp64 logsumexp (the relative term
covers q * scale rounded to fp16 when |scale log2 e| <= 1).
"""

import random

import numpy as np
import pytest
import torch

from oracle import attention as OA
from tests.conftest import SEED

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2
LSE_ATOL, LSE_RTOL = 2e-3, 2e-4


def _close(got, ref, what):
    got, ref = got.float().cpu(), torch.as_tensor(ref).float().cpu()
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    assert not torch.isnan(got).any() and not torch.isnan(ref).any(), what
    err = (got - ref).abs()
    assert not (err > ATOL + RTOL * ref.abs()).any(), f"{what}: max abs err {err.max():.3e}"


def _lse_close(lse, q, k, v, scale, is_causal, mask, what):
    """LSE against the fp64 decomposition; a negative scale as |scale| on -q
    (the decomposition takes sqrt(scale))."""
    sign = -1.0 if scale is not None and scale < 0 else 1.0
    _, lse64 = OA.sdpa_decomposition_fp64(sign * q.double(), k, v, scale=None if scale is None else abs(scale),
                                          attn_mask=None if mask is None else mask.numpy(), is_causal=is_causal,
                                          return_lse=True)
    got = lse.cpu().double().numpy()
    assert np.allclose(got, lse64, atol=LSE_ATOL, rtol=LSE_RTOL), \
        f"{what}: max LSE err {np.abs(got - lse64).max():.3e}"


def _randn(shape, gen):
    return torch.randn(shape, generator=gen, dtype=torch.float32).half()


def _decode_shapes(n):
    rnd = random.Random(SEED + 900)
    out = []
    while len(out) < n:
        D = rnd.choice([64, 128])
        Hkv = rnd.choice([1, 2, 4, 8, 16])
        g = rnd.choice([1, 2, 4, 8])
        B = rnd.choice([1, 2, 3, 8, 24, 40, 64])
        Skv = rnd.choice([1, 7, 64, 65, 300, 1000, 2047, 2049, 4096, 5000])
        pad = rnd.choice([0, 0, 8, 64])
        if Hkv * g > 64 or B * Hkv * g * Skv > 400_000:  # keep the fp64 reference to seconds
            continue
        out.append((B, Hkv * g, Hkv, Skv, pad, D))
    return out


@pytest.mark.parametrize("B,Hq,Hkv,Skv,pad,D", _decode_shapes(28), ids=str)
def test_decode_sweep(cuda, B, Hq, Hkv, Skv, pad, D):
    """One query per sequence (the decode routes), K / V views with a padded
    token stride, every sequence against CPU fp32 SDPA and its LSE against
    the fp64 logsumexp."""
    import torch_spyre_amd as tsa

    gen = torch.Generator().manual_seed(SEED + B * 7919 + Hq * 31 + Skv)
    q = _randn((B, Hq, 1, D), gen)
    kf, vf = _randn((B, Hkv, Skv, D + pad), gen), _randn((B, Hkv, Skv, D + pad), gen)
    k, v = kf.to(cuda)[..., :D], vf.to(cuda)[..., :D]
    out, lse = tsa.scaled_dot_product_attention(q.to(cuda), k, v, enable_gqa=Hq != Hkv, return_lse=True)
    kc, vc = kf[..., :D], vf[..., :D]
    _close(out, OA.sdpa_cpu_fp32(q, kc, vc), "out")
    _lse_close(lse, q, kc, vc, None, False, None, "lse")


def _prefill_shapes(n):
    rnd = random.Random(SEED + 901)
    out = []
    while len(out) < n:
        D = rnd.choice([64, 128])
        Hkv = rnd.choice([1, 2, 4])
        g = rnd.choice([1, 2, 4])
        B = rnd.choice([1, 2])
        Sq = rnd.choice([2, 17, 33, 64, 129, 256, 300, 700])
        Skv = rnd.choice([1, 40, 64, 200, 511, 900])
        mask = rnd.choice([None, None, "causal", "f16", "bool", "f16_row", "bool_bcast", "f32"])
        scale = rnd.choice([None, None, 0.05, -0.1, 1.3])
        out.append((B, Hkv * g, Hkv, Sq, Skv, D, mask, scale))
    return out


@pytest.mark.parametrize("B,Hq,Hkv,Sq,Skv,D,mask,scale", _prefill_shapes(24), ids=str)
def test_prefill_sweep(cuda, B, Hq, Hkv, Sq, Skv, D, mask, scale):
    """Any-Sq SDPA: causal, fp16 / boolean / fp32 masks of full and broadcast
    shapes, scales inside and outside the prescaled range and negative, GQA;
    against CPU fp32 SDPA, LSE against the fp64 logsumexp."""
    import torch_spyre_amd as tsa

    gen = torch.Generator().manual_seed(SEED + Sq * 131 + Skv * 17 + Hq)
    q, k, v = _randn((B, Hq, Sq, D), gen), _randn((B, Hkv, Skv, D), gen), _randn((B, Hkv, Skv, D), gen)
    causal = mask == "causal"
    m = None
    if mask == "f16":
        m = torch.randn((B, Hq, Sq, Skv), generator=gen).half()
    elif mask == "f16_row":  # one bias row per key, broadcast over heads and queries
        m = torch.randn((1, 1, 1, Skv), generator=gen).half()
    elif mask == "f32":
        m = torch.randn((Sq, Skv), generator=gen)
    elif mask in ("bool", "bool_bcast"):
        shape = (B, Hq, Sq, Skv) if mask == "bool" else (B, 1, Sq, Skv)
        m = torch.rand(shape, generator=gen) < 0.6
        m[..., 0] = True  # every row sees a key
    out, lse = tsa.scaled_dot_product_attention(q.to(cuda), k.to(cuda), v.to(cuda),
                                                attn_mask=None if m is None else m.to(cuda), is_causal=causal,
                                                scale=scale, enable_gqa=Hq != Hkv, return_lse=True)
    _close(out, OA.sdpa_cpu_fp32(q, k, v, scale=scale, attn_mask=m, is_causal=causal), "out")
    _lse_close(lse, q, k, v, scale, causal, m, "lse")
