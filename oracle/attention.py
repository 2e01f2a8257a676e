"""Oracle: decode attention semantics.

Test infrastructure only (see ``oracle/__init__.py``).

* ``sdpa_decomposition_fp64`` restates the reference's SDPA decomposition
  (torch_spyre/_inductor/decompositions.py:546-609): sqrt(scale) applied to q
  and k (:552-558), GQA by expanding each KV head over its g query heads
  (:560-563), the causal bias triu(-inf, diagonal=1) over [Sq, Skv] (:567-570),
  the additive attention bias (:572-573), softmax over keys (:576), then P.V
  (:591).  Computed in fp64.  A boolean mask is first turned into an additive
  one (-inf where False), as torch does before it calls the overrideable op.
  ``return_lse`` adds the natural-log logsumexp of the biased scores (the
  reference returns an uninitialised tensor there, :584-586).
* ``sdpa_cpu_fp32`` is the reference's CPU eager path that its tests compare
  against (tests/inductor/utils_inductor.py:662; tests/inductor/test_inductor_ops.py:5386-5392):
  torch.nn.functional.scaled_dot_product_attention on fp32 CPU tensors (a
  causal call with a scale <= 0 as the explicit lower-triangular mask:
  torch's own is_causal path gives NaN there).
* ``gather_pages`` rebuilds per-sequence dense K/V from the paged stick
  layouts through ``oracle.layout`` (the layouts' own semantics).

Parity pins (tests/test_oracle_attention.py): the fp64 restatement agrees with
torch's CPU SDPA; closed cases: one key -> out = v; identical keys -> mean
of v; a one-hot score limit; GQA head mapping h -> h // g equals
repeat_interleave; the empty context gives zeros (torch's behaviour); a
negative scale equals |scale| on negated queries, its logsumexp scipy's.
"""

from __future__ import annotations

import math

import numpy as np
import torch

from . import layout as L

PAGE = 64


def additive_mask(attn_mask):
    """A boolean mask (True = attend) as the additive bias torch builds from
    it: 0 where True, -inf where False.  Float masks pass through."""
    m = np.asarray(attn_mask)
    if m.dtype == np.bool_:
        return np.where(m, 0.0, -np.inf)
    return m.astype(np.float64)


def sdpa_decomposition_fp64(q, k, v, scale=None, attn_mask=None, is_causal=False, return_lse=False):
    """q [B, Hq, Sq, D], k/v [B, Hkv, S, D] (numpy or torch) -> fp64 numpy
    [B, Hq, Sq, D] (and the logsumexp [B, Hq, Sq] with return_lse).  A row
    whose keys are all masked gives NaN, as torch.softmax does."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    B, Hq, Sq, D = q.shape
    Hkv = k.shape[1]
    s = 1.0 / math.sqrt(D) if scale is None else scale
    r = math.sqrt(s)
    q = q * r
    k = k * r
    g = Hq // Hkv
    if g != 1:
        k = np.repeat(k, g, axis=1)  # expand(...).flatten(1, 2): head h reads KV head h // g
        v = np.repeat(v, g, axis=1)
    if k.shape[2] == 0:
        out = np.zeros((B, Hq, Sq, D))
        return (out, np.full((B, Hq, Sq), -np.inf)) if return_lse else out
    att = q @ np.swapaxes(k, -1, -2)
    if is_causal:
        assert attn_mask is None
        att = att + np.triu(np.full(att.shape[-2:], -np.inf), 1)
    if attn_mask is not None:
        att = att + additive_mask(attn_mask)
    mx = att.max(axis=-1, keepdims=True)
    with np.errstate(invalid="ignore"):
        e = np.exp(att - mx)
        tot = e.sum(axis=-1, keepdims=True)
        out = (e / tot) @ v
    if not return_lse:
        return out
    with np.errstate(divide="ignore", invalid="ignore"):
        lse = (mx + np.log(tot))[..., 0]
    return out, lse


def decode_lse_fp64(q, k, scale=None):
    """The logsumexp of sdpa_decomposition_fp64 for one query token without
    a mask, without forming P.V or expanding K over the group: q [Hq, D],
    k [Hkv, S, D] -> [Hq] fp64.  The scale is applied to the score once
    (the decomposition's sqrt(s) on q and on k multiplies to s)."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    Hq, D = q.shape
    Hkv = k.shape[0]
    s = 1.0 / math.sqrt(D) if scale is None else scale
    g = Hq // Hkv
    out = np.empty(Hq)
    for h in range(Hkv):
        att = s * (q[h * g:(h + 1) * g] @ k[h].T)  # [g, S]
        mx = att.max(axis=1)
        out[h * g:(h + 1) * g] = mx + np.log(np.exp(att - mx[:, None]).sum(axis=1))
    return out


def sdpa_cpu_fp32(q, k, v, scale=None, attn_mask=None, is_causal=False) -> torch.Tensor:
    """torch CPU eager SDPA in fp32 (enable_gqa when Hq != Hkv).  Fully
    masked rows give zeros here (torch's safe softmax)."""
    q = torch.as_tensor(q).float().cpu()
    k = torch.as_tensor(k).float().cpu()
    v = torch.as_tensor(v).float().cpu()
    if attn_mask is not None:
        attn_mask = torch.as_tensor(attn_mask).cpu()
        if attn_mask.dtype != torch.bool:
            attn_mask = attn_mask.float()
    gqa = q.shape[1] != k.shape[1]
    if is_causal and scale is not None and scale <= 0:
        # torch's CPU is_causal path returns NaN for a scale of 0 or below;
        # its documented meaning, the top-left lower-triangular keep-mask,
        # goes through the mask path, which handles both.
        attn_mask = torch.ones(q.shape[-2], k.shape[-2], dtype=torch.bool).tril()
        is_causal = False
    return torch.nn.functional.scaled_dot_product_attention(q, k, v, attn_mask=attn_mask, is_causal=is_causal,
                                                            scale=scale, enable_gqa=gqa)


def k_page_layout(num_pages, Hkv, D) -> L.Layout:
    return L.Layout([num_pages, Hkv, D // 64, PAGE, 64], [Hkv * PAGE * D, PAGE * D, 64, D, 1])


def v_page_layout(num_pages, Hkv, D) -> L.Layout:
    return L.Layout([num_pages, Hkv, 1, D, PAGE], [Hkv * PAGE * D, PAGE * D, PAGE * D, 1, D])


def pages_to_logical(k_dev: np.ndarray, v_dev: np.ndarray, num_pages, Hkv, D):
    """Device-layout caches (flat or shaped raw arrays) -> logical pages
    [P, Hkv, 64, D] via the D2H DMA loop nests of the two page layouts."""
    sizes = [num_pages, Hkv, PAGE, D]
    k = L.d2h(np.ascontiguousarray(k_dev).reshape(-1), sizes, k_page_layout(num_pages, Hkv, D))
    v = L.d2h(np.ascontiguousarray(v_dev).reshape(-1), sizes, v_page_layout(num_pages, Hkv, D))
    return np.ascontiguousarray(k), np.ascontiguousarray(v)


def logical_to_pages(k_log: np.ndarray, v_log: np.ndarray):
    """Logical pages [P, Hkv, 64, D] -> device-layout caches (flat) via H2D."""
    P, Hkv, T, D = k_log.shape
    st = L.contiguous_strides([P, Hkv, T, D])
    k = L.h2d(np.ascontiguousarray(k_log).reshape(-1), [P, Hkv, T, D], st, 0, k_page_layout(P, Hkv, D))
    v = L.h2d(np.ascontiguousarray(v_log).reshape(-1), [P, Hkv, T, D], st, 0, v_page_layout(P, Hkv, D))
    return k, v


def gather_sequence(k_log: np.ndarray, v_log: np.ndarray, table_row, ctx: int):
    """Dense K/V [Hkv, ctx, D] of one sequence from logical pages."""
    n = (ctx + PAGE - 1) // PAGE
    idx = np.asarray(table_row[:n], dtype=np.int64)
    k = k_log[idx].transpose(1, 0, 2, 3).reshape(k_log.shape[1], n * PAGE, -1)[:, :ctx]
    v = v_log[idx].transpose(1, 0, 2, 3).reshape(v_log.shape[1], n * PAGE, -1)[:, :ctx]
    return k, v


def paged_decode_reference(q, k_log, v_log, block_table, ctx_lens, scale, rows=None):
    """fp32 CPU SDPA per sequence over gathered pages -> [len(rows), Hq, D] fp32 torch."""
    q = torch.as_tensor(q)
    rows = range(q.shape[0]) if rows is None else rows
    outs = []
    for b in rows:
        kb, vb = gather_sequence(k_log, v_log, block_table[b], int(ctx_lens[b]))
        o = sdpa_cpu_fp32(q[b][None, :, None, :], torch.from_numpy(np.ascontiguousarray(kb))[None],
                          torch.from_numpy(np.ascontiguousarray(vb))[None], scale=scale)
        outs.append(o[0, :, 0, :])
    return torch.stack(outs)
