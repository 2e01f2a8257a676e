"""Paged split-KV decode attention and the stick-layout paged KV cache.

The reference has no paged cache and no decode kernel: its SDPA is the
overrideable decomposition (torch_spyre/_inductor/decompositions.py:523-609,
selected by torch_spyre/csrc/attn_utils.cpp:22-37) and cache writes are
``spyre::overwrite`` (torch_spyre/_inductor/customops.py:260-308).  This
module keeps those semantics (softmax(scale q k^T) v, GQA q head h -> KV head
h // g, empty context -> zeros) and adds the paged decode entry point.

Page layouts, as SpyreTensorLayouts of the logical cache [num_pages, Hkv, 64, D]
(page, KV head, token, feature):
  K: device_size [P, Hkv, D/64, 64, 64], stride_map [Hkv*64*D, 64*D, 64, D, 1]
     -- sticks along D (default tiling of each page);
  V: device_size [P, Hkv, 1, D, 64],     stride_map [Hkv*64*D, 64*D, 64*D, 1, D]
     -- sticks along tokens (transpose-restick of each page).
Each (page, KV head) is 16 KiB contiguous in both.
"""

from __future__ import annotations

import math
from typing import Optional

import torch

from . import _lib
from .layout import DataFormats, SpyreTensorLayout
from .relayout import _require_cuda, _require_on, _stream_ptr, h2d_buffer

PAGE = 64
# Wavefronts per decode workgroup: a sequence is cut into chunks of at most
# CHUNK_WAVES * split_tokens tokens (one workgroup each); a call whose
# max_context_len fits one chunk runs a single kernel, longer ones add the
# merge pass.  Equal to kWaves in csrc/decode_attn.hip.
CHUNK_WAVES = 8


def decode_passes(B: int, Hq: int, Hkv: int, D: int, max_context_len: int, split_tokens: int = 512) -> int:
    """Kernels one decode call launches on the current device: 1 when every
    context fits one chunk or the chunks merge inside the split kernel (its
    work list fits one round of the device), else 2 (the merge pass
    combines the chunks)."""
    n = _lib.lib().spyre_paged_decode_attn_kernels(B, Hq, Hkv, D, max_context_len, split_tokens)
    _lib.check("spyre_paged_decode_attn_kernels", n if n < 0 else 0)
    return int(n)


def k_page_layout(num_pages: int, Hkv: int, D: int) -> SpyreTensorLayout:
    return SpyreTensorLayout([num_pages, Hkv, D // 64, PAGE, 64],
                             [Hkv * PAGE * D, PAGE * D, 64, D, 1], DataFormats.SEN169_FP16)


def v_page_layout(num_pages: int, Hkv: int, D: int) -> SpyreTensorLayout:
    return SpyreTensorLayout([num_pages, Hkv, 1, D, PAGE],
                             [Hkv * PAGE * D, PAGE * D, PAGE * D, 1, D], DataFormats.SEN169_FP16)


class PagedKVCache:
    """fp16 paged KV cache in the stick layouts above."""

    def __init__(self, num_pages: int, Hkv: int, D: int, device=None, zero: bool = True):
        if D not in (64, 128):
            raise ValueError("head_dim must be 64 or 128")
        device = device if device is not None else torch.device("cuda", torch.cuda.current_device())
        alloc = torch.zeros if zero else torch.empty
        self.num_pages, self.Hkv, self.D = num_pages, Hkv, D
        self.k = alloc((num_pages, Hkv, D // 64, PAGE, 64), dtype=torch.float16, device=device)
        self.v = alloc((num_pages, Hkv, D, PAGE), dtype=torch.float16, device=device)
        self.k_layout = k_page_layout(num_pages, Hkv, D)
        self.v_layout = v_page_layout(num_pages, Hkv, D)

    @classmethod
    def from_pages(cls, k_pages: torch.Tensor, v_pages: torch.Tensor) -> "PagedKVCache":
        """Builds the cache from logical pages [P, Hkv, 64, D] (token-major)
        with the relayout engine."""
        P, Hkv, T, D = k_pages.shape
        if T != PAGE or v_pages.shape != k_pages.shape:
            raise ValueError("pages must be [P, Hkv, 64, D] for both K and V")
        self = cls.__new__(cls)
        self.num_pages, self.Hkv, self.D = P, Hkv, D
        self.k_layout = k_page_layout(P, Hkv, D)
        self.v_layout = v_page_layout(P, Hkv, D)
        self.k = h2d_buffer(k_pages, self.k_layout).view(P, Hkv, D // 64, PAGE, 64)
        self.v = h2d_buffer(v_pages, self.v_layout).view(P, Hkv, D, PAGE)
        return self

    def append(self, k_new: torch.Tensor, v_new: torch.Tensor, block_table: torch.Tensor,
               positions: torch.Tensor) -> None:
        kv_append(k_new, v_new, self.k, self.v, block_table, positions)


def _check_cache(k_cache: torch.Tensor, v_cache: torch.Tensor, Hkv: int, D: int) -> int:
    for name, t in (("k_cache", k_cache), ("v_cache", v_cache)):
        _require_cuda(t, name)
        if t.dtype != torch.float16 or not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous float16")
    per_page = Hkv * D * PAGE
    if k_cache.numel() % per_page or k_cache.numel() != v_cache.numel():
        raise ValueError(f"caches must hold whole pages of {per_page} elements (Hkv={Hkv}, D={D})")
    if k_cache.dim() >= 2 and k_cache.shape[1] != Hkv:
        raise ValueError(f"k_cache has {k_cache.shape[1]} KV heads, expected {Hkv}")
    return k_cache.numel() // per_page


def kv_append(k_new: torch.Tensor, v_new: torch.Tensor, k_cache: torch.Tensor,
              v_cache: torch.Tensor, block_table: torch.Tensor, positions: torch.Tensor) -> None:
    """Writes token positions[b] of every sequence b (k_new/v_new [B, Hkv, D])
    into its page slot, in one launch.  positions[b] < 0 skips b.  The C++
    kernel of ``spyre::kv_append`` checks and launches."""
    try:
        _KV_APPEND(k_new, v_new, k_cache, v_cache, block_table, positions)
    except RuntimeError as e:
        raise _lib.library_error(e) from None


_KV_APPEND = torch.ops.spyre.kv_append.default
_PAGED_DECODE = torch.ops.spyre.paged_decode_attention.default


def workspace_bytes(B: int, Hq: int, Hkv: int, D: int, max_context_len: int, split_tokens: int = 512) -> int:
    return int(_lib.lib().spyre_paged_decode_attn_workspace_bytes(B, Hq, Hkv, D, max_context_len, split_tokens))


class _DecodeArgs:
    """Validated arguments shared by the decode entry points."""

    def __init__(self, q, k_cache, v_cache, block_table, context_lens, scale, split_tokens,
                 max_context_len, workspace):
        _require_cuda(q, "q")
        if q.dtype != torch.float16 or q.dim() != 3 or not q.is_contiguous():
            raise ValueError("q must be contiguous float16 [B, Hq, D]")
        B, Hq, D = q.shape
        Hkv = k_cache.shape[1]
        if Hq % Hkv:
            raise ValueError(f"Hq={Hq} is not a multiple of Hkv={Hkv}")
        self.num_pages = _check_cache(k_cache, v_cache, Hkv, D)
        for name, t in (("k_cache", k_cache), ("v_cache", v_cache), ("block_table", block_table),
                        ("context_lens", context_lens)):
            _require_on(t, q.device, name)
        if workspace is not None:
            _require_on(workspace, q.device, "workspace")
        if block_table.dtype != torch.int32 or block_table.dim() != 2 or block_table.shape[0] != B \
                or block_table.stride(1) != 1 or not block_table.is_cuda:
            raise ValueError("block_table must be a CUDA int32 [B, W] tensor with unit column stride")
        if context_lens.dtype != torch.int32 or context_lens.shape != (B,) or not context_lens.is_contiguous() \
                or not context_lens.is_cuda:
            raise ValueError("context_lens must be a contiguous CUDA int32 [B] tensor")
        if max_context_len is None:
            max_context_len = int(context_lens.max().item()) if B else 0
        if max_context_len > block_table.shape[1] * PAGE:
            raise ValueError(f"max_context_len {max_context_len} exceeds the block table's "
                             f"{block_table.shape[1]} pages")
        self.scale = 1.0 / math.sqrt(D) if scale is None else float(scale)
        need = workspace_bytes(B, Hq, Hkv, D, max_context_len, split_tokens)
        if workspace is None:
            workspace = torch.empty(max(need, 4), dtype=torch.uint8, device=q.device)
        elif workspace.numel() * workspace.element_size() < need:
            raise ValueError(f"workspace holds {workspace.numel() * workspace.element_size()} bytes, need {need}")
        self.q, self.k, self.v, self.table, self.lens = q, k_cache, v_cache, block_table, context_lens
        self.B, self.Hq, self.Hkv, self.D = B, Hq, Hkv, D
        self.max_ctx, self.split = max_context_len, split_tokens
        self.ws = workspace
        self.ws_bytes = workspace.numel() * workspace.element_size()
        self.stream = _stream_ptr(q.device)


def paged_decode_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                           block_table: torch.Tensor, context_lens: torch.Tensor,
                           scale: Optional[float] = None, split_tokens: int = 512,
                           max_context_len: Optional[int] = None,
                           workspace: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None,
                           return_lse: bool = False):
    """out[b, h] = softmax(scale * q[b, h] . K[b, h // g]^T) V[b, h // g] over
    the first context_lens[b] tokens of sequence b's pages.

    q [B, Hq, D] fp16; caches as PagedKVCache; block_table int32 [B, W];
    context_lens int32 [B].  ``max_context_len`` bounds every context (if
    omitted it is read from context_lens, which synchronises).  One kernel
    when max_context_len <= CHUNK_WAVES * split_tokens, else the split pass
    then the merge pass."""
    if workspace is None and out is None:  # the C++ kernel of spyre::paged_decode_attention
        if scale is None:
            scale = 1.0 / math.sqrt(q.shape[-1])
        try:
            o, lse = _PAGED_DECODE(q, k_cache, v_cache, block_table, context_lens, float(scale), split_tokens,
                                   -1 if max_context_len is None else int(max_context_len))
        except RuntimeError as e:
            raise _lib.library_error(e) from None
        return (o, lse) if return_lse else o
    a = _DecodeArgs(q, k_cache, v_cache, block_table, context_lens, scale, split_tokens,
                    max_context_len, workspace)
    if out is None:
        out = torch.empty_like(q)
    _require_on(out, q.device, "out")
    if out.shape != q.shape or out.dtype != q.dtype or not out.is_contiguous():
        raise ValueError("out must be contiguous and shaped like q")
    lse = torch.empty((a.B, a.Hq), dtype=torch.float32, device=q.device) if return_lse else None
    rc = _lib.lib().spyre_paged_decode_attn_f16(
        q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), block_table.data_ptr(),
        block_table.stride(0), context_lens.data_ptr(), out.data_ptr(),
        lse.data_ptr() if lse is not None else None, a.ws.data_ptr(), a.ws_bytes, a.B, a.Hq, a.Hkv,
        a.D, PAGE, a.num_pages, a.max_ctx, a.split, a.scale, a.stream)
    _lib.check("spyre_paged_decode_attn_f16", rc)
    return (out, lse) if return_lse else out


class PagedDecode:
    """A validated decode call that can be launched repeatedly.

    Checks shapes, dtypes and the workspace once; each launch then only
    passes the stored device pointers to the library (the tensors must stay
    alive and keep their storage).  ``__call__`` is the single-call entry
    (one kernel when max_context_len fits one chunk); ``split()`` and
    ``merge()`` launch the two passes separately (the split pass then
    writes every chunk's partial to the workspace).  Each launch goes to the
    stream current at that moment, so the calls can be captured into a HIP
    graph (the library allocates and clears nothing: the arrival flags of
    chunks merged in the kernel are cleared by the call that sets them)."""

    def __init__(self, q, k_cache, v_cache, block_table, context_lens, scale=None,
                 split_tokens: int = 512, max_context_len: Optional[int] = None, workspace=None,
                 out: Optional[torch.Tensor] = None, lse: Optional[torch.Tensor] = None):
        a = _DecodeArgs(q, k_cache, v_cache, block_table, context_lens, scale, split_tokens,
                        max_context_len, workspace)
        self.out = torch.empty_like(q) if out is None else out
        _require_on(self.out, q.device, "out")
        if lse is not None:
            _require_on(lse, q.device, "lse")
        if self.out.shape != q.shape or self.out.dtype != q.dtype or not self.out.is_contiguous():
            raise ValueError("out must be contiguous and shaped like q")
        if lse is not None and (lse.dtype != torch.float32 or lse.shape != (a.B, a.Hq)):
            raise ValueError("lse must be float32 [B, Hq]")
        self.lse = lse
        self._a = a
        self.passes = decode_passes(a.B, a.Hq, a.Hkv, a.D, a.max_ctx, a.split)
        if a.ws.data_ptr() % 16 and a.max_ctx > CHUNK_WAVES * a.split:
            self.passes = 2  # a workspace aligned to less than 16 bytes takes the merge pass
        L = _lib.lib()
        self._call_fn = L.spyre_paged_decode_attn_f16
        self._split_fn = L.spyre_paged_decode_attn_split_f16
        self._merge_fn = L.spyre_paged_decode_attn_merge_f16
        lse_ptr = lse.data_ptr() if lse is not None else None
        self._device = q.device
        self._call_args = (q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), block_table.data_ptr(),
                           block_table.stride(0), context_lens.data_ptr(), self.out.data_ptr(), lse_ptr,
                           a.ws.data_ptr(), a.ws_bytes, a.B, a.Hq, a.Hkv, a.D, PAGE, a.num_pages,
                           a.max_ctx, a.split, a.scale)
        self._split_args = (q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), block_table.data_ptr(),
                            block_table.stride(0), context_lens.data_ptr(), a.ws.data_ptr(), a.ws_bytes,
                            a.B, a.Hq, a.Hkv, a.D, PAGE, a.num_pages, a.max_ctx, a.split, a.scale)
        self._merge_args = (context_lens.data_ptr(), a.ws.data_ptr(), a.ws_bytes, self.out.data_ptr(),
                            lse_ptr, a.B, a.Hq, a.Hkv, a.D, a.max_ctx, a.split)

    def split(self) -> None:
        _lib.check("spyre_paged_decode_attn_split_f16",
                   self._split_fn(*self._split_args, _stream_ptr(self._device)))

    def merge(self) -> torch.Tensor:
        _lib.check("spyre_paged_decode_attn_merge_f16",
                   self._merge_fn(*self._merge_args, _stream_ptr(self._device)))
        return self.out

    def __call__(self) -> torch.Tensor:
        _lib.check("spyre_paged_decode_attn_f16", self._call_fn(*self._call_args, _stream_ptr(self._device)))
        return self.out


def paged_decode_split(q, k_cache, v_cache, block_table, context_lens, workspace: torch.Tensor,
                       scale: Optional[float] = None, split_tokens: int = 512,
                       max_context_len: Optional[int] = None) -> None:
    """Pass 1 only: every chunk's partial into ``workspace``."""
    a = _DecodeArgs(q, k_cache, v_cache, block_table, context_lens, scale, split_tokens,
                    max_context_len, workspace)
    rc = _lib.lib().spyre_paged_decode_attn_split_f16(
        q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), block_table.data_ptr(),
        block_table.stride(0), context_lens.data_ptr(), a.ws.data_ptr(), a.ws_bytes, a.B, a.Hq,
        a.Hkv, a.D, PAGE, a.num_pages, a.max_ctx, a.split, a.scale, a.stream)
    _lib.check("spyre_paged_decode_attn_split_f16", rc)


def paged_decode_merge(context_lens: torch.Tensor, workspace: torch.Tensor, out: torch.Tensor,
                       Hkv: int, max_context_len: int, split_tokens: int = 512,
                       lse: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Pass 2 only: combine the partials written by ``paged_decode_split``
    (same context_lens, max_context_len and split_tokens) into out [B, Hq, D]."""
    _require_cuda(out, "out")
    if out.dtype != torch.float16 or out.dim() != 3 or not out.is_contiguous():
        raise ValueError("out must be contiguous float16 [B, Hq, D]")
    B, Hq, D = out.shape
    _require_on(context_lens, out.device, "context_lens")
    _require_on(workspace, out.device, "workspace")
    if lse is not None:
        _require_on(lse, out.device, "lse")
    if context_lens.dtype != torch.int32 or context_lens.shape != (B,) or not context_lens.is_contiguous():
        raise ValueError("context_lens must be contiguous int32 [B]")
    if lse is not None and (lse.dtype != torch.float32 or lse.shape != (B, Hq) or not lse.is_contiguous()):
        raise ValueError("lse must be contiguous float32 [B, Hq]")
    rc = _lib.lib().spyre_paged_decode_attn_merge_f16(
        context_lens.data_ptr(), workspace.data_ptr(), workspace.numel() * workspace.element_size(),
        out.data_ptr(), lse.data_ptr() if lse is not None else None, B, Hq, Hkv, D,
        max_context_len, split_tokens, _stream_ptr(out.device))
    _lib.check("spyre_paged_decode_attn_merge_f16", rc)
    return out


def dense_to_pages(k: torch.Tensor, v: torch.Tensor) -> tuple[PagedKVCache, torch.Tensor]:
    """Dense K/V [B, Hkv, S, D] -> paged cache (sequence b's page p is page
    b*P + p) and its block table.  Each tensor is moved in one relayout pass:
    the strided view [B, P, Hkv, 64, D] of the dense tensor is laid out with
    the page layouts (K keeps its sticks on D, V is transpose-resticked onto
    tokens).  Tokens past S are zero."""
    B, Hkv, S, D = k.shape
    P = max(1, (S + PAGE - 1) // PAGE)
    S2 = P * PAGE
    if S2 != S:
        k = torch.nn.functional.pad(k, (0, 0, 0, S2 - S))
        v = torch.nn.functional.pad(v, (0, 0, 0, S2 - S))
    k, v = k.contiguous(), v.contiguous()
    k5 = k.view(B, Hkv, P, PAGE, D).permute(0, 2, 1, 3, 4)  # [B, P, Hkv, 64, D]
    v5 = v.view(B, Hkv, P, PAGE, D).permute(0, 2, 1, 3, 4)
    k_lay = SpyreTensorLayout([B, P, Hkv, D // 64, PAGE, 64],
                              [Hkv * S2 * D, PAGE * D, S2 * D, 64, D, 1], DataFormats.SEN169_FP16)
    v_lay = SpyreTensorLayout([B, P, Hkv, 1, D, PAGE],
                              [Hkv * S2 * D, PAGE * D, S2 * D, PAGE * D, 1, D], DataFormats.SEN169_FP16)
    cache = PagedKVCache.__new__(PagedKVCache)
    cache.num_pages, cache.Hkv, cache.D = B * P, Hkv, D
    cache.k_layout = k_page_layout(B * P, Hkv, D)
    cache.v_layout = v_page_layout(B * P, Hkv, D)
    cache.k = h2d_buffer(k5, k_lay).view(B * P, Hkv, D // 64, PAGE, 64)
    cache.v = h2d_buffer(v5, v_lay).view(B * P, Hkv, D, PAGE)
    table = torch.arange(B * P, dtype=torch.int32, device=k.device).view(B, P)
    return cache, table


def sdpa_decode(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                scale: Optional[float] = None, enable_gqa: bool = False) -> torch.Tensor:
    """F.scaled_dot_product_attention for one query token (Sq == 1), no mask,
    no dropout: query [B, Hq, 1, D], key/value [B, Hkv, S, D] fp16 ->
    [B, Hq, 1, D].  The reference serves decode through the same overrideable
    SDPA op as prefill (torch_spyre/_inductor/decompositions.py:523-609), and
    so does this: the SDPA forward kernels with Sq = 1.  Paged caches use
    ``paged_decode_attention``."""
    if query.dim() != 4 or query.shape[2] != 1:
        raise ValueError("sdpa_decode handles exactly one query token: query [B, Hq, 1, D]")
    f16 = torch.float16
    if query.dtype != f16 or key.dtype != f16 or value.dtype != f16:
        query, key, value = query.to(f16), key.to(f16), value.to(f16)
    try:  # the C++ kernel of spyre::sdpa_fwd, without the logsumexp
        return _SDPA_FWD(query, key, value, None, False, scale, enable_gqa, False)[0]
    except RuntimeError as e:
        raise _lib.library_error(e) from None


_SDPA_FWD = torch.ops.spyre.sdpa_fwd.default
