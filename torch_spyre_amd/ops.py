"""torch.library registrations of the ``spyre::`` ops on this path.

CUDA (HIP) kernels only: there is no CPU kernel and no fallback, so calling
an op on CPU tensors raises.  Fake kernels make the ops traceable.

  spyre::restickify           torch_spyre/_inductor/customops.py:338-342 (layouts
                              explicit here; the reference carries them in IR,
                              torch_spyre/_inductor/ir.py:80-107)
  spyre::to_device_layout     Tensor.to(device_layout=) (torch_spyre/_monkey_patch.py:106-155)
  spyre::from_device_layout   device -> host copy (torch_spyre/csrc/spyre_mem.cpp:594-651)
  spyre::overwrite / overwrite_f   torch_spyre/_inductor/customops.py:260-335
  spyre::kv_append            batched paged-cache write (no reference counterpart)
  spyre::paged_decode_attention    paged split-KV decode (no reference counterpart;
                              semantics of torch_spyre/_inductor/decompositions.py:523-609)
  spyre::sdpa_fwd             SDPA forward with logsumexp (the overrideable op's
                              decomposition, torch_spyre/_inductor/decompositions.py:523-609)
"""

from __future__ import annotations

import math
from typing import Optional, Sequence

import torch

from . import attention, relayout
from . import sdpa as _sdpa
from .layout import DataFormats, SpyreTensorLayout, get_device_dtype

_CUDA = ("cuda",)


def _layout(device_size, stride_map, dtype) -> SpyreTensorLayout:
    return SpyreTensorLayout(list(device_size), list(stride_map), get_device_dtype(dtype))


@torch.library.custom_op("spyre::to_device_layout", mutates_args=(), device_types=_CUDA)
def to_device_layout(x: torch.Tensor, device_size: Sequence[int], stride_map: Sequence[int]) -> torch.Tensor:
    return relayout.to_device_layout(x, _layout(device_size, stride_map, x.dtype)).clone()


@to_device_layout.register_fake
def _(x, device_size, stride_map):
    return x.new_empty(list(device_size))


@torch.library.custom_op("spyre::from_device_layout", mutates_args=(), device_types=_CUDA)
def from_device_layout(x: torch.Tensor, device_size: Sequence[int], stride_map: Sequence[int],
                       host_size: Sequence[int]) -> torch.Tensor:
    return relayout.from_device_layout(x, _layout(device_size, stride_map, x.dtype), list(host_size))


@from_device_layout.register_fake
def _(x, device_size, stride_map, host_size):
    return x.new_empty(list(host_size))


@torch.library.custom_op("spyre::restickify", mutates_args=(), device_types=_CUDA)
def restickify(x: torch.Tensor, host_size: Sequence[int], src_device_size: Sequence[int],
               src_stride_map: Sequence[int], dst_device_size: Sequence[int],
               dst_stride_map: Sequence[int]) -> torch.Tensor:
    src = _layout(src_device_size, src_stride_map, x.dtype)
    dst = _layout(dst_device_size, dst_stride_map, x.dtype)
    out = relayout.restickify(x, dst, src_layout=src, host_size=list(host_size))
    return out.view(list(dst_device_size)) if out.numel() == math.prod(dst_device_size) else out


@restickify.register_fake
def _(x, host_size, src_device_size, src_stride_map, dst_device_size, dst_stride_map):
    return x.new_empty(list(dst_device_size))


@torch.library.custom_op("spyre::overwrite", mutates_args=("output",), device_types=_CUDA)
def overwrite(input: torch.Tensor, output: torch.Tensor, dims: Sequence[int], offsets: Sequence[int]) -> None:
    relayout.overwrite(input, output, list(dims), list(offsets))


@overwrite.register_fake
def _(input, output, dims, offsets):
    return None


@torch.library.custom_op("spyre::overwrite_f", mutates_args=(), device_types=_CUDA)
def overwrite_f(input: torch.Tensor, output: torch.Tensor, dims: Sequence[int],
                offsets: Sequence[int]) -> torch.Tensor:
    result = output.clone()
    relayout.overwrite(input, result, list(dims), list(offsets))
    return result


@overwrite_f.register_fake
def _(input, output, dims, offsets):
    return output.clone()


@torch.library.custom_op("spyre::kv_append", mutates_args=("k_cache", "v_cache"), device_types=_CUDA)
def kv_append(k_new: torch.Tensor, v_new: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
              block_table: torch.Tensor, positions: torch.Tensor) -> None:
    attention.kv_append(k_new, v_new, k_cache, v_cache, block_table, positions)


@kv_append.register_fake
def _(k_new, v_new, k_cache, v_cache, block_table, positions):
    return None


@torch.library.custom_op("spyre::paged_decode_attention", mutates_args=(), device_types=_CUDA)
def paged_decode_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                           block_table: torch.Tensor, context_lens: torch.Tensor, scale: float,
                           split_tokens: int = 512, max_context_len: int = -1) -> tuple[torch.Tensor, torch.Tensor]:
    out, lse = attention.paged_decode_attention(
        q, k_cache, v_cache, block_table, context_lens, scale=scale, split_tokens=split_tokens,
        max_context_len=None if max_context_len < 0 else max_context_len, return_lse=True)
    return out, lse


@paged_decode_attention.register_fake
def _(q, k_cache, v_cache, block_table, context_lens, scale, split_tokens=512, max_context_len=-1):
    return q.new_empty(q.shape), q.new_empty(q.shape[:2], dtype=torch.float32)


__all__ = ["to_device_layout", "from_device_layout", "restickify", "overwrite", "overwrite_f",
           "kv_append", "paged_decode_attention", "DataFormats"]


@torch.library.custom_op("spyre::sdpa_fwd", mutates_args=(), device_types=_CUDA)
def sdpa_fwd(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, attn_mask: Optional[torch.Tensor],
             is_causal: bool, scale: Optional[float], enable_gqa: bool) -> tuple[torch.Tensor, torch.Tensor]:
    out, lse = _sdpa.scaled_dot_product_attention(query, key, value, attn_mask=attn_mask, is_causal=is_causal,
                                                   scale=scale, enable_gqa=enable_gqa, return_lse=True)
    return out.clone(), lse


@sdpa_fwd.register_fake
def _(query, key, value, attn_mask, is_causal, scale, enable_gqa):
    B, Hq, Sq, D = query.shape
    out = query.new_empty((B, Sq, Hq, D)).transpose(1, 2)
    return out, query.new_empty((B, Hq, Sq), dtype=torch.float32)
