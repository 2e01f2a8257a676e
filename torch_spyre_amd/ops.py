"""torch.library registrations of the ops on this path.

CUDA (HIP) kernels only: there is no CPU kernel and no fallback, so calling
an op on CPU tensors raises.  Fake kernels make the ops traceable.

  spyre::restickify(Tensor x) -> Tensor
        the reference's schema (torch_spyre/_inductor/customops.py:338-342);
        x is a SpyreTensor and the target layout comes out of band, as the
        reference's comes from the compiler's plan
        (torch_spyre/_inductor/ir.py:80-107, insert_restickify.py:139)
  spyre::relayout(src, host_size, host_stride, src_device_size, src_stride_map,
                  dst_device_size, dst_stride_map) -> Tensor
        the explicit companion on plain buffers (no reference counterpart)
  spyre::copy_from_d2d(Tensor src, Tensor(a!) dst) -> ()
        torch_spyre/_inductor/customops.py:240-257
  spyre::to_device_layout / spyre::from_device_layout
        Tensor.to(device_layout=) and the D2H copy on plain buffers
        (torch_spyre/_monkey_patch.py:106-155, torch_spyre/csrc/spyre_mem.cpp:594-651)
  spyre::overwrite / overwrite_f   torch_spyre/_inductor/customops.py:260-335 (overwrite_f
                              reinplaces to overwrite under torch.compile)
  spyre::kv_append            batched paged-cache write (no reference counterpart)
  spyre::paged_decode_attention    paged split-KV decode (no reference counterpart;
                              semantics of torch_spyre/_inductor/decompositions.py:523-609)
  spyre::sdpa_fwd             SDPA forward with logsumexp
  aten::_scaled_dot_product_fused_attention_overrideable (CUDA kernel)
        the reference's decomposition target (decompositions.py:523-609),
        returning its 9-tuple
"""

from __future__ import annotations

from typing import Optional, Sequence

import torch

from . import attention, device_tensor, relayout
from . import sdpa as _sdpa
from .layout import DataFormats, SpyreTensorLayout, get_device_dtype

_CUDA = ("cuda",)


def _layout(device_size, stride_map, dtype) -> SpyreTensorLayout:
    return SpyreTensorLayout(list(device_size), list(stride_map), get_device_dtype(dtype))


@torch.library.custom_op("spyre::relayout", mutates_args=(), device_types=_CUDA)
def relayout_op(src: torch.Tensor, host_size: Sequence[int], host_stride: Sequence[int],
                src_device_size: Sequence[int], src_stride_map: Sequence[int],
                dst_device_size: Sequence[int], dst_stride_map: Sequence[int]) -> torch.Tensor:
    """src, a buffer holding the host geometry (host_size, host_stride) in
    the source layout, moved to a new buffer in the destination layout."""
    return relayout.relayout_buffer(src, list(host_size), list(host_stride),
                                    _layout(src_device_size, src_stride_map, src.dtype),
                                    _layout(dst_device_size, dst_stride_map, src.dtype))


@relayout_op.register_fake
def _(src, host_size, host_stride, src_device_size, src_stride_map, dst_device_size, dst_stride_map):
    dst = _layout(dst_device_size, dst_stride_map, src.dtype)
    return src.new_empty(relayout.alloc_shape(list(host_size), src.dtype, dst))


@torch.library.custom_op("spyre::restickify", mutates_args=(), device_types=_CUDA)
def restickify(x: torch.Tensor) -> torch.Tensor:
    raise TypeError("spyre::restickify moves a tensor between Spyre device layouts: pass a SpyreTensor "
                    "(torch_spyre_amd.to_device_layout), or use spyre::relayout with explicit layouts "
                    "for a plain buffer")


@restickify.register_fake
def _(x):
    return torch.empty_like(x)


@torch.library.custom_op("spyre::copy_from_d2d", mutates_args=("dst",), device_types=_CUDA)
def copy_from_d2d(src: torch.Tensor, dst: torch.Tensor) -> None:
    """Plain CUDA tensors: dst <- src.  SpyreTensors (any layouts) are served
    by their dispatcher through the relayout kernels."""
    if src.shape != dst.shape or src.dtype != dst.dtype:
        raise ValueError("copy_from_d2d: src and dst differ in shape or dtype")
    dst.copy_(src)


@copy_from_d2d.register_fake
def _(src, dst):
    return None


@torch.library.custom_op("spyre::to_device_layout", mutates_args=(), device_types=_CUDA)
def to_device_layout(x: torch.Tensor, device_size: Sequence[int], stride_map: Sequence[int]) -> torch.Tensor:
    """x (any strides) -> a new buffer in the layout, whose stride_map refers
    to x's sizes and strides."""
    return relayout.h2d_buffer(x, _layout(device_size, stride_map, x.dtype))


@to_device_layout.register_fake
def _(x, device_size, stride_map):
    return x.new_empty(relayout.alloc_shape(list(x.shape), x.dtype, _layout(device_size, stride_map, x.dtype)))


@torch.library.custom_op("spyre::from_device_layout", mutates_args=(), device_types=_CUDA)
def from_device_layout(x: torch.Tensor, device_size: Sequence[int], stride_map: Sequence[int],
                       host_size: Sequence[int]) -> torch.Tensor:
    """A buffer in the layout of a contiguous host tensor of host_size ->
    that host tensor (contiguous)."""
    size = list(host_size)
    return relayout.d2h_buffer(x, _layout(device_size, stride_map, x.dtype), size,
                               relayout._contiguous_strides(size))


@from_device_layout.register_fake
def _(x, device_size, stride_map, host_size):
    return x.new_empty(list(host_size))


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


# Under torch.compile, inductor's reinplace pass turns overwrite_f into an
# in-place overwrite of its output argument (index 1) where that buffer is
# not read afterwards, so a compiled loop of token writes does not copy the
# cache per write: the reference's registration
# (torch_spyre/_inductor/customops.py:333-335).
from torch._inductor.fx_passes.reinplace import InplaceableOp, inplaceable_ops  # noqa: E402
from torch._inductor.lowering import fallback_handler, register_lowering  # noqa: E402

inplaceable_ops[torch.ops.spyre.overwrite_f.default] = InplaceableOp(torch.ops.spyre.overwrite.default, 1)


# The reinplace pass only retargets the node; its users still read the
# node's value.  As the reference's lowering does
# (torch_spyre/_inductor/lowering.py:786-800), the value of an overwrite is
# the output it wrote: the op runs as an extern kernel (the HIP relayout
# engine) and the lowering returns that buffer.
@register_lowering(torch.ops.spyre.overwrite.default, type_promotion_kind=None)
def _lower_overwrite(input, output, dims, offsets):
    fallback_handler(torch.ops.spyre.overwrite.default, add_to_fallback_set=False)(input, output, dims, offsets)
    return output


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


@torch.library.custom_op("spyre::sdpa_fwd", mutates_args=(), device_types=_CUDA)
def sdpa_fwd(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, attn_mask: Optional[torch.Tensor],
             is_causal: bool, scale: Optional[float], enable_gqa: bool) -> tuple[torch.Tensor, torch.Tensor]:
    """(out, lse); out has the strides of a contiguous [B, Sq, Hq, D] tensor."""
    return _sdpa.scaled_dot_product_attention(query, key, value, attn_mask=attn_mask, is_causal=is_causal,
                                              scale=scale, enable_gqa=enable_gqa, return_lse=True)


@sdpa_fwd.register_fake
def _(query, key, value, attn_mask, is_causal, scale, enable_gqa):
    B, Hq, Sq, D = query.shape
    out = query.new_empty((B, Sq, Hq, D)).transpose(1, 2)
    return out, query.new_empty((B, Hq, Sq), dtype=torch.float32)


# The reference decomposes aten::_scaled_dot_product_fused_attention_overrideable
# for its device (torch_spyre/_inductor/decompositions.py:523-609); here the op
# gets a CUDA kernel returning the same 9-tuple.  torch registers only a
# CompositeExplicitAutograd kernel for it, so this one serves CUDA tensors.
_ATEN_IMPL = torch.library.Library("aten", "IMPL")


def _sdpa_overrideable_cuda(query, key, value, attn_bias=None, dropout_p=0.0, is_causal=False,
                            return_debug_mask=False, *, scale=None):
    return _sdpa.sdpa_overrideable(query, key, value, attn_bias=attn_bias, dropout_p=dropout_p,
                                   is_causal=is_causal, return_debug_mask=return_debug_mask, scale=scale)


_ATEN_IMPL.impl("_scaled_dot_product_fused_attention_overrideable", _sdpa_overrideable_cuda, "CUDA")

device_tensor.register_spyre_ops()

__all__ = ["relayout_op", "restickify", "copy_from_d2d", "to_device_layout", "from_device_layout", "overwrite",
           "overwrite_f", "kv_append", "paged_decode_attention", "sdpa_fwd", "DataFormats"]
