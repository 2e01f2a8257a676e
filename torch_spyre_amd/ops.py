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
The last four are defined and implemented in C++ (csrc/torch_ops.cpp); this
module gives them fake kernels.
"""

from __future__ import annotations

from typing import Optional, Sequence

import torch

from . import device_tensor, relayout
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


# spyre::kv_append, spyre::paged_decode_attention, spyre::sdpa_fwd and the
# CUDA kernel of aten::_scaled_dot_product_fused_attention_overrideable are
# C++ (csrc/torch_ops.cpp, loaded from libspyre_torch.so at import): they
# check, allocate and launch without a Python frame.  Their fake kernels
# (shapes only) make them traceable.

@torch.library.register_fake("spyre::kv_append")
def _(k_new, v_new, k_cache, v_cache, block_table, positions):
    return None


@torch.library.register_fake("spyre::paged_decode_attention")
def _(q, k_cache, v_cache, block_table, context_lens, scale, split_tokens=512, max_context_len=-1):
    return q.new_empty(q.shape), q.new_empty(q.shape[:2], dtype=torch.float32)


@torch.library.register_fake("spyre::sdpa_fwd")
def _(query, key, value, attn_mask=None, is_causal=False, scale=None, enable_gqa=False, return_lse=True):
    B, Hq, Sq, D = query.shape
    out = query.new_empty((B, Sq, Hq, D)).transpose(1, 2)
    return out, query.new_empty((B if return_lse else 0, Hq, Sq), dtype=torch.float32)


device_tensor.register_spyre_ops()

__all__ = ["relayout_op", "restickify", "copy_from_d2d", "to_device_layout", "from_device_layout", "overwrite",
           "overwrite_f", "DataFormats"]
