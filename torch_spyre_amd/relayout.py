"""Stick relayout on the GPU: host order <-> device (stick) order, and
device-to-device restickify.

On MI355X there is no separate device memory to DMA into: "host" tensors are
ordinary strided CUDA tensors and "device" tensors are CUDA tensors whose
storage is in the stick layout.  The reference's DMA descriptors
(torch_spyre/csrc/spyre_mem.cpp:176-440) are computed by the native library
and executed by its HIP kernels (spyre_dma_copy).

This module works on plain buffers: a buffer in stick order holds a host
geometry (sizes, strides) in a SpyreTensorLayout.  device_tensor.py builds
the Spyre tensor (logical geometry, views, copies) on top of it.
"""

from __future__ import annotations

import math
from typing import Optional, Sequence

import torch

from . import _lib
from .layout import SpyreTensorLayout, dma_plan, get_device_dtype, restick_plan


def _stream_ptr(device: torch.device) -> int:
    """The raw handle of the device's current stream (what
    ``torch.cuda.current_stream(device).cuda_stream`` returns, without
    building the Stream object: ~0.2 against ~1.9 µs per call)."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    return torch._C._cuda_getCurrentRawStream(idx)


def _require_cuda(t: torch.Tensor, name: str) -> None:
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be a CUDA (HIP) tensor; this package has no CPU path")


def _require_on(t: torch.Tensor, device: torch.device, name: str) -> None:
    """t must be a CUDA tensor on ``device``: a kernel launched there reads
    or writes it through its pointer."""
    if t.device != device:
        raise ValueError(f"{name} is on {t.device}; the call runs on {device} (no CPU path)")


def _contiguous_strides(size: Sequence[int]) -> list[int]:
    st, run = [0] * len(size), 1
    for i in range(len(size) - 1, -1, -1):
        st[i] = run
        run *= int(size[i])
    return st


def _storage_span(t: torch.Tensor) -> tuple[int, int]:
    """(base pointer, bytes) of the storage behind t."""
    s = t.untyped_storage()
    return s.data_ptr(), s.nbytes()


def dma_copy(src: torch.Tensor, dst: torch.Tensor, infos, elem_bytes: Optional[int] = None) -> None:
    """Runs DMA loop nests (offsets relative to each tensor's storage start)."""
    _require_cuda(dst, "dst")
    _require_on(src, dst.device, "src")
    if not infos:
        return
    esz = elem_bytes or src.element_size()
    sp, sb = _storage_span(src)
    dp, db = _storage_span(dst)
    arr = (_lib.StrideInfo * len(infos))(*infos)
    rc = _lib.lib().spyre_dma_copy(sp, sb, dp, db, esz, arr, len(infos), _stream_ptr(dst.device))
    _lib.check("spyre_dma_copy", rc)


class DmaCopy:
    """A validated ``dma_copy`` that can be launched repeatedly: the loop-nest
    array and the pointers are built once, each call only enters the library
    (the tensors must stay alive and keep their storage).  Each call launches
    on the stream current at that moment, so calls can be captured into a
    HIP graph."""

    def __init__(self, src: torch.Tensor, dst: torch.Tensor, infos, elem_bytes: Optional[int] = None):
        _require_cuda(dst, "dst")
        _require_on(src, dst.device, "src")
        esz = elem_bytes or src.element_size()
        sp, sb = _storage_span(src)
        dp, db = _storage_span(dst)
        self._infos = (_lib.StrideInfo * max(1, len(infos)))(*infos)
        self._args = (sp, sb, dp, db, esz, self._infos, len(infos))
        self._device = dst.device
        self._fn = _lib.lib().spyre_dma_copy

    def __call__(self) -> None:
        _lib.check("spyre_dma_copy", self._fn(*self._args, _stream_ptr(self._device)))


def alloc_bytes(size: Sequence[int], dtype: torch.dtype, layout: SpyreTensorLayout) -> int:
    """Allocation of a host tensor of ``size`` in ``layout``:
    max(128 x prod(device_size[:-1]), host bytes)
    (torch_spyre/csrc/spyre_mem.cpp:468-473, :547-579)."""
    esz = torch.empty((), dtype=dtype).element_size()
    return max(layout.device_size_in_bytes(), math.prod(int(v) for v in size) * esz)


def alloc_shape(size: Sequence[int], dtype: torch.dtype, layout: SpyreTensorLayout) -> list[int]:
    """Shape of the buffer holding that allocation: ``device_size`` when the
    allocation is exactly the layout's elements, else flat."""
    esz = torch.empty((), dtype=dtype).element_size()
    ds = list(layout.device_size)
    nbytes = alloc_bytes(size, dtype, layout)
    return ds if math.prod(ds) * esz == nbytes else [nbytes // esz]


def alloc_buffer(size: Sequence[int], dtype: torch.dtype, layout: SpyreTensorLayout, device,
                 zero: bool = True) -> torch.Tensor:
    return (torch.zeros if zero else torch.empty)(alloc_shape(size, dtype, layout), dtype=dtype, device=device)


def _check_layout_dtype(dtype: torch.dtype, layout: SpyreTensorLayout) -> None:
    if get_device_dtype(dtype) != layout.device_dtype:
        raise TypeError(f"layout device dtype {layout.device_dtype} does not hold {dtype} "
                        "(relayout moves raw elements; no format conversion)")
    if torch.empty((), dtype=dtype).element_size() * layout.elems_per_stick() != 128:
        raise TypeError(f"{dtype} elements do not fill 128-byte sticks of {layout.device_dtype}")


def _covers_all(infos, layout: SpyreTensorLayout) -> bool:
    n = sum(math.prod(info.size[: info.rank]) for info in infos)
    return n >= math.prod(layout.device_size)


def h2d_into(x: torch.Tensor, buf: torch.Tensor, layout: SpyreTensorLayout,
             dma_stride: Sequence[int]) -> None:
    """Writes host-order x (any strides) into ``buf`` in ``layout``, whose
    stride_map refers to a host geometry of x's sizes and ``dma_stride``."""
    _require_cuda(x, "x")
    _require_cuda(buf, "buf")
    _check_layout_dtype(x.dtype, layout)
    if x.numel() == 0:
        return
    dma_copy(x, buf, dma_plan(list(x.size()), list(dma_stride), list(x.stride()), x.storage_offset(), layout, True))


def h2d_buffer(x: torch.Tensor, layout: SpyreTensorLayout) -> torch.Tensor:
    """A new buffer holding x (any strides) in ``layout``, whose stride_map
    refers to x's own sizes and strides."""
    _require_cuda(x, "x")
    _check_layout_dtype(x.dtype, layout)
    size, stride = list(x.size()), list(x.stride())
    if x.numel() == 0:
        return alloc_buffer(size, x.dtype, layout, x.device)
    infos = dma_plan(size, stride, stride, x.storage_offset(), layout, True)
    buf = alloc_buffer(size, x.dtype, layout, x.device, zero=not _covers_all(infos, layout))
    dma_copy(x, buf, infos)
    return buf


def d2h_buffer(buf: torch.Tensor, layout: SpyreTensorLayout, size: Sequence[int],
               stride: Sequence[int]) -> torch.Tensor:
    """A new strided CUDA tensor of (size, stride) read from ``buf`` in
    ``layout`` (the DMA geometry the buffer was written with)."""
    _require_cuda(buf, "buf")
    _check_layout_dtype(buf.dtype, layout)
    size, stride = list(size), list(stride)
    out = torch.empty_strided(size, stride, dtype=buf.dtype, device=buf.device)
    if out.numel() == 0:
        return out
    dma_copy(buf, out, dma_plan(size, stride, stride, 0, layout, False))
    return out


def flat_plan(n: int) -> list:
    """The DMA nest of a contiguous copy of n elements."""
    info = _lib.StrideInfo()
    info.rank = 1
    info.size[0], info.stride_src[0], info.stride_dst[0] = n, 1, 1
    return [info]


def copy_buffer(src: torch.Tensor, dst: torch.Tensor) -> None:
    """dst <- src byte for byte (same allocation size): one flat DMA nest."""
    if src.untyped_storage().nbytes() != dst.untyped_storage().nbytes() or src.dtype != dst.dtype:
        raise ValueError("copy_buffer: allocations differ")
    n = src.untyped_storage().nbytes() // src.element_size()
    if n == 0:
        return
    dma_copy(src, dst, flat_plan(n))


def relayout_into(src: torch.Tensor, dst: torch.Tensor, host_size: Sequence[int], host_stride: Sequence[int],
                  src_layout: SpyreTensorLayout, dst_layout: SpyreTensorLayout) -> None:
    """dst (in dst_layout) <- src (in src_layout), both holding the host
    geometry (host_size, host_stride).  One pass when the geometry is dense
    and the two tilings nest (spyre_restick_plan); otherwise through host
    order (two passes)."""
    _require_cuda(src, "src")
    _require_cuda(dst, "dst")
    _check_layout_dtype(src.dtype, dst_layout)
    size, stride = list(host_size), list(host_stride)
    if math.prod(size) == 0:
        return
    info = restick_plan(size, src_layout, dst_layout) if stride == _contiguous_strides(size) else None
    if info is not None:
        dma_copy(src, dst, [info])
        return
    h2d_into(d2h_buffer(src, src_layout, size, stride), dst, dst_layout, stride)


def relayout_buffer(src: torch.Tensor, host_size: Sequence[int], host_stride: Sequence[int],
                    src_layout: SpyreTensorLayout, dst_layout: SpyreTensorLayout) -> torch.Tensor:
    """A new buffer holding src's host values in dst_layout (see
    ``relayout_into``); padding positions are zero."""
    size, stride = list(host_size), list(host_stride)
    if src_layout == dst_layout:  # the allocation byte for byte
        dst = alloc_buffer(size, src.dtype, dst_layout, src.device, zero=False)
        if dst.untyped_storage().nbytes() != src.untyped_storage().nbytes():
            raise ValueError("relayout: src is not an allocation of its layout")
        copy_buffer(src, dst)
        return dst
    info = restick_plan(size, src_layout, dst_layout) if stride == _contiguous_strides(size) else None
    exact = info is not None and math.prod(info.size[: info.rank]) >= math.prod(dst_layout.device_size)
    dst = alloc_buffer(size, src.dtype, dst_layout, src.device, zero=not exact)
    if info is not None:
        _check_layout_dtype(src.dtype, dst_layout)
        dma_copy(src, dst, [info])
    else:
        relayout_into(src, dst, size, stride, src_layout, dst_layout)
    return dst


def transpose_restick_layout(rows: int, cols: int, dtype=torch.float16) -> SpyreTensorLayout:
    """Layout of [rows, cols] with the stick on the row dim (dim_order [1, 0]):
    the sticks of the transposed matrix (torch_spyre/model_utils.py:111-138)."""
    return SpyreTensorLayout([rows, cols], [cols, 1], dtype, [1, 0])


def overwrite(input: torch.Tensor, output: torch.Tensor, dims: Sequence[int],
              offsets: Sequence[int]) -> None:
    """output.narrow(dims[i], offsets[i], input.size(dims[i])).copy_(input) for
    all i, as one loop nest on the GPU (the reference's spyre::overwrite,
    torch_spyre/_inductor/customops.py:260-308; its CPU kernel :298-308).
    Offsets are launch arguments, so no per-offset program is built."""
    _require_cuda(input, "input")
    _require_cuda(output, "output")
    if input.dtype != output.dtype:
        raise TypeError("overwrite: dtype mismatch")
    if input.dim() != output.dim():
        raise ValueError("overwrite: input and output ranks differ")
    if len(dims) != len(offsets):
        raise ValueError("overwrite: dims and offsets differ in length")
    off = output.storage_offset()
    for d, o in zip(dims, offsets):
        d = d % output.dim()
        if o < 0 or o + input.size(d) > output.size(d):
            raise IndexError(f"overwrite: offset {o} + {input.size(d)} exceeds dim {d} of size {output.size(d)}")
        off += o * output.stride(d)
    for d in range(input.dim()):
        if d not in [x % output.dim() for x in dims] and input.size(d) != output.size(d):
            raise ValueError(f"overwrite: size mismatch in dim {d}")
    if input.numel() == 0:
        return
    info = _lib.StrideInfo()
    r = max(1, input.dim())
    if r > _lib.SPYRE_MAX_RANK:
        raise ValueError("overwrite: rank too large")
    info.rank = r
    for q in range(input.dim()):
        k = input.dim() - 1 - q
        info.size[q] = input.size(k)
        info.stride_src[q] = input.stride(k)
        info.stride_dst[q] = output.stride(k)
    if input.dim() == 0:
        info.size[0], info.stride_src[0], info.stride_dst[0] = 1, 1, 1
    info.offset_src = input.storage_offset()
    info.offset_dst = off
    dma_copy(input, output, [info])
