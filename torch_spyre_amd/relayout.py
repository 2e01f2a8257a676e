"""Stick relayout on the GPU: host order <-> device (stick) order, and
device-to-device restickify.

On MI355X there is no separate device memory to DMA into: "host" tensors are
ordinary strided CUDA tensors and "device" tensors are CUDA tensors whose
storage is in the stick layout.  The reference's DMA descriptors
(torch_spyre/csrc/spyre_mem.cpp:176-440) are computed by the native library
and executed by its HIP kernels (spyre_dma_copy).

A device tensor returned here has shape ``layout.device_size`` (contiguous)
and carries its layout and host geometry as attributes, read back with
``device_tensor_layout`` (the reference's Tensor.device_tensor_layout,
torch_spyre/_monkey_patch.py:63-71).
"""

from __future__ import annotations

import math
from typing import Optional, Sequence

import torch

from . import _lib
from .layout import SpyreTensorLayout, dma_plan, get_device_dtype, restick_plan


def _stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _require_cuda(t: torch.Tensor, name: str) -> None:
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be a CUDA (HIP) tensor; this package has no CPU path")


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
        esz = elem_bytes or src.element_size()
        sp, sb = _storage_span(src)
        dp, db = _storage_span(dst)
        self._infos = (_lib.StrideInfo * max(1, len(infos)))(*infos)
        self._args = (sp, sb, dp, db, esz, self._infos, len(infos))
        self._device = dst.device
        self._fn = _lib.lib().spyre_dma_copy

    def __call__(self) -> None:
        _lib.check("spyre_dma_copy", self._fn(*self._args, _stream_ptr(self._device)))


def _tag(t: torch.Tensor, layout: SpyreTensorLayout, size, stride) -> torch.Tensor:
    t._spyre_layout = layout
    t._spyre_host_size = [int(v) for v in size]
    t._spyre_host_stride = [int(v) for v in stride]
    return t


def device_tensor_layout(t: torch.Tensor) -> Optional[SpyreTensorLayout]:
    """Layout of a device tensor made by this module, else None."""
    return getattr(t, "_spyre_layout", None)


def spyre_empty_with_layout(size: Sequence[int], stride: Sequence[int], dtype: torch.dtype,
                            device_layout: SpyreTensorLayout, device=None, *,
                            zero: bool = True) -> torch.Tensor:
    """Allocates a device tensor for a host tensor of (size, stride) in
    ``device_layout``: max(stick bytes, host bytes), as
    torch_spyre/csrc/spyre_mem.cpp:547-579.  Zero-filled unless ``zero`` is
    False (padding positions are never written by the relayout)."""
    device = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    esz = torch.empty((), dtype=dtype).element_size()
    dev_bytes = device_layout.device_size_in_bytes()
    host_bytes = math.prod(int(v) for v in size) * esz
    ds = list(device_layout.device_size)
    if math.prod(ds) * esz == dev_bytes and dev_bytes >= host_bytes:
        shape = ds
    else:
        shape = [max(dev_bytes, host_bytes) // esz]
    t = (torch.zeros if zero else torch.empty)(shape, dtype=dtype, device=device)
    return _tag(t, device_layout, size, stride)


def _check_layout_dtype(dtype: torch.dtype, layout: SpyreTensorLayout) -> None:
    if get_device_dtype(dtype) != layout.device_dtype:
        raise TypeError(f"layout device dtype {layout.device_dtype} does not hold {dtype} "
                        "(relayout moves raw elements; no format conversion)")
    if torch.empty((), dtype=dtype).element_size() * layout.elems_per_stick() != 128:
        raise TypeError(f"{dtype} elements do not fill 128-byte sticks of {layout.device_dtype}")


def _covers_all(infos, layout: SpyreTensorLayout) -> bool:
    n = sum(math.prod(info.size[: info.rank]) for info in infos)
    return n >= math.prod(layout.device_size)


def to_device_layout(x: torch.Tensor, device_layout: SpyreTensorLayout) -> torch.Tensor:
    """x (any strides) -> new device tensor in ``device_layout``.

    The reference's ``Tensor.to(device_layout=stl)`` + ``copy_tensor``
    (torch_spyre/_monkey_patch.py:106-155, torch_spyre/csrc/spyre_mem.cpp:594-651):
    the device tensor keeps x's sizes and strides as its dma geometry."""
    _require_cuda(x, "x")
    _check_layout_dtype(x.dtype, device_layout)
    size, stride = list(x.size()), list(x.stride())
    if x.numel() == 0:  # nothing to move
        return spyre_empty_with_layout(size, stride, x.dtype, device_layout, x.device)
    infos = dma_plan(size, stride, stride, x.storage_offset(), device_layout, True)
    dst = spyre_empty_with_layout(size, stride, x.dtype, device_layout, x.device,
                                  zero=not _covers_all(infos, device_layout))
    dma_copy(x, dst, infos)
    return dst


def from_device_layout(dev: torch.Tensor, device_layout: Optional[SpyreTensorLayout] = None,
                       size: Optional[Sequence[int]] = None,
                       stride: Optional[Sequence[int]] = None) -> torch.Tensor:
    """Device tensor -> new strided tensor (the reference's ``.cpu()`` D2H,
    torch_spyre/csrc/spyre_mem.cpp:594-651).  Geometry defaults to what
    ``to_device_layout`` recorded; the result has those strides."""
    _require_cuda(dev, "dev")
    layout = device_layout or device_tensor_layout(dev)
    if layout is None:
        raise ValueError("dev carries no layout; pass device_layout")
    size = list(size if size is not None else dev._spyre_host_size)
    if stride is None:
        stride = getattr(dev, "_spyre_host_stride", None) if size == getattr(dev, "_spyre_host_size", None) else None
    stride = list(stride) if stride is not None else _contiguous_strides(size)
    _check_layout_dtype(dev.dtype, layout)
    out = torch.empty_strided(size, stride, dtype=dev.dtype, device=dev.device)
    if out.numel() == 0:
        return out
    dma_copy(dev, out, dma_plan(size, stride, stride, 0, layout, False))
    return out


def copy_tensor(src: torch.Tensor, dst: torch.Tensor) -> torch.Tensor:
    """The reference's _C.copy_tensor (torch_spyre/csrc/module.cpp:339-341):
    H2D when dst carries a layout, D2H when src does."""
    if device_tensor_layout(dst) is not None:
        lay = device_tensor_layout(dst)
        size, stride = list(src.size()), list(src.stride())
        dma_copy(src, dst, dma_plan(size, dst._spyre_host_stride, stride, src.storage_offset(), lay, True))
        return dst
    if device_tensor_layout(src) is not None:
        lay = device_tensor_layout(src)
        dma_copy(src, dst, dma_plan(list(dst.size()), src._spyre_host_stride, list(dst.stride()),
                                    dst.storage_offset(), lay, False))
        return dst
    raise ValueError("copy_tensor: neither tensor carries a device layout")


def restickify(dev: torch.Tensor, dst_layout: SpyreTensorLayout,
               src_layout: Optional[SpyreTensorLayout] = None,
               host_size: Optional[Sequence[int]] = None) -> torch.Tensor:
    """Device-to-device relayout of the same host tensor into ``dst_layout``
    (the reference's spyre::restickify, whose target layout is computed by
    torch_spyre/_inductor/pass_utils.py:749-833).  One pass when the two
    tilings nest; otherwise through a host-order buffer (two passes)."""
    _require_cuda(dev, "dev")
    src_layout = src_layout or device_tensor_layout(dev)
    if src_layout is None:
        raise ValueError("dev carries no layout; pass src_layout")
    size = list(host_size if host_size is not None else dev._spyre_host_size)
    _check_layout_dtype(dev.dtype, dst_layout)
    dense = getattr(dev, "_spyre_host_stride", _contiguous_strides(size)) == _contiguous_strides(size)
    info = restick_plan(size, src_layout, dst_layout) if dense else None
    if info is None:
        host = from_device_layout(dev, src_layout, size, _contiguous_strides(size))
        return to_device_layout(host, dst_layout)
    exact = math.prod(info.size[: info.rank]) >= math.prod(dst_layout.device_size)
    out = spyre_empty_with_layout(size, _contiguous_strides(size), dev.dtype, dst_layout, dev.device,
                                  zero=not exact)
    dma_copy(dev, out, [info])
    return out


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
