"""Tensors held in a Spyre stick layout on the GPU.

The reference's Spyre tensor (SpyreTensorImpl, torch_spyre/csrc/spyre_tensor_impl.h:140-160)
has host (logical) sizes, strides and storage offset, a SpyreTensorLayout
that says where each element sits in the device allocation, and the host
geometry the allocation was written with (``dma_sizes`` / ``dma_strides``).
Views (transpose, slices, expand, reshape) change only the logical geometry;
copies back to host order move the recorded geometry whole and apply the
view afterwards (torch_spyre/csrc/spyre_mem.cpp:594-651).

``SpyreTensor`` is that tensor on MI355X: a wrapper subclass whose size /
stride / storage_offset are the logical ones and whose bytes live in a
plain CUDA buffer (``device_buffer(t)``) in stick order.  Every byte moves
through the relayout kernels of libspyre_hip.so (spyre_dma_copy); the
dispatcher serves

* view ops (geometry computed on a meta twin, buffer and layout shared);
* ``.cpu()`` / ``.to("cpu")`` (D2H), ``copy_`` in every direction (H2D,
  D2H, D2D between layouts), ``clone``, ``index_copy_``; a view that is a
  box of the allocation (slices, selects, permuted dims) moves only its own
  elements;
* ``spyre::restickify(x)`` (the reference's one-tensor schema,
  torch_spyre/_inductor/customops.py:338-342) and ``spyre::copy_from_d2d``
  (:240-257).

Other ops raise: the reference runs them as compiled device programs,
which are not part of this path.
"""

from __future__ import annotations

import math
from typing import Optional, Sequence

import torch
from torch.utils.weak import WeakIdKeyDictionary

from . import relayout as R
from .layout import SpyreTensorLayout
from .relayout import _contiguous_strides, _require_cuda

aten = torch.ops.aten


def _span(size: Sequence[int], stride: Sequence[int]) -> int:
    """Elements a storage needs for (size, stride) at offset 0."""
    if any(int(s) == 0 for s in size):
        return 0
    return 1 + sum((int(s) - 1) * int(st) for s, st in zip(size, stride))


class SpyreTensor(torch.Tensor):
    """A tensor in a Spyre device layout (see the module docstring).

    ``_data``: the CUDA buffer (stick order; ``device_size``-shaped when the
    allocation is exactly the layout's bytes, else flat); ``_layout``: its
    SpyreTensorLayout; ``_dma_size`` / ``_dma_stride``: the host geometry
    the buffer was written with.  The tensor's own size / stride /
    storage_offset index that geometry's element space."""

    _data: torch.Tensor
    _layout: SpyreTensorLayout
    _dma_size: tuple
    _dma_stride: tuple

    @staticmethod
    def __new__(cls, data: torch.Tensor, layout: SpyreTensorLayout, dma_size: Sequence[int],
                dma_stride: Sequence[int], size: Optional[Sequence[int]] = None,
                stride: Optional[Sequence[int]] = None, storage_offset: int = 0):
        size = list(dma_size) if size is None else list(size)
        stride = list(dma_stride) if stride is None else list(stride)
        # The wrapper's own storage reports the allocation's size (it holds
        # no data: the bytes are data's), as the reference's storage is the
        # device allocation (tests/test_spyre.py:384-393 checks its size).
        r = torch.Tensor._make_wrapper_subclass(cls, size, strides=stride, storage_offset=int(storage_offset),
                                                dtype=data.dtype, device=data.device, requires_grad=False,
                                                storage_size=data.untyped_storage().nbytes())
        r._data = data
        r._layout = layout
        r._dma_size = tuple(int(v) for v in dma_size)
        r._dma_stride = tuple(int(v) for v in dma_stride)
        return r

    __torch_function__ = torch._C._disabled_torch_function_impl

    # Tracing (fake tensors, torch.compile) sees the buffer as the inner
    # tensor and the layout and geometries as constants.
    def __tensor_flatten__(self):
        return ["_data"], (self._layout, self._dma_size, self._dma_stride, self.storage_offset())

    @staticmethod
    def __tensor_unflatten__(inner, ctx, outer_size, outer_stride):
        layout, dma_size, dma_stride, offset = ctx
        return SpyreTensor(inner["_data"], layout, dma_size, dma_stride, outer_size, outer_stride, offset)

    def __repr__(self) -> str:
        return (f"SpyreTensor(size={list(self.shape)}, stride={list(self.stride())}, "
                f"storage_offset={self.storage_offset()}, dtype={self.dtype}, device={self.device}, "
                f"layout={self._layout})")

    def data_ptr(self) -> int:
        return self._data.data_ptr()

    def device_tensor_layout(self) -> SpyreTensorLayout:
        return self._layout

    def is_base(self) -> bool:
        """True when the logical geometry is the recorded DMA geometry."""
        return (tuple(self.shape) == self._dma_size and tuple(self.stride()) == self._dma_stride
                and self.storage_offset() == 0)

    def _with_view(self, size, stride, offset) -> "SpyreTensor":
        return SpyreTensor(self._data, self._layout, self._dma_size, self._dma_stride, size, stride, offset)

    def _meta(self) -> torch.Tensor:
        """A meta tensor with this tensor's geometry over the DMA geometry's
        element space, for computing the geometry of views."""
        n = max(_span(self._dma_size, self._dma_stride), self.storage_offset() + _span(self.shape, self.stride()), 1)
        return torch.empty(n, dtype=self.dtype, device="meta").as_strided(
            self.shape, self.stride(), self.storage_offset())

    @classmethod
    def __torch_dispatch__(cls, func, types, args=(), kwargs=None):
        kwargs = kwargs or {}
        handler = _HANDLERS.get(func)
        if handler is not None:
            return handler(*args, **kwargs)
        if getattr(func, "is_view", False):
            return _view(func, args, kwargs)
        raise NotImplementedError(
            f"{func} is not available on SpyreTensor: Spyre device tensors support views, copies "
            "(cpu(), copy_, clone) and the spyre:: ops; move the values to host order with "
            "from_device_layout() for other work")


# ------------------------------------------------------------ construction --

def _default_layout(size: Sequence[int], stride: Sequence[int], dtype: torch.dtype) -> SpyreTensorLayout:
    """The layout spyre_empty_strided gives (torch_spyre/csrc/spyre_mem.cpp:508-516):
    the generic stick dim order 0..r-1 over the host strides."""
    if len(size) == 0:
        return SpyreTensorLayout([1], dtype)
    return SpyreTensorLayout(list(size), list(stride), dtype, list(range(len(size))))


def spyre_empty_with_layout(size: Sequence[int], stride: Sequence[int], dtype: torch.dtype,
                            device_layout: SpyreTensorLayout, device=None, *,
                            zero: bool = True) -> SpyreTensor:
    """A SpyreTensor of host geometry (size, stride) in ``device_layout``:
    max(128 x prod(device_size[:-1]), host bytes), as
    torch_spyre/csrc/spyre_mem.cpp:547-579.  Zero-filled unless ``zero`` is
    False (the relayout never writes padding positions)."""
    device = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    data = R.alloc_buffer(size, dtype, device_layout, device, zero=zero)
    return SpyreTensor(data, device_layout, size, stride)


def to_device_layout(x: torch.Tensor, device_layout: Optional[SpyreTensorLayout] = None) -> SpyreTensor:
    """x -> a new SpyreTensor in ``device_layout`` (default: the generic
    layout of x's sizes and strides, as ``x.to("spyre")``).

    The reference's ``Tensor.to(device_layout=stl)`` (torch_spyre/_monkey_patch.py:106-155):
    from host order (any strides; CPU tensors are first moved to the GPU)
    the DMA writes x's elements in the layout and the result keeps x's sizes
    and strides as its DMA geometry; from a SpyreTensor it is a
    device-to-device relayout (``copy_from_d2d``), or x itself when the
    layout is already ``device_layout``."""
    if isinstance(x, SpyreTensor):
        if device_layout is None or device_layout == x._layout:
            return x
        dst = spyre_empty_with_layout(list(x.shape), _contiguous_strides(x.shape), x.dtype, device_layout,
                                      x.device, zero=True)
        _copy_d2d(dst, x)
        return dst
    if not x.is_cuda:
        x = x.to(torch.device("cuda", torch.cuda.current_device()))
    size, stride = list(x.size()), list(x.stride())
    layout = device_layout if device_layout is not None else _default_layout(size, stride, x.dtype)
    return SpyreTensor(R.h2d_buffer(x, layout), layout, size, stride)


def from_device_layout(dev: torch.Tensor, device_layout: Optional[SpyreTensorLayout] = None,
                       size: Optional[Sequence[int]] = None,
                       stride: Optional[Sequence[int]] = None) -> torch.Tensor:
    """Device -> host order, as a CUDA tensor (the reference's D2H,
    torch_spyre/csrc/spyre_mem.cpp:594-651).

    For a SpyreTensor (no other argument): its logical values.  A base
    tensor is moved straight into its own strides; a view (expanded,
    strided, sliced, transposed) moves the whole recorded DMA geometry and
    then applies the view, so stride-0 dims and offsets read what the
    reference's do.  The result keeps the view's strides when they are
    dense and non-overlapping, else it is contiguous.

    For a plain buffer in stick order: ``device_layout`` and the host
    ``size`` (and ``stride``, default contiguous) are required."""
    if isinstance(dev, SpyreTensor):
        if device_layout is not None or size is not None or stride is not None:
            raise ValueError("a SpyreTensor carries its own layout and geometry")
        return _d2h(dev)
    if device_layout is None or size is None:
        raise ValueError("a plain device buffer needs device_layout and size")
    size = list(size)
    stride = list(stride) if stride is not None else _contiguous_strides(size)
    return R.d2h_buffer(dev, device_layout, size, stride)


def device_tensor_layout(t: torch.Tensor) -> Optional[SpyreTensorLayout]:
    """The layout of a SpyreTensor, else None (the reference's
    Tensor.device_tensor_layout, torch_spyre/_monkey_patch.py:63-71)."""
    return t._layout if isinstance(t, SpyreTensor) else None


def device_buffer(t: SpyreTensor) -> torch.Tensor:
    """The CUDA buffer behind a SpyreTensor: its bytes in stick order."""
    if not isinstance(t, SpyreTensor):
        raise TypeError("device_buffer takes a SpyreTensor")
    return t._data


def _relabel(x: SpyreTensor, size, stride, offset: int, layout: SpyreTensorLayout) -> SpyreTensor:
    """x's allocation seen with (size, stride, offset) in ``layout``: the
    DMA geometry stays x's when the layout does, else it becomes (size,
    stride) (torch_spyre/csrc/spyre_views.cpp:137-143, :168-174)."""
    if not isinstance(x, SpyreTensor):
        raise TypeError("expected a SpyreTensor")
    if not isinstance(layout, SpyreTensorLayout):
        raise TypeError("device_layout must be a SpyreTensorLayout")
    size, stride = [int(v) for v in size], [int(v) for v in stride]
    if len(size) != len(stride):
        raise ValueError("size and stride differ in length")
    if layout == x._layout:
        return SpyreTensor(x._data, layout, x._dma_size, x._dma_stride, size, stride, int(offset))
    need = R.alloc_bytes(size, x.dtype, layout)
    have = x._data.untyped_storage().nbytes()
    if need > have:
        raise ValueError(f"the allocation holds {have} bytes; {list(size)} in {layout} needs {need}")
    return SpyreTensor(x._data, layout, size, stride, size, stride, int(offset))


def as_strided_with_layout(x: SpyreTensor, size: Sequence[int], stride: Sequence[int],
                           storage_offset: Optional[int], device_layout: SpyreTensorLayout) -> SpyreTensor:
    """A view of x's allocation with (size, stride, storage_offset -- x's
    when None) in ``device_layout`` (torch_spyre/csrc/spyre_views.cpp:123-146,
    bound at torch_spyre/csrc/module.cpp:290)."""
    off = x.storage_offset() if storage_offset is None else int(storage_offset)
    return _relabel(x, size, stride, off, device_layout)


def reinterpret_tensor(x: SpyreTensor, size: Sequence[int], stride: Sequence[int],
                       offset_increment: int = 0) -> SpyreTensor:
    """x's allocation as (size, stride) at x's offset + offset_increment, in
    x's layout (torch_spyre/csrc/spyre_views.cpp:148-157)."""
    return reinterpret_tensor_with_layout(x, size, stride, offset_increment, x._layout)


def reinterpret_tensor_with_layout(x: SpyreTensor, size: Sequence[int], stride: Sequence[int],
                                   offset_increment: int, stl: SpyreTensorLayout) -> SpyreTensor:
    """x's allocation as (size, stride) at x's offset + offset_increment in
    layout ``stl``: the reference's buffer reuse in generated code
    (torch_spyre/csrc/spyre_views.cpp:159-181, emitted by
    torch_spyre/_inductor/wrapper.py:149)."""
    return _relabel(x, size, stride, x.storage_offset() + int(offset_increment), stl)


# ----------------------------------------------------------------- copies --

def _d2h_base(t: SpyreTensor) -> torch.Tensor:
    """The whole recorded DMA geometry in host order (a strided CUDA tensor
    whose storage the logical view indexes)."""
    return R.d2h_buffer(t._data, t._layout, list(t._dma_size), list(t._dma_stride))


def _d2h(t: SpyreTensor) -> torch.Tensor:
    if t.is_base():
        return _d2h_base(t)
    # the view's strides when they are dense and non-overlapping, as clone()
    # keeps them; else contiguous
    out = torch.empty_like(t._meta(), device=t.device)
    if t.numel() == 0:
        return out
    infos = _box_infos(t, out, host2device=False)
    if infos is not None:  # a box: its own elements only
        _run_infos(t._data, out, infos)
        return out
    view = _d2h_base(t).as_strided(t.shape, t.stride(), t.storage_offset())
    return view.clone()  # keeps dense strides, else contiguous


# ------------------------------------------------------- views as boxes --
#
# A view that selects a box of the allocation's host geometry -- slices,
# selects, narrows and permutations of its dims, each view dim stepping one
# host dim by 1 -- is moved by loop nests of its own, so its bytes are moved
# and no others.  The layout must tile each host dim (of more than one
# element) as the reference's tilings do: a unit device dim whose stride_map
# is the host stride and, when that does not hold the whole dim, a tile dim
# above it whose stride_map is the unit dim's run times the host stride (the
# stick dim: runs of 64 elements).  Element (host coords c) then sits at the
# row-major device position sum_j (c_j % run_j) RM[unit_j] + (c_j // run_j)
# RM[tile_j].  A box that crosses run boundaries along a host dim is cut
# there: the part before the first boundary, the whole runs (a tile loop and
# a unit loop) and the part after the last one.  Other views and layouts
# take the round trip through the whole geometry.

def _dim_owners(layout: SpyreTensorLayout, dma_size, dma_stride):
    """{host dim: (unit device dim, tile device dim or None, run)} for the
    host dims of more than one element, or None when the layout does not
    tile the geometry that way."""
    ds, sm = list(layout.device_size), list(layout.stride_map)
    owners, claimed = {}, set()
    for j, (n, hs) in enumerate(zip(dma_size, dma_stride)):
        if n <= 1:
            continue
        unit = [d for d in range(len(ds)) if sm[d] == hs and ds[d] > 1]
        if len(unit) != 1:
            return None
        u = unit[0]
        run = ds[u]
        tile = None
        if run < n:
            tiles = [d for d in range(len(ds)) if d != u and sm[d] == hs * run and ds[d] * run >= n]
            if len(tiles) != 1:
                return None
            tile = tiles[0]
        if u in claimed or tile in claimed:
            return None
        claimed.add(u)
        if tile is not None:
            claimed.add(tile)
        owners[j] = (u, tile, run)
    if any(ds[d] > 1 and d not in claimed for d in range(len(ds))):
        return None
    return owners


def _row_major(sizes):
    st, run = [0] * len(sizes), 1
    for i in range(len(sizes) - 1, -1, -1):
        st[i] = run
        run *= int(sizes[i])
    return st


def _view_box(t: SpyreTensor, allow_broadcast: bool):
    """(host dim of each view dim -- None for size-1 dims, -1 for broadcast
    ones --, start host coords) of a view that is a box of the geometry,
    else None."""
    n, hs = t._dma_size, t._dma_stride
    big = sorted((j for j in range(len(n)) if n[j] > 1), key=lambda j: -hs[j])
    c0, off = [0] * len(n), t.storage_offset()
    for j in big:
        if hs[j] <= 0:
            return None
        c0[j], off = divmod(off, hs[j])
        if c0[j] >= n[j]:
            return None
    if off != 0:
        return None
    dims, used = [], set()
    for k in range(t.dim()):
        size, st = t.shape[k], t.stride(k)
        if size == 1:
            dims.append(None)
            continue
        if st == 0:
            if not allow_broadcast:
                return None
            dims.append(-1)
            continue
        js = [j for j in big if hs[j] == st]
        if len(js) != 1 or js[0] in used or c0[js[0]] + size > n[js[0]]:
            return None
        used.add(js[0])
        dims.append(js[0])
    return dims, c0


def _box_infos(t: SpyreTensor, host: torch.Tensor, host2device: bool):
    """DMA loop nests moving the box view t to / from the host-order tensor
    ``host`` (t's shape, any strides), or None when t is no box of a layout
    _dim_owners understands.  Offsets are relative to the storage starts of
    t's buffer and of ``host``."""
    owners = _dim_owners(t._layout, t._dma_size, t._dma_stride)
    box = _view_box(t, allow_broadcast=not host2device)
    if owners is None or box is None:
        return None
    dims, c0 = box
    RM = _row_major(t._layout.device_size)

    def dev_pos(coords):
        p = 0
        for j, (u, tile, run) in owners.items():
            p += (coords[j] % run) * RM[u] + ((coords[j] // run) * RM[tile] if tile is not None else 0)
        return p

    # Per view dim: its pieces (view start, loops [(count, device stride,
    # host stride)], host dim or None).
    per_dim = []
    for k, j in enumerate(dims):
        size, hst = t.shape[k], host.stride(k)
        if j is None:
            continue
        if j == -1:  # broadcast (reads only): the same device elements
            per_dim.append([(k, 0, [(size, 0, hst)], None)])
            continue
        u, tile, run = owners[j]
        a = c0[j]
        if tile is None or a % run + size <= run:
            per_dim.append([(k, 0, [(size, RM[u], hst)], j)])
            continue
        pieces = []
        head = (-a) % run
        if head:
            pieces.append((k, 0, [(head, RM[u], hst)], j))
        whole = (size - head) // run
        if whole:
            pieces.append((k, head, [(run, RM[u], hst), (whole, RM[tile], run * hst)], j))
        tail = size - head - whole * run
        if tail:
            pieces.append((k, head + whole * run, [(tail, RM[u], hst)], j))
        per_dim.append(pieces)
    import itertools

    infos = []
    dbase = t._data.storage_offset()
    for combo in itertools.product(*per_dim) if per_dim else [()]:
        coords = list(c0)
        hoff = host.storage_offset()
        loops = []
        for k, start, lps, j in combo:
            if j is not None:
                coords[j] = c0[j] + start
            hoff += start * host.stride(k)
            loops += lps
        if not loops:
            loops = [(1, 1, 1)]
        if len(loops) > _lib_max_rank():
            return None
        loops.sort(key=lambda lp: (abs(lp[1]), abs(lp[2])))  # innermost: contiguous on the device
        info = R._lib.StrideInfo()
        info.rank = len(loops)
        for q, (cnt, dst_st, host_st) in enumerate(loops):
            info.size[q] = cnt
            info.stride_src[q] = host_st if host2device else dst_st
            info.stride_dst[q] = dst_st if host2device else host_st
        dpos = dbase + dev_pos(coords)
        info.offset_src = hoff if host2device else dpos
        info.offset_dst = dpos if host2device else hoff
        infos.append(info)
    return infos


def _lib_max_rank() -> int:
    return R._lib.SPYRE_MAX_RANK


def _run_infos(src: torch.Tensor, dst: torch.Tensor, infos) -> None:
    step = R._lib.SPYRE_MAX_INFOS
    for i in range(0, len(infos), step):
        R.dma_copy(src, dst, infos[i:i + step])


def _h2d_into(dst: SpyreTensor, src: torch.Tensor) -> None:
    """dst (a SpyreTensor, base or view) <- src (host order, any strides;
    broadcast to dst's shape)."""
    if src.device != dst.device:
        src = src.to(dst.device)
    if src.dtype != dst.dtype:
        src = src.to(dst.dtype)
    src = src.expand(dst.shape)
    if dst.is_base():
        R.h2d_into(src, dst._data, dst._layout, list(dst._dma_stride))
        return
    if dst.numel() == 0:
        return
    infos = _box_infos(dst, src, host2device=True)
    if infos is not None:  # a box: its own elements only
        R._check_layout_dtype(src.dtype, dst._layout)
        _run_infos(src, dst._data, infos)
        return
    # Another view: the rest of the allocation keeps its values, so the
    # whole geometry goes to host order, takes src through the view and
    # returns.
    base = _d2h_base(dst)
    base.as_strided(dst.shape, dst.stride(), dst.storage_offset()).copy_(src)
    R.h2d_into(base, dst._data, dst._layout, list(dst._dma_stride))


def _copy_d2d(dst: SpyreTensor, src: SpyreTensor) -> None:
    """dst <- src, both SpyreTensors of one logical shape (any layouts)."""
    if (tuple(src.shape) == tuple(dst.shape) and src.is_base() and dst.is_base()
            and src._dma_stride == dst._dma_stride):
        R.relayout_into(src._data, dst._data, list(src.shape), list(src._dma_stride), src._layout, dst._layout)
        return
    _h2d_into(dst, _d2h(src))


def copy_tensor(src: torch.Tensor, dst: torch.Tensor, non_blocking: bool = False) -> torch.Tensor:
    """The reference's _C.copy_tensor(self, dst, non_blocking)
    (torch_spyre/csrc/module.cpp:339-341): H2D when dst is a SpyreTensor,
    D2H when src is, D2D when both are.  Blocking unless ``non_blocking``:
    the call then waits for the copy on the current stream, as
    spyre_copy_from does (torch_spyre/csrc/spyre_mem.cpp:640-643)."""
    if isinstance(dst, SpyreTensor) and isinstance(src, SpyreTensor):
        _copy_d2d(dst, src)
    elif isinstance(dst, SpyreTensor):
        _h2d_into(dst, src)
    elif isinstance(src, SpyreTensor):
        dst.copy_(_d2h(src))
    else:
        raise ValueError("copy_tensor: neither tensor is a SpyreTensor")
    if not non_blocking:
        torch.cuda.current_stream((dst if dst.is_cuda else src).device).synchronize()
    return dst


# -------------------------------------------------------------- restickify --

# Out-of-band restickify targets, keyed by the buffer a tensor's views share
# (the reference carries the target in the compiler's layout of the
# restickify node, torch_spyre/_inductor/insert_restickify.py:139).
_TARGETS = WeakIdKeyDictionary()


def set_restickify_target(t: SpyreTensor, layout: Optional[SpyreTensorLayout]) -> None:
    """Records the layout ``spyre::restickify`` moves t's allocation (and
    every view of it) to; None clears it."""
    if not isinstance(t, SpyreTensor):
        raise TypeError("set_restickify_target takes a SpyreTensor")
    if layout is None:
        _TARGETS.pop(t._data, None)
    else:
        _TARGETS[t._data] = layout


def restickify_target_layout(layout: SpyreTensorLayout, host_size: Sequence[int], host_stride: Sequence[int],
                             new_stick_dim: int) -> SpyreTensorLayout:
    """``layout`` with its stick moved to host dim ``new_stick_dim``: the
    rule of restickify_device_size / restickify_stride_map
    (torch_spyre/_inductor/pass_utils.py:749-781).  The stick's old host dim
    and the two device dims that change are found by their strides: the
    stick's tile dim steps 64 x its host stride, the new dim's device dim
    steps its host stride."""
    size, hst = [int(v) for v in host_size], [int(v) for v in host_stride]
    ds, sm = list(layout.device_size), list(layout.stride_map)
    r = len(ds)
    eps = layout.elems_per_stick()
    old = [h for h in range(len(size)) if hst[h] == sm[-1] and size[h] > 1] or \
          [h for h in range(len(size)) if hst[h] == sm[-1]]
    if len(old) != 1:
        raise NotImplementedError("restickify: the layout's stick dim is ambiguous; set an explicit target")
    old_sd, new_sd = old[0], int(new_stick_dim) % len(size)
    if new_sd == old_sd:
        return layout
    old_outer = [j for j in range(r - 1) if sm[j] == eps * hst[old_sd]]
    new_outer = [j for j in range(r - 1) if sm[j] == hst[new_sd] and ds[j] == size[new_sd]]
    if len(old_outer) != 1 or len(new_outer) != 1:
        raise NotImplementedError("restickify: the layout does not tile the two dims as the default "
                                  "rule does; set an explicit target")
    ds2, sm2 = list(ds), list(sm)
    ds2[-1] = eps
    ds2[old_outer[0]] = (size[new_sd] + eps - 1) // eps
    ds2[new_outer[0]] = size[old_sd]
    sm2[-1] = hst[new_sd]
    sm2[old_outer[0]] = hst[new_sd] * eps
    sm2[new_outer[0]] = hst[old_sd]
    return SpyreTensorLayout(ds2, sm2, layout.device_dtype)


def _default_target(x: SpyreTensor) -> SpyreTensorLayout:
    """The stick moves to the host dim x's innermost logical dim steps
    along, so x read in its own (logical) order runs along sticks."""
    inner = [k for k in range(x.dim()) if x.shape[k] > 1]
    if not inner:
        return x._layout
    s = x.stride(inner[-1])
    dims = [d for d in range(len(x._dma_size)) if x._dma_stride[d] == s and x._dma_size[d] > 1]
    if len(dims) != 1:
        raise NotImplementedError("restickify: the view's innermost dim is no single dim of the "
                                  "allocation; set an explicit target with set_restickify_target")
    return restickify_target_layout(x._layout, x._dma_size, x._dma_stride, dims[0])


def restickify(x: torch.Tensor, dst_layout: Optional[SpyreTensorLayout] = None,
               src_layout: Optional[SpyreTensorLayout] = None,
               host_size: Optional[Sequence[int]] = None) -> torch.Tensor:
    """Device-to-device relayout of the same host values into another stick
    layout (the reference's spyre::restickify; its target layout comes from
    torch_spyre/_inductor/pass_utils.py:749-833).

    For a SpyreTensor: the whole allocation moves to ``dst_layout`` (else the
    target recorded by ``set_restickify_target``, else the stick moves to the
    dim x's innermost logical dim steps along) and the result is x's view
    over the new allocation.  For a plain buffer in stick order:
    ``src_layout`` and ``host_size`` are required and the result is the new
    buffer.  One pass when the two tilings nest; otherwise through host
    order."""
    if isinstance(x, SpyreTensor):
        if src_layout is not None or host_size is not None:
            raise ValueError("a SpyreTensor carries its own layout and geometry")
        target = dst_layout or _TARGETS.get(x._data) or _default_target(x)
        buf = torch.ops.spyre.relayout(x._data, list(x._dma_size), list(x._dma_stride),
                                       list(x._layout.device_size), list(x._layout.stride_map),
                                       list(target.device_size), list(target.stride_map))
        return SpyreTensor(buf, target, x._dma_size, x._dma_stride, x.shape, x.stride(), x.storage_offset())
    _require_cuda(x, "x")
    if dst_layout is None or src_layout is None or host_size is None:
        raise ValueError("a plain device buffer needs dst_layout, src_layout and host_size")
    size = list(host_size)
    return R.relayout_buffer(x, size, _contiguous_strides(size), src_layout, dst_layout)


# -------------------------------------------------------------- dispatch --

def _view(func, args, kwargs):
    x = args[0]
    out = func(x._meta(), *args[1:], **kwargs)

    def wrap(m):
        if m.dtype != x.dtype:
            raise NotImplementedError("dtype views of a SpyreTensor are not supported")
        return x._with_view(m.shape, m.stride(), m.storage_offset())

    if isinstance(out, (list, tuple)):
        return type(out)(wrap(m) for m in out)
    return wrap(out)


def _to_copy(x, dtype=None, layout=None, device=None, pin_memory=None, non_blocking=False,
             memory_format=None):
    host = _d2h(x)
    if device is None or torch.device(device).type == "cuda":
        if dtype is None or dtype == x.dtype:
            raise NotImplementedError("a SpyreTensor copy to the GPU stays in its layout: use clone(), "
                                      "or from_device_layout() for host order")
    return host.to(dtype=dtype, device=device, non_blocking=non_blocking,
                   memory_format=memory_format or torch.preserve_format)


def _copy_(dst, src, non_blocking=False):
    if isinstance(dst, SpyreTensor) and isinstance(src, SpyreTensor):
        _copy_d2d(dst, src)
    elif isinstance(dst, SpyreTensor):
        _h2d_into(dst, src)
    else:
        dst.copy_(_d2h(src))
    return dst


def _clone(x, memory_format=None):
    if x.is_base():  # the allocation byte for byte, through the traceable op
        lay = x._layout
        buf = torch.ops.spyre.relayout(x._data, list(x._dma_size), list(x._dma_stride), list(lay.device_size),
                                       list(lay.stride_map), list(lay.device_size), list(lay.stride_map))
        return SpyreTensor(buf, lay, x._dma_size, x._dma_stride)
    host = _d2h(x).contiguous()
    return to_device_layout(host, _default_layout(list(host.shape), list(host.stride()), host.dtype))


def _detach(x):
    return x._with_view(x.shape, x.stride(), x.storage_offset())


def _copy_from_d2d(src, dst):
    if not isinstance(dst, SpyreTensor):
        raise TypeError("spyre::copy_from_d2d writes into a SpyreTensor")
    if isinstance(src, SpyreTensor):
        _copy_d2d(dst, src)
    else:
        _h2d_into(dst, src)


def _restickify_op(x):
    return restickify(x)


def _index_copy_(x, dim, index, source):
    """x.index_copy_(dim, index, source): source's slice i goes to x's
    slice index[i] along dim.  Runs of consecutive indices are one box
    each, moved by its own loop nests (bytes in proportion to source), in as
    few launches as the nests allow.  The reference serves the op as a CPU
    fallback over the whole tensor (tests/inductor/test_inductor_ops.py:5688-5739)."""
    if not isinstance(x, SpyreTensor):
        raise TypeError("index_copy_ writes into a SpyreTensor")
    dim = dim % max(1, x.dim())
    if index.dim() > 1 or index.dtype not in (torch.int64, torch.int32):
        raise IndexError("index_copy_(): index must be a 1-D integer tensor")
    idx = [int(v) for v in index.reshape(-1).tolist()]
    n = x.shape[dim] if x.dim() else 1
    if source.dim() != x.dim() or (x.dim() and source.shape[dim] != len(idx)):
        raise IndexError("index_copy_(): source must have the rank of self and index.numel() slices along dim")
    for d in range(x.dim()):
        if d != dim and source.shape[d] != x.shape[d]:
            raise IndexError(f"index_copy_(): source and self differ in dim {d}")
    if any(v < -n or v >= n for v in idx):
        raise IndexError(f"index_copy_(): index out of range for dim {dim} of size {n}")
    idx = [v % n for v in idx]
    if source.device != x.device:
        source = source.to(x.device)
    if source.dtype != x.dtype:
        source = source.to(x.dtype)
    i = 0
    while i < len(idx):  # a run of consecutive indices -> one box
        j = i + 1
        while j < len(idx) and idx[j] == idx[j - 1] + 1:
            j += 1
        _h2d_into(x.narrow(dim, idx[i], j - i), source.narrow(dim, i, j - i))
        i = j
    return x


def _index_copy(x, dim, index, source):
    return _index_copy_(_clone(x), dim, index, source)


_HANDLERS = {
    aten._to_copy.default: _to_copy,
    aten.copy_.default: _copy_,
    aten.clone.default: _clone,
    aten.detach.default: _detach,
    aten.alias.default: _detach,
    aten.index_copy_.default: _index_copy_,
    aten.index_copy.default: _index_copy,
}


def register_spyre_ops() -> None:
    """Adds the spyre:: ops (registered by torch_spyre_amd.ops) to the
    SpyreTensor dispatch table."""
    _HANDLERS[torch.ops.spyre.restickify.default] = _restickify_op
    _HANDLERS[torch.ops.spyre.copy_from_d2d.default] = _copy_from_d2d


__all__ = ["SpyreTensor", "spyre_empty_with_layout", "to_device_layout", "from_device_layout",
           "device_tensor_layout", "device_buffer", "copy_tensor", "set_restickify_target",
           "restickify_target_layout", "restickify", "as_strided_with_layout", "reinterpret_tensor",
           "reinterpret_tensor_with_layout"]
