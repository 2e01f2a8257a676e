"""SpyreTensorLayout: the stick-layout descriptor.

Same constructors, attributes, equality/hash, pickle format (v3 tuple) and
str format as the reference's pybind class (torch_spyre/csrc/module.cpp:206-286,
torch_spyre/csrc/spyre_tensor_impl.h:50-138).  Construction and the DMA plans
are computed by the native library (torch_spyre_amd/csrc/layout.cpp).
"""

from __future__ import annotations

import ctypes
import enum
from typing import Sequence

import torch

from . import _lib

PICKLE_VERSION = 3  # torch_spyre/csrc/module.cpp:60


class DataFormats(enum.IntEnum):
    """Device data formats on this path (names as the reference's DataFormats)."""

    INVALID = 0
    SEN169_FP16 = 1
    IEEE_FP32 = 2
    IEEE_INT32 = 3

    def __str__(self) -> str:
        return f"DataFormats.{self.name}"


class ElementArrangement(enum.IntEnum):
    """torch_spyre/csrc/spyre_tensor_impl.h:40-48."""

    STANDARD = 0
    DL16_TO_FP32 = 1
    QFP8CH = 2
    EXX2 = 3


# torch dtype -> c10::ScalarType code understood by spyre_stl_init.
_SCALAR_TYPE = {
    torch.int32: 3,
    torch.int64: 4,
    torch.float16: 5,
    torch.float32: 6,
    torch.bool: 11,
    torch.bfloat16: 15,
}


def _scalar_type(dtype: torch.dtype) -> int:
    if dtype not in _SCALAR_TYPE:
        raise TypeError(f"Spyre stick layouts do not support dtype {dtype}")
    return _SCALAR_TYPE[dtype]


def get_device_dtype(dtype: torch.dtype) -> DataFormats:
    """Device format of a torch dtype (torch_spyre/csrc/module.cpp:143-152)."""
    code = _SCALAR_TYPE.get(dtype)
    if code is None:
        return DataFormats.INVALID
    return DataFormats(_lib.lib().spyre_device_format(code))


class SpyreTensorLayout:
    """Device tiling of a tensor: ``device_size`` (row-major on the device,
    last dim = one 128-byte stick) and ``stride_map`` (host elements advanced
    per step along each device dim, -1 for synthetic/padded dims).

    Constructors (as the reference's):
      SpyreTensorLayout(host_size, dtype)
      SpyreTensorLayout(host_size, host_strides, dtype, dim_order, element_arrangement=STANDARD)
      SpyreTensorLayout(device_size, stride_map, device_dtype: DataFormats, element_arrangement=STANDARD)
    """

    __slots__ = ("device_size", "stride_map", "device_dtype", "element_arrangement")

    def __init__(self, *args, **kwargs):
        args = list(args)
        names3 = ("host_size", "host_strides", "dtype", "dim_order", "element_arrangement")
        names_explicit = ("device_size", "stride_map", "device_dtype", "element_arrangement")
        if "device_size" in kwargs or "device_dtype" in kwargs or (
                len(args) >= 3 and isinstance(args[2], (DataFormats, int)) and not isinstance(args[2], bool)
                and not isinstance(args[2], torch.dtype)):
            vals = dict(zip(names_explicit, args))
            vals.update(kwargs)
            self._init_explicit(vals["device_size"], vals["stride_map"], vals["device_dtype"],
                                vals.get("element_arrangement", ElementArrangement.STANDARD))
            return
        vals = dict(zip(names3 if len(args) != 2 else ("host_size", "dtype"), args))
        vals.update(kwargs)
        host_size = [int(v) for v in vals["host_size"]]
        dtype = vals["dtype"]
        strides = vals.get("host_strides")
        dim_order = vals.get("dim_order")
        ea = vals.get("element_arrangement", ElementArrangement.STANDARD)
        if (strides is None) != (dim_order is None):
            raise TypeError("host_strides and dim_order must be given together")
        self._init_host(host_size, strides, dtype, dim_order, ea)

    # -- construction -------------------------------------------------------
    def _init_explicit(self, device_size, stride_map, device_dtype, ea):
        device_size = [int(v) for v in device_size]
        stride_map = [int(v) for v in stride_map]
        if len(device_size) != len(stride_map):
            raise ValueError("device_size and stride_map must have the same length")
        if not 1 <= len(device_size) <= _lib.SPYRE_MAX_RANK:
            raise ValueError(f"device rank must be in [1, {_lib.SPYRE_MAX_RANK}]")
        self.device_size = device_size
        self.stride_map = stride_map
        self.device_dtype = DataFormats(int(device_dtype))
        self.element_arrangement = ElementArrangement(int(ea))

    def _init_host(self, host_size, strides, dtype, dim_order, ea):
        L = _lib.lib()
        ds = (ctypes.c_int64 * _lib.SPYRE_MAX_RANK)()
        sm = (ctypes.c_int64 * _lib.SPYRE_MAX_RANK)()
        rank = ctypes.c_int()
        fmt = ctypes.c_int()
        hs = _lib.i64_array(host_size)
        st = _lib.i64_array(strides) if strides is not None else None
        do = _lib.i32_array(dim_order) if dim_order is not None else None
        rc = L.spyre_stl_init(hs, len(host_size), st, _scalar_type(dtype), do,
                              len(dim_order) if dim_order is not None else 0, ds, sm,
                              ctypes.byref(rank), ctypes.byref(fmt))
        _lib.check("spyre_stl_init", rc)
        self.device_size = list(ds[: rank.value])
        self.stride_map = list(sm[: rank.value])
        self.device_dtype = DataFormats(fmt.value)
        self.element_arrangement = ElementArrangement(int(ea))

    # -- reference API --------------------------------------------------------
    def elems_per_stick(self) -> int:
        return int(_lib.lib().spyre_elems_per_stick(int(self.device_dtype)))

    def with_element_arrangement(self, element_arrangement) -> "SpyreTensorLayout":
        return SpyreTensorLayout(self.device_size, self.stride_map, self.device_dtype,
                                 element_arrangement)

    def device_size_in_bytes(self) -> int:
        """128 bytes per stick (torch_spyre/csrc/spyre_tensor_impl.cpp:286-292)."""
        return int(_lib.lib().spyre_device_size_in_bytes(_lib.i64_array(self.device_size),
                                                           len(self.device_size)))

    def _key(self):
        return (tuple(self.device_size), tuple(self.stride_map), int(self.device_dtype),
                int(self.element_arrangement))

    def __eq__(self, other) -> bool:
        return isinstance(other, SpyreTensorLayout) and self._key() == other._key()

    def __ne__(self, other) -> bool:
        return not self == other

    def __hash__(self) -> int:
        return hash(self._key())

    def __str__(self) -> str:
        ds = ", ".join(str(v) for v in self.device_size)
        sm = ", ".join(str(v) for v in self.stride_map)
        return f"SpyreTensorLayout(device_size=[{ds}], stride_map =[{sm}], device_dtype={self.device_dtype})"

    __repr__ = __str__

    # pickle: (version, device_size, stride_map, device_dtype, element_arrangement)
    def __getstate__(self):
        return (PICKLE_VERSION, list(self.device_size), list(self.stride_map), self.device_dtype,
                self.element_arrangement)

    def __setstate__(self, t):
        version = int(t[0])
        if version == 1:  # (1, device_size, dim_map, stride_map, device_dtype)
            if len(t) != 5:
                raise ValueError("Invalid SpyreTensorLayout pickle v1: wrong tuple size")
            self._init_explicit(t[1], t[3], t[4], ElementArrangement.STANDARD)
        elif version == 2:
            if len(t) != 4:
                raise ValueError("Invalid SpyreTensorLayout pickle v2: wrong tuple size")
            self._init_explicit(t[1], t[2], t[3], ElementArrangement.STANDARD)
        elif version == 3:
            if len(t) != 5:
                raise ValueError("Invalid SpyreTensorLayout pickle v3: wrong tuple size")
            self._init_explicit(t[1], t[2], t[3], t[4])
        else:
            raise ValueError(f"Unsupported SpyreTensorLayout pickle version: {version}")

    def __reduce__(self):
        return (_from_state, (self.__getstate__(),))

    def __deepcopy__(self, memo):
        return SpyreTensorLayout(list(self.device_size), list(self.stride_map), self.device_dtype,
                                 self.element_arrangement)


def _from_state(state) -> SpyreTensorLayout:
    obj = SpyreTensorLayout.__new__(SpyreTensorLayout)
    obj.__setstate__(state)
    return obj


def dma_plan(sizes: Sequence[int], dma_strides: Sequence[int], cpu_strides: Sequence[int],
             storage_offset: int, layout: SpyreTensorLayout, host2device: bool):
    """DMA loop nests (list of _lib.StrideInfo) for a host<->device relayout
    (torch_spyre/csrc/spyre_mem.cpp:176-354)."""
    L = _lib.lib()
    if len(sizes) == 0:  # scalars travel as [1]/[1] (spyre_mem.cpp:395-405)
        sizes, dma_strides, cpu_strides = [1], [1], [1]
    infos = (_lib.StrideInfo * _lib.SPYRE_MAX_INFOS)()
    n = ctypes.c_int()
    rc = L.spyre_dma_plan(_lib.i64_array(sizes), _lib.i64_array(dma_strides), _lib.i64_array(cpu_strides),
                          len(sizes), int(storage_offset), _lib.i64_array(layout.device_size),
                          _lib.i64_array(layout.stride_map), len(layout.device_size),
                          1 if host2device else 0, infos, _lib.SPYRE_MAX_INFOS, ctypes.byref(n))
    _lib.check("spyre_dma_plan", rc)
    return [infos[i] for i in range(n.value)]


def restick_plan(host_size: Sequence[int], src: SpyreTensorLayout, dst: SpyreTensorLayout):
    """Single loop nest moving a dense tensor from layout ``src`` to ``dst``,
    or None when the tilings do not nest."""
    L = _lib.lib()
    info = _lib.StrideInfo()
    rc = L.spyre_restick_plan(_lib.i64_array(host_size), len(host_size),
                              _lib.i64_array(src.device_size), _lib.i64_array(src.stride_map),
                              len(src.device_size), _lib.i64_array(dst.device_size),
                              _lib.i64_array(dst.stride_map), len(dst.device_size), ctypes.byref(info))
    if rc == _lib.SPYRE_EUNSUPPORTED:
        return None
    _lib.check("spyre_restick_plan", rc)
    return info
