"""Oracle: SpyreTensorLayout semantics and the DMA stride-info loop nests.

Test infrastructure only (see ``oracle/__init__.py``).

Restates, in plain Python / numpy:

* ``SpyreTensorLayout`` construction  -- torch_spyre/csrc/spyre_tensor_impl.cpp:46-179
  (default tiling ``get_generic_stick_layout`` :46-80, ``dim_map_to_stride_map``
  :102-122, ``init`` :124-179) and the device byte size :286-292.
* the host<->device DMA description -- torch_spyre/csrc/spyre_mem.cpp:60-354
  (``get_dim_map`` :60-96, ``get_tile_map`` :107-162,
  ``get_device_stride_infos`` :176-354).
* execution of the resulting loop nests (what the DMA engine does with a
  ``DataConversionStrideInfo``), as documented in
  docs/source/user_guide/tensors_and_layouts.md:290-321.

Parity pins (tests/test_oracle_layout.py):
* descriptor tables of tests/tensor/test_tensor_layout.py:39-104 and the str
  format of :106-111 (fixture tests/golden/stl_golden.json);
* the documented DMA known answer ((4,1024,64),(65536,64,1),(64,256,1)) for a
  (1024,256) fp16 tensor (tensors_and_layouts.md:305-318);
* the identity ``host_offset = dot(device_coords, stride_map)`` on every valid
  device coordinate (tensors_and_layouts.md:210-217), checked by brute force;
* the round trip x == D2H(H2D(x)) for every explicit layout case of
  tests/tensor/test_tensor_layout.py:193-405 (same fixture).
"""

from __future__ import annotations

import itertools
import math
from dataclasses import dataclass, field

import numpy as np

BYTES_IN_STICK = 128  # torch_spyre/csrc/spyre_tensor_impl.cpp:31

# Device data formats on this path and their elements per stick.
# torch dtype name -> device format: torch_spyre/csrc/types_mapping.h:71-92.
# elems per stick: fp16 = 64 (tensors_and_layouts.md:121), int32 = 32
# (spyre_tensor_impl.cpp:35-37), fp32 = 128 B / 4 B = 32.
ELEMS_PER_STICK = {"SEN169_FP16": 64, "IEEE_FP32": 32, "IEEE_INT32": 32}
TORCH_TO_DEVICE_FORMAT = {
    "float16": "SEN169_FP16",
    "bfloat16": "SEN169_FP16",
    "bool": "SEN169_FP16",
    "float32": "IEEE_FP32",
    "int32": "IEEE_INT32",
    "int64": "IEEE_INT32",
}


def device_format(dtype_name: str) -> str:
    if dtype_name not in TORCH_TO_DEVICE_FORMAT:
        raise ValueError(f"unsupported dtype {dtype_name}")
    return TORCH_TO_DEVICE_FORMAT[dtype_name]


def generic_stick_dim_map(dim_order: list[int]) -> list[int]:
    """Default tiling: spyre_tensor_impl.cpp:46-80.

    Ranks 1..6 all follow [o1, ..., o_{r-1}, o0, o_{r-1}]: non-stick dims once,
    the stick dim (last of dim_order) twice -- as the tile index placed after
    the other dims and again as the innermost stick.
    """
    r = len(dim_order)
    if r < 1 or r > 6:
        raise RuntimeError(f"Unsupported tensor rank: {r}")
    table = {
        1: lambda o: [o[0], o[0]],
        2: lambda o: [o[1], o[0], o[1]],
        3: lambda o: [o[1], o[2], o[0], o[2]],
        4: lambda o: [o[1], o[2], o[3], o[0], o[3]],
        5: lambda o: [o[1], o[2], o[3], o[4], o[0], o[4]],
        6: lambda o: [o[1], o[2], o[3], o[4], o[5], o[0], o[5]],
    }
    return table[r](list(dim_order))


def contiguous_strides(size: list[int]) -> list[int]:
    """spyre_tensor_impl.cpp:90-100."""
    st = [0] * len(size)
    s = 1
    for i in range(len(size) - 1, -1, -1):
        st[i] = s
        s *= size[i]
    return st


def dim_map_to_stride_map(dim_map, host_size, host_stride, device_size):
    """spyre_tensor_impl.cpp:102-122."""
    n = len(dim_map)
    stride_map = [-1] * n
    last = [-1] * n
    for j in range(n - 1, -1, -1):
        d = dim_map[j]
        if d == -1 or host_size[d] == 1:
            stride_map[j] = -1
        elif last[d] == -1:
            stride_map[j] = host_stride[d]
            last[d] = stride_map[j] * device_size[j]
        else:
            stride_map[j] = last[d]
            last[d] = stride_map[j] * device_size[j]
    return stride_map


@dataclass
class Layout:
    device_size: list[int]
    stride_map: list[int]
    device_dtype: str = "SEN169_FP16"
    element_arrangement: str = "STANDARD"

    def elems_per_stick(self) -> int:
        return ELEMS_PER_STICK[self.device_dtype]

    def __str__(self) -> str:  # spyre_tensor_impl.cpp:181-202
        ds = ", ".join(str(v) for v in self.device_size)
        sm = ", ".join(str(v) for v in self.stride_map)
        return (f"SpyreTensorLayout(device_size=[{ds}], stride_map =[{sm}], "
                f"device_dtype=DataFormats.{self.device_dtype})")


def stl_init(host_size, host_strides, dtype_name, dim_order) -> Layout:
    """SpyreTensorLayout::init -- spyre_tensor_impl.cpp:132-179."""
    host_size = list(host_size)
    dim_order = list(dim_order)
    if not (len(host_size) == len(dim_order)
            or (len(host_size) + 1 == len(dim_order) and dim_order[-1] == -1)):
        raise RuntimeError("Incompatible host_size and dim_order")
    fmt = device_format(dtype_name)
    eps = ELEMS_PER_STICK[fmt]
    if len(host_size) == 0:
        return Layout([1, eps], [-1, -1], fmt)
    dim_map = generic_stick_dim_map(dim_order)
    sparse = dim_order[-1] == -1
    in_stick = 1 if sparse else eps
    stick_dim = dim_map[-1]
    device_size = [0] * len(dim_map)
    device_size[-1] = eps
    for i in range(len(dim_map) - 1):
        d = dim_map[i]
        if d == stick_dim:
            device_size[i] = 1 if sparse else (host_size[stick_dim] + in_stick - 1) // in_stick
        else:
            device_size[i] = host_size[d]
    stride_map = dim_map_to_stride_map(dim_map, host_size, list(host_strides), device_size)
    return Layout(device_size, stride_map, fmt)


def stl_default(host_size, dtype_name="float16") -> Layout:
    """SpyreTensorLayout(host_size, dtype) -- spyre_tensor_impl.cpp:124-130."""
    return stl_init(host_size, contiguous_strides(list(host_size)), dtype_name,
                    list(range(len(host_size))))


def device_size_in_bytes(device_size) -> int:
    """spyre_tensor_impl.cpp:286-292: 128 B per stick, one stick per outer coordinate."""
    n = BYTES_IN_STICK
    for v in device_size[:-1]:
        n *= v
    return n


# --------------------------------------------------------------------------
# DMA stride infos (torch_spyre/csrc/spyre_mem.cpp)
# --------------------------------------------------------------------------

@dataclass
class StrideInfo:
    """One loop nest; lists are innermost-first (the reference reverses them,
    spyre_mem.cpp:327-329)."""
    size: list[int]
    stride_src: list[int]
    stride_dst: list[int]
    offset_src: int = 0
    offset_dst: int = 0

    def as_tuple(self):
        return (tuple(self.size), tuple(self.stride_src), tuple(self.stride_dst),
                self.offset_src, self.offset_dst)


def get_dim_map(sizes, strides, device_size, stride_map):
    """spyre_mem.cpp:60-96."""
    host_rank = len(strides)
    dev_rank = len(stride_map)
    stick_dim_index = dev_rank - 3 if dev_rank > 2 else 0
    max_le = [0] * dev_rank
    dm = [-1] * dev_rank
    for i in range(host_rank):
        if sizes[i] == 1:
            continue
        hst = strides[i]
        if hst == 0:
            continue
        for j in range(dev_rank):
            if device_size[j] == 1:
                continue
            dst = stride_map[j]
            if hst > max_le[j] and hst <= dst:
                max_le[j] = hst
                dm[j] = i
    if dm[stick_dim_index] != -1:
        dm[stick_dim_index] = dm[dev_rank - 1]
    return dm


def get_tile_map(sizes, strides, device_size, stride_map):
    """spyre_mem.cpp:107-162: per host dim, its device dims by increasing
    stride_map (the stick dim first, keyed -1).  First insertion wins on equal
    keys (std::map::insert)."""
    dm = get_dim_map(sizes, strides, device_size, stride_map)
    host_rank = len(strides)
    dev_rank = len(stride_map)
    pairs: list[dict] = [dict() for _ in range(host_rank)]
    stick = dm[dev_rank - 1]
    if stick != -1:
        pairs[stick].setdefault(-1, dev_rank - 1)
    for i in range(dev_rank - 2, -1, -1):
        d = dm[i]
        if d == -1:
            continue
        pairs[d].setdefault(stride_map[i], i)
    return [[idx for _, idx in sorted(p.items())] for p in pairs]


def device_stride_infos(sizes, dma_strides, storage_offset, device_size, stride_map,
                        host2device: bool, cpu_strides) -> list[StrideInfo]:
    """get_device_stride_infos -- spyre_mem.cpp:176-354."""
    sizes = list(sizes)
    dma_strides = list(dma_strides)
    cpu_strides = list(cpu_strides)
    tmap = get_tile_map(sizes, dma_strides, device_size, stride_map)
    host_rank = len(cpu_strides)
    dev_rank = len(stride_map)
    host_strides = [1] * dev_rank
    cpu_layout = [1] * dev_rank
    dev_strides = [1] * dev_rank
    dcsi = [1] * dev_rank
    prev = 1
    for i in range(dev_rank - 1, -1, -1):
        if stride_map[i] == 0:
            dcsi[i] = device_size[i]
        dev_strides[i] = prev
        prev *= device_size[i]
        if stride_map[i] == -1:
            continue
        host_strides[i] = stride_map[i]
        cpu_layout[i] = stride_map[i]
    for dd in range(dev_rank):
        v = stride_map[dd]
        if v <= 0:
            continue
        for hd in range(host_rank):
            if dma_strides[hd] == v:
                cpu_layout[dd] = cpu_strides[hd]
                break

    remainders, host_offs, dev_offs = [], [], []
    for i in range(host_rank - 1, -1, -1):
        if not tmap[i]:
            continue
        hstride = dma_strides[i]
        hsize = sizes[i]
        j = i - 1
        while j > -1 and not tmap[j]:  # fold unmapped outer host dims
            if dma_strides[j] != 0:
                hsize *= sizes[j]
            j -= 1
        eb = 1
        j = len(tmap[i]) - 1
        while j > -1:
            ti = tmap[i][j]
            tsize = device_size[ti]
            tstride = host_strides[ti] // hstride
            if tsize == 1:
                j -= 1
                continue
            if hsize % eb != 0:
                raise RuntimeError("Invalid device sizes and stride map for host sizes and strides")
            cur = hsize // eb
            rem = cur // tstride
            if rem <= 0:
                raise RuntimeError("Invalid device sizes and stride map for host sizes and strides")
            if cur % tstride == 0:
                dcsi[ti] = min(rem, tsize)
                eb *= dcsi[ti]
            else:
                if j == 0:
                    raise RuntimeError("Invalid tiling for dimension")
                j -= 1
                ni = tmap[i][j]
                nsize = device_size[ni]
                nstride = host_strides[ni] // hstride
                tiled = cur // nstride
                dcsi[ti] = rem
                dcsi[ni] = nsize
                eb *= tiled
                r = [0] * dev_rank
                r[ti] = 1
                r[ni] = tiled % nsize
                remainders.append(r)
                host_offs.append(rem * host_strides[ti])
                dev_offs.append(rem * dev_strides[ti])
            j -= 1

    first = StrideInfo(
        size=list(reversed(dcsi)),
        stride_src=list(reversed(cpu_layout if host2device else dev_strides)),
        stride_dst=list(reversed(dev_strides if host2device else cpu_layout)),
        offset_src=storage_offset if host2device else 0,
        offset_dst=0 if host2device else storage_offset,
    )
    infos = [first]
    for r, ho, do in zip(remainders, host_offs, dev_offs):
        r = list(reversed(r))
        osrc = ho if host2device else do
        odst = do if host2device else ho
        for k in range(len(infos)):
            base = infos[k]
            infos.append(StrideInfo(
                size=[r[q] if r[q] != 0 else base.size[q] for q in range(dev_rank)],
                stride_src=list(base.stride_src), stride_dst=list(base.stride_dst),
                offset_src=base.offset_src + osrc, offset_dst=base.offset_dst + odst))
    return infos


def loop_indices(size, strides, offset) -> np.ndarray:
    """Flat element offsets of a loop nest (innermost-first lists), in the
    row-major order of the reversed nest (outermost loop slowest)."""
    idx = np.array(offset, dtype=np.int64)
    for s, st in zip(reversed(size), reversed(strides)):
        idx = (idx[..., None] + np.arange(s, dtype=np.int64) * st)
    return idx.reshape(-1)


def execute_infos(src_flat: np.ndarray, dst_flat: np.ndarray, infos: list[StrideInfo]) -> None:
    """What the DMA engine does with a DataConversionInfo: for every index
    tuple of every stride info, dst[off_d + i.sd] = src[off_s + i.ss]
    (tensors_and_layouts.md:313-318)."""
    esz = src_flat.dtype.itemsize
    for info in infos:
        if any(s == 0 for s in info.size):
            continue
        shape = list(reversed(info.size))  # outermost loop first
        src = np.lib.stride_tricks.as_strided(
            src_flat[info.offset_src:], shape=shape,
            strides=[s * esz for s in reversed(info.stride_src)], writeable=False)
        dst = np.lib.stride_tricks.as_strided(
            dst_flat[info.offset_dst:], shape=shape,
            strides=[s * esz for s in reversed(info.stride_dst)])
        dst[...] = src


def h2d(host_flat: np.ndarray, sizes, strides, storage_offset, layout: Layout,
        fill=0) -> np.ndarray:
    """Host tensor (flat storage + sizes/strides/offset) -> flat device buffer.

    The device buffer is the stick-padded allocation (device_size_in_bytes);
    positions the DMA does not write keep ``fill`` (the reference leaves them
    as whatever the allocation held; the product zero-fills them)."""
    esz = host_flat.dtype.itemsize
    n = max(device_size_in_bytes(layout.device_size) // esz, int(np.prod(sizes)) if sizes else 1)
    dev = np.full(n, fill, dtype=host_flat.dtype)
    infos = device_stride_infos(sizes, strides, storage_offset, layout.device_size,
                                layout.stride_map, True, strides)
    execute_infos(host_flat, dev, infos)
    return dev


def d2h(dev_flat: np.ndarray, sizes, layout: Layout, strides=None) -> np.ndarray:
    """Flat device buffer -> host array of ``sizes`` (the ``.cpu()`` path,
    spyre_mem.cpp:594-651 and generate_dci :414-434).

    ``strides`` are the device tensor's dma_strides (the host strides it was
    created with, spyre_mem.cpp:573-576); the D2H DMA writes the host buffer
    with those strides, so the result is returned as a view with them.
    Defaults to contiguous strides."""
    sizes = list(sizes)
    strides = contiguous_strides(sizes) if strides is None else list(strides)
    span = 1 + sum((s - 1) * st for s, st in zip(sizes, strides)) if sizes else 1
    host = np.zeros(span, dtype=dev_flat.dtype)
    infos = device_stride_infos(sizes, strides, 0, layout.device_size, layout.stride_map,
                                False, strides)
    execute_infos(dev_flat, host, infos)
    esz = host.dtype.itemsize
    return np.lib.stride_tricks.as_strided(host, shape=sizes, strides=[s * esz for s in strides])


def valid_device_coords(layout: Layout, sizes, strides):
    """Brute force over every device coordinate: yields (device_offset,
    host_offset) for the coordinates the H2D loop nests write.  Used to check
    the identity host_offset = dot(coords, stride_map) on tiny shapes."""
    infos = device_stride_infos(sizes, strides, 0, layout.device_size, layout.stride_map,
                                True, strides)
    seen = {}
    for info in infos:
        ranges = [range(s) for s in reversed(info.size)]
        for idx in itertools.product(*ranges):
            idx = list(reversed(idx))
            so = info.offset_src + sum(i * s for i, s in zip(idx, info.stride_src))
            do = info.offset_dst + sum(i * s for i, s in zip(idx, info.stride_dst))
            seen[do] = so
    return seen


def device_coords_of_offset(layout: Layout, off: int) -> list[int]:
    coords = []
    for s in reversed(layout.device_size):
        coords.append(off % s)
        off //= s
    return list(reversed(coords))


def stride_map_offset(layout: Layout, coords) -> int:
    """offset = dot(device_coordinates, stride_map), -1 dims contribute 0
    (tensors_and_layouts.md:210-217)."""
    return sum(c * s for c, s in zip(coords, layout.stride_map) if s != -1)
