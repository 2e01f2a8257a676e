"""The reference's method-form layout API on torch itself.

Importing torch_spyre makes ``Tensor.to(..., device_layout=stl)``,
``torch.empty(..., device_layout=stl)`` and ``Tensor.device_tensor_layout()``
available (torch_spyre/_monkey_patch.py:26-196, applied at import by
torch_spyre/__init__.py:279-281).  This module does the same for
torch_spyre_amd: calls without ``device_layout`` go to torch's own
functions untouched; with it they produce SpyreTensors, whose bytes move
through the relayout kernels.

There is no "spyre" device here: a device argument of "spyre" (or
"spyre:N") means the current (or N-th) GPU, and "cuda" devices are taken
as given.
"""

from __future__ import annotations

from typing import Optional

import torch

from .layout import SpyreTensorLayout


def _device_of(dev) -> Optional[torch.device]:
    if dev is None:
        return None
    if isinstance(dev, str) and dev.split(":")[0] == "spyre":
        idx = dev.split(":")[1] if ":" in dev else None
        return torch.device("cuda", int(idx) if idx is not None else torch.cuda.current_device())
    if isinstance(dev, int):
        return torch.device("cuda", dev)
    return torch.device(dev)


def apply() -> None:
    if getattr(torch.Tensor, "_spyre_amd_patched", False):
        return
    from torch.utils._device import _device_constructors

    _device_constructors()  # cache the constructor set with torch's own torch.empty

    from . import device_tensor as DT

    orig_to = torch.Tensor.to
    orig_empty = torch.empty

    def device_tensor_layout(self: torch.Tensor) -> Optional[SpyreTensorLayout]:
        """The layout of a SpyreTensor, else None (torch_spyre/_monkey_patch.py:63-71)."""
        return DT.device_tensor_layout(self)

    def spyre_to(self, *args, device_layout=None, **kwargs):
        """torch_spyre/_monkey_patch.py:73-155: with device_layout, a copy of
        self in that layout -- H2D from host order (CPU or plain GPU
        tensors, any strides, keeping self's sizes and strides as the DMA
        geometry), D2D from a SpyreTensor (self itself when the layout is
        already device_layout, the dtype is kept and copy is not set)."""
        if device_layout is None:
            return orig_to(self, *args, **kwargs)
        if not isinstance(device_layout, SpyreTensorLayout):
            raise TypeError("device_layout must be a SpyreTensorLayout")
        dtype, device = kwargs.get("dtype"), kwargs.get("device")
        for a in args:
            if isinstance(a, torch.dtype):
                dtype = a
            elif isinstance(a, torch.Tensor):
                dtype = a.dtype
                device = a.device
            elif isinstance(a, (str, torch.device, int)):
                device = a
        if dtype is None and isinstance(kwargs.get("tensor"), torch.Tensor):
            dtype = kwargs["tensor"].dtype
        dtype = dtype or self.dtype
        dev = _device_of(device)
        if dev is not None and dev.type != "cuda":
            raise ValueError(f"a tensor in a device layout lives on a GPU, not {dev}")
        if isinstance(self, DT.SpyreTensor):
            if not kwargs.get("copy") and dtype == self.dtype and self._layout == device_layout:
                return self
            dst = DT.spyre_empty_with_layout(list(self.shape), list(self.stride()), dtype, device_layout,
                                             dev or self.device, zero=True)
            torch.ops.spyre.copy_from_d2d(self, dst)
            return dst
        dst = DT.spyre_empty_with_layout(list(self.shape), list(self.stride()), dtype, device_layout,
                                         dev or (self.device if self.is_cuda else None), zero=True)
        DT.copy_tensor(self, dst, non_blocking=False)
        return dst

    def spyre_empty(*args, device_layout=None, out=None, dtype=None, layout=torch.strided, device=None,
                    requires_grad=False, pin_memory=False, memory_format=torch.contiguous_format):
        """torch_spyre/_monkey_patch.py:157-188: with device_layout, an
        allocation of the (contiguous) size in that layout."""
        if device_layout is None:
            kw = dict(out=out, dtype=dtype, layout=layout, requires_grad=requires_grad, pin_memory=pin_memory,
                      memory_format=memory_format)
            if device is not None:
                kw["device"] = device
            return orig_empty(*args, **kw)
        size = list(args[0]) if len(args) == 1 and isinstance(args[0], (list, tuple, torch.Size)) else list(args)
        size = [int(v) for v in size]
        dev = _device_of(device)
        if dev is not None and dev.type != "cuda":
            raise ValueError(f"a tensor in a device layout lives on a GPU, not {dev}")
        return DT.spyre_empty_with_layout(size, DT._contiguous_strides(size), dtype or torch.get_default_dtype(),
                                          device_layout, dev, zero=False)

    torch.Tensor.device_tensor_layout = device_tensor_layout
    torch.Tensor.to = spyre_to
    torch.empty = spyre_empty
    torch.Tensor._spyre_amd_patched = True
