"""ctypes binding of libspyre_hip.so (the C ABI declared in include/spyre_hip.h).

There is no fallback: if the library is not built, importing the package's
GPU entry points raises.  Build it with ``python torch_spyre_amd/build.py``
(or ``__graft_entry__.build()``).
"""

from __future__ import annotations

import ctypes
import os
import re
from ctypes import POINTER, c_char_p, c_float, c_int, c_int32, c_int64, c_size_t, c_uint64, c_void_p

# torch first: its HIP runtime (soname libamdhip64.so.7) is then the one the
# native libraries bind to, not a second copy from the ROCm install
import torch

LIB_NAME = "libspyre_hip.so"
LIB_PATH = os.environ.get("SPYRE_HIP_LIB") or os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)
# The PyTorch kernels of the attention and KV ops (csrc/torch_ops.cpp),
# linked against libspyre_hip.so beside them.
TORCH_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libspyre_torch.so")

SPYRE_OK = 0
SPYRE_EINVAL = -1
SPYRE_EUNSUPPORTED = -2
SPYRE_ENOSPC = -3
SPYRE_EHIP = -4
SPYRE_MAX_RANK = 8
SPYRE_MAX_INFOS = 64
ABI_VERSION = 1


class StrideInfo(ctypes.Structure):
    """spyre_stride_info: one DMA loop nest, innermost loop first."""

    _fields_ = [
        ("rank", c_int32),
        ("reserved", c_int32),
        ("size", c_int64 * SPYRE_MAX_RANK),
        ("stride_src", c_int64 * SPYRE_MAX_RANK),
        ("stride_dst", c_int64 * SPYRE_MAX_RANK),
        ("offset_src", c_int64),
        ("offset_dst", c_int64),
    ]

    def as_tuple(self):
        r = self.rank
        return (tuple(self.size[:r]), tuple(self.stride_src[:r]), tuple(self.stride_dst[:r]),
                int(self.offset_src), int(self.offset_dst))

    def __repr__(self) -> str:
        s, ss, sd, os_, od = self.as_tuple()
        return f"StrideInfo(size={list(s)}, stride_src={list(ss)}, stride_dst={list(sd)}, offset_src={os_}, offset_dst={od})"


# name -> (restype, argtypes); every symbol include/spyre_hip.h declares.
SIGNATURES = {
    "spyre_abi_version": (c_int, []),
    "spyre_last_error": (c_char_p, []),
    "spyre_device_format": (c_int, [c_int]),
    "spyre_elems_per_stick": (c_int64, [c_int]),
    "spyre_stl_init": (c_int, [POINTER(c_int64), c_int, POINTER(c_int64), c_int, POINTER(c_int32),
                               c_int, POINTER(c_int64), POINTER(c_int64), POINTER(c_int),
                               POINTER(c_int)]),
    "spyre_device_size_in_bytes": (c_uint64, [POINTER(c_int64), c_int]),
    "spyre_dma_plan": (c_int, [POINTER(c_int64), POINTER(c_int64), POINTER(c_int64), c_int, c_int64,
                               POINTER(c_int64), POINTER(c_int64), c_int, c_int,
                               POINTER(StrideInfo), c_int, POINTER(c_int)]),
    "spyre_restick_plan": (c_int, [POINTER(c_int64), c_int, POINTER(c_int64), POINTER(c_int64), c_int,
                                   POINTER(c_int64), POINTER(c_int64), c_int, POINTER(StrideInfo)]),
    "spyre_dma_copy": (c_int, [c_void_p, c_size_t, c_void_p, c_size_t, c_int, POINTER(StrideInfo),
                               c_int, c_void_p]),
    "spyre_kv_append_f16": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int64,
                                    c_void_p, c_int, c_int, c_int, c_int, c_int64, c_void_p]),
    "spyre_paged_decode_attn_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int, c_int, c_int]),
    "spyre_paged_decode_attn_kernels": (c_int, [c_int, c_int, c_int, c_int, c_int, c_int]),
    "spyre_paged_decode_attn_f16": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_void_p,
                                            c_void_p, c_void_p, c_void_p, c_size_t, c_int, c_int,
                                            c_int, c_int, c_int, c_int64, c_int, c_int, c_float,
                                            c_void_p]),
    "spyre_paged_decode_attn_split_f16": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_void_p,
                                                  c_void_p, c_size_t, c_int, c_int, c_int, c_int, c_int,
                                                  c_int64, c_int, c_int, c_float, c_void_p]),
    "spyre_paged_decode_attn_merge_f16": (c_int, [c_void_p, c_void_p, c_size_t, c_void_p, c_void_p, c_int,
                                                  c_int, c_int, c_int, c_int, c_int, c_void_p]),
    "spyre_paged_decode_attn_noalloc_f16": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_void_p,
                                                    c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int,
                                                    c_int64, c_int, c_int, c_float, c_void_p]),
    "spyre_dense_decode_load_extent": (c_int, [c_int, c_int, c_int64, c_int64, POINTER(c_int64), POINTER(c_int64),
                                               POINTER(c_int64)]),
    "spyre_sdpa_fwd_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int]),
    "spyre_sdpa_fwd_call_workspace_bytes": (c_size_t, [c_void_p, c_int, POINTER(c_int64), c_int, c_int, c_int,
                                                       c_int, c_int, c_int]),
    "spyre_sdpa_fwd_f16": (c_int, [c_void_p, POINTER(c_int64), c_void_p, POINTER(c_int64), c_void_p,
                                   POINTER(c_int64), c_void_p, c_int, POINTER(c_int64), c_int, c_float,
                                   c_void_p, c_void_p, c_void_p, c_size_t, c_int, c_int, c_int, c_int,
                                   c_int, c_int, c_void_p]),
}

_lib = None


class SpyreHipError(RuntimeError):
    """A C-ABI call returned an error (message from spyre_last_error)."""

    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} failed ({code}): {msg}")
        self.code = code


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is not built; run `python torch_spyre_amd/build.py` first "
                "(the package has no CPU fallback)")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        if handle.spyre_abi_version() != ABI_VERSION:
            raise ImportError(f"{LIB_PATH}: ABI version {handle.spyre_abi_version()} != {ABI_VERSION}")
        _lib = handle
    return _lib


_torch_ops_loaded = False


def load_torch_ops() -> None:
    """Registers the spyre:: attention / KV ops and the CUDA kernel of
    aten::_scaled_dot_product_fused_attention_overrideable (libspyre_torch.so)."""
    global _torch_ops_loaded
    if _torch_ops_loaded:
        return
    if not os.path.exists(TORCH_LIB_PATH):
        raise ImportError(f"{TORCH_LIB_PATH} is not built; run `python torch_spyre_amd/build.py` first "
                          "(the package has no CPU fallback)")
    lib()
    torch.ops.load_library(TORCH_LIB_PATH)
    _torch_ops_loaded = True


_OP_ERROR = re.compile(r"\[spyre_hip (\S+) (-?\d+)\] ?(.*)")


def library_error(e: RuntimeError) -> RuntimeError:
    """The SpyreHipError a torch op's RuntimeError carries (a failure the
    library reported, tagged "[spyre_hip <fn> <code>]" by libspyre_torch.so),
    else e itself."""
    m = _OP_ERROR.search(str(e).splitlines()[0] if str(e) else "")
    return SpyreHipError(m.group(1), int(m.group(2)), m.group(3)) if m else e


def check(name: str, rc: int) -> None:
    if rc != SPYRE_OK:
        msg = lib().spyre_last_error()
        raise SpyreHipError(name, rc, msg.decode() if msg else "")


def i64_array(values) -> ctypes.Array:
    values = [int(v) for v in values]
    return (c_int64 * max(1, len(values)))(*values)


def i32_array(values) -> ctypes.Array:
    values = [int(v) for v in values]
    return (c_int32 * max(1, len(values)))(*values)
