"""MI355X (gfx950) stick relayout and paged split-KV decode attention.

A drop-in for torch-spyre's relayout / restickify / overwrite / decode-SDPA
path: the SpyreTensorLayout descriptor, the host<->device DMA descriptors and
the ``spyre::`` ops, executed by hand-written HIP kernels in
``libspyre_hip.so`` (C ABI: include/spyre_hip.h).

Importing the package loads the native library; it raises ImportError when
the library is not built.  There is no CPU path.
"""

from . import _lib

_lib.lib()  # fail loudly at import when the native library is missing
_lib.load_torch_ops()  # the C++ kernels of the attention and KV ops

from .layout import (  # noqa: E402
    DataFormats,
    ElementArrangement,
    SpyreTensorLayout,
    dma_plan,
    get_device_dtype,
    restick_plan,
)
from .relayout import (  # noqa: E402
    DmaCopy,
    overwrite,
    transpose_restick_layout,
)
from .device_tensor import (  # noqa: E402
    SpyreTensor,
    copy_tensor,
    device_buffer,
    device_tensor_layout,
    from_device_layout,
    restickify,
    restickify_target_layout,
    set_restickify_target,
    spyre_empty_with_layout,
    to_device_layout,
    as_strided_with_layout,
    reinterpret_tensor,
    reinterpret_tensor_with_layout,
)
from .attention import (  # noqa: E402
    PagedDecode,
    PagedKVCache,
    dense_to_pages,
    k_page_layout,
    kv_append,
    paged_decode_attention,
    paged_decode_merge,
    paged_decode_split,
    sdpa_decode,
    v_page_layout,
    workspace_bytes,
)
from .sdpa import (  # noqa: E402
    SdpaCall,
    Unsupported,
    scaled_dot_product_attention,
    sdpa_override,
    sdpa_overrideable,
)
from . import ops  # noqa: E402,F401  (registers the spyre:: ops)
from . import _torch_patch  # noqa: E402

_torch_patch.apply()  # Tensor.to(device_layout=), torch.empty(device_layout=), Tensor.device_tensor_layout()

__all__ = [
    "DataFormats", "ElementArrangement", "SpyreTensorLayout", "dma_plan", "get_device_dtype",
    "restick_plan", "DmaCopy", "overwrite", "transpose_restick_layout",
    "SpyreTensor", "copy_tensor", "device_buffer", "device_tensor_layout", "from_device_layout", "restickify",
    "restickify_target_layout", "set_restickify_target", "spyre_empty_with_layout", "to_device_layout",
    "as_strided_with_layout", "reinterpret_tensor", "reinterpret_tensor_with_layout",
    "PagedDecode", "PagedKVCache", "dense_to_pages", "k_page_layout", "kv_append", "paged_decode_attention",
    "paged_decode_merge", "paged_decode_split",
    "sdpa_decode", "v_page_layout", "workspace_bytes",
    "SdpaCall", "Unsupported", "scaled_dot_product_attention", "sdpa_override", "sdpa_overrideable",
]
