"""Scaled dot-product attention forward (prefill and any query length).

Mirrors ``torch.nn.functional.scaled_dot_product_attention`` and the
reference's overrideable op ``aten::_scaled_dot_product_fused_attention_overrideable``
(torch_spyre/_inductor/decompositions.py:523-609, chosen by
``_fused_sdp_choice`` in torch_spyre/csrc/attn_utils.cpp:22-37):

* GQA by head: q head h reads KV head h // (Hq // Hkv) (:560-563);
* ``is_causal``: the bias triu(-inf, diagonal=1) over [Sq, Skv], top-left
  aligned (:565-570); it excludes an explicit mask (the reference asserts);
* ``attn_mask`` / ``attn_bias``: an additive fp16/fp32 bias or a boolean
  keep-mask, broadcast to [B, Hq, Sq, Skv];
* dropout raises ``Unsupported``, as the reference does (:578-580);
* the output has the strides of a contiguous [B, Sq, Hq, D] tensor viewed as
  [B, Hq, Sq, D] (the reference's "API promise", :593-596);
* the logsumexp is real (natural log, [B, Hq, Sq] fp32); the reference
  leaves it uninitialised (:584-586).

A row whose keys are all masked gives zeros (torch's CPU SDPA), not the NaN
of the reference's plain softmax.  All work runs in the HIP kernels of
``spyre_sdpa_fwd_f16``, called by the C++ kernels of ``spyre::sdpa_fwd`` and
of the aten op (csrc/torch_ops.cpp), or here through the C ABI by the
prepared ``SdpaCall`` and calls given a workspace.
"""

from __future__ import annotations

import math
from collections import OrderedDict
from typing import Optional

import torch

from . import _lib
from .relayout import _require_cuda, _require_on, _stream_ptr

MASK_NONE, MASK_F16, MASK_F32, MASK_BOOL = 0, 1, 2, 3
_MASK_KIND = {torch.float16: MASK_F16, torch.float32: MASK_F32, torch.bool: MASK_BOOL, torch.uint8: MASK_BOOL}


class Unsupported(RuntimeError):
    """An SDPA feature the device path does not implement (the reference's
    ``torch_spyre._inductor.errors.Unsupported``, errors.py:16)."""


def workspace_bytes(B: int, Hkv: int, Skv: int, D: int) -> int:
    return int(_lib.lib().spyre_sdpa_fwd_workspace_bytes(B, Hkv, Skv, D))


def _kernel_ready(t: torch.Tensor) -> bool:
    """Rows the kernel can read as 16-byte vectors: feature stride 1, other
    strides multiples of 8, 16-byte aligned."""
    st = t.stride()
    return st[3] == 1 and st[0] % 8 == 0 and st[1] % 8 == 0 and st[2] % 8 == 0 and t.data_ptr() % 16 == 0


def _operand(t: torch.Tensor, name: str, copy: bool = True) -> torch.Tensor:
    """fp16 CUDA [B, H, S, D] in kernel form; anything else is copied into
    that form first (copy=False: refused instead)."""
    if not t.is_cuda:
        _require_cuda(t, name)
    if t.dim() != 4:
        raise ValueError(f"{name} must be 4-D [B, H, S, D]")
    if t.dtype != torch.float16:
        raise TypeError(f"{name} must be float16 (got {t.dtype})")
    if _kernel_ready(t):
        return t
    if not copy:
        raise ValueError(f"{name} needs feature stride 1, other strides multiples of 8 and 16-byte alignment")
    # contiguous() would hand back a tensor torch already counts as
    # contiguous (odd strides on size-1 dims, an unaligned storage offset)
    return t.clone(memory_format=torch.contiguous_format)


# What a call needs that depends only on its geometry -- the stride arrays
# handed to the library and the workspace size -- kept per geometry, so a
# repeated call builds neither again.
_PLANS: "OrderedDict[tuple, tuple]" = OrderedDict()
_PLANS_MAX = 256


def _geometry_plan(q, k, v, mask, kind: int, is_causal: bool):
    key = (q.shape, q.stride(), k.shape, k.stride(), v.stride(), kind, bool(is_causal), q.device.index,
           None if mask is None else (mask.stride(), mask.data_ptr() % 16))
    plan = _PLANS.get(key)
    if plan is not None:
        _PLANS.move_to_end(key)
        return plan
    B, Hq, Sq, D = q.shape
    _, Hkv, Skv, _ = k.shape
    mstrides = _lib.i64_array(mask.stride()) if mask is not None else None
    # The call's workspace: without a mask, a key split's partials when the
    # blocks would not fill the device (none for causal calls); none for
    # masks the kernel stages as they lie, a copy with 16-byte rows for other
    # fp16 / bool masks, V's relayout for fp32 masks.
    need = 0
    if kind != MASK_NONE or not is_causal:
        need = int(_lib.lib().spyre_sdpa_fwd_call_workspace_bytes(
            mask.data_ptr() if mask is not None else None, kind, mstrides, B, Hq, Hkv, Sq, Skv, D))
    plan = (_lib.i64_array(q.stride()[:3]), _lib.i64_array(k.stride()[:3]), _lib.i64_array(v.stride()[:3]),
            mstrides, need)
    _PLANS[key] = plan
    if len(_PLANS) > _PLANS_MAX:
        _PLANS.popitem(last=False)
    return plan


def _prepare(query, key, value, attn_mask, dropout_p, is_causal, scale, enable_gqa, return_lse, workspace,
             copy_operands: bool):
    """Validates a call and allocates its output: (library arguments less
    the stream, output view, lse, tensors the arguments point into)."""
    q = _operand(query, "query", copy_operands)
    k = _operand(key, "key", copy_operands)
    v = _operand(value, "value", copy_operands)
    _require_on(k, q.device, "key")
    _require_on(v, q.device, "value")
    B, Hq, Sq, D = q.shape
    Bk, Hkv, Skv, Dk = k.shape
    if v.shape != k.shape or Bk != B or Dk != D:
        raise ValueError("key/value must be [B, Hkv, Skv, D] matching query")
    if Hq != Hkv and not enable_gqa:
        raise ValueError("Hq != Hkv requires enable_gqa=True")
    if Hq % Hkv:
        raise ValueError(f"Hq={Hq} is not a multiple of Hkv={Hkv}")
    if dropout_p > 0.0:
        raise Unsupported("Attention dropout not implemented")
    if is_causal and attn_mask is not None:
        raise ValueError("is_causal and attn_mask are exclusive")
    kind, mask = MASK_NONE, None
    if attn_mask is not None:
        m = torch.as_tensor(attn_mask, device=q.device)
        if m.dtype not in _MASK_KIND:
            raise TypeError(f"attn_mask dtype {m.dtype} not supported (float16, float32, bool)")
        kind = _MASK_KIND[m.dtype]
        mask = m.expand(B, Hq, Sq, Skv)
        if mask.dtype == torch.bool:
            mask = mask.view(torch.uint8)
    qs, ks, vs, mstrides, need = _geometry_plan(q, k, v, mask, kind, is_causal)
    s = 1.0 / math.sqrt(D) if scale is None else float(scale)
    out = torch.empty((B, Sq, Hq, D), dtype=torch.float16, device=q.device)
    lse = torch.empty((B, Hq, Sq), dtype=torch.float32, device=q.device) if return_lse else None
    if workspace is not None:
        _require_on(workspace, q.device, "workspace")
    if workspace is None and need:
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
    elif workspace is not None and need and kind != MASK_NONE:
        # a workspace that holds V's relayout also serves (the fp32-mask kernel runs)
        floor = min(need, workspace_bytes(B, Hkv, Skv, D))
        if workspace.numel() * workspace.element_size() < floor:
            raise ValueError(f"workspace holds {workspace.numel() * workspace.element_size()} bytes, need {floor}")
    ws_ptr = workspace.data_ptr() if workspace is not None else None
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    args = (q.data_ptr(), qs, k.data_ptr(), ks, v.data_ptr(), vs, mask.data_ptr() if mask is not None else None,
            kind, mstrides, int(bool(is_causal)), s, out.data_ptr(), lse.data_ptr() if lse is not None else None,
            ws_ptr, ws_bytes, B, Hq, Hkv, Sq, Skv, D)
    return args, out.transpose(1, 2), lse, (q, k, v, mask, workspace)


_SDPA_FWD = torch.ops.spyre.sdpa_fwd.default


def scaled_dot_product_attention(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                                 attn_mask: Optional[torch.Tensor] = None, dropout_p: float = 0.0,
                                 is_causal: bool = False, scale: Optional[float] = None,
                                 enable_gqa: bool = False, return_lse: bool = False,
                                 workspace: Optional[torch.Tensor] = None):
    """``F.scaled_dot_product_attention`` on fp16 CUDA tensors: query
    [B, Hq, Sq, D], key/value [B, Hkv, Skv, D], D in {64, 128}.

    Runs the C++ kernel of ``spyre::sdpa_fwd`` (checks, outputs and the
    call's workspace from the caching allocator, launch on the current
    stream); with a ``workspace`` of the caller's, the library call is made
    here with that workspace."""
    if dropout_p > 0.0:
        raise Unsupported("Attention dropout not implemented")
    if workspace is not None:
        args, out, lse, _ = _prepare(query, key, value, attn_mask, dropout_p, is_causal, scale, enable_gqa,
                                     return_lse, workspace, True)
        _lib.check("spyre_sdpa_fwd_f16", _lib.lib().spyre_sdpa_fwd_f16(*args, _stream_ptr(query.device)))
        return (out, lse) if return_lse else out
    if attn_mask is not None and not isinstance(attn_mask, torch.Tensor):
        attn_mask = torch.as_tensor(attn_mask, device=query.device)
    try:
        out, lse = _SDPA_FWD(query, key, value, attn_mask, is_causal, scale, enable_gqa, return_lse)
    except RuntimeError as e:
        raise _lib.library_error(e) from None
    return (out, lse) if return_lse else out


class SdpaCall:
    """A validated ``scaled_dot_product_attention`` that can be launched
    repeatedly, the dense counterpart of ``PagedDecode``: shapes, strides,
    the workspace and the output are settled once, and each call only passes
    the stored pointers to the library.  The operands must already be in
    kernel form (feature stride 1, other strides multiples of 8, 16-byte
    aligned; no copy is made) and must stay alive with their storage; the
    caller may rewrite their contents between calls.  Every call writes the
    same ``out`` (and ``lse``), on the stream current at that moment, so the
    calls can be captured into a HIP graph (the library allocates and clears
    nothing)."""

    def __init__(self, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                 attn_mask: Optional[torch.Tensor] = None, is_causal: bool = False, scale: Optional[float] = None,
                 enable_gqa: bool = False, return_lse: bool = False, workspace: Optional[torch.Tensor] = None):
        self._args, self.out, self.lse, self._keep = _prepare(query, key, value, attn_mask, 0.0, is_causal,
                                                              scale, enable_gqa, return_lse, workspace, False)
        self._fn = _lib.lib().spyre_sdpa_fwd_f16
        self._device = query.device
        self._return_lse = return_lse

    def __call__(self):
        _lib.check("spyre_sdpa_fwd_f16", self._fn(*self._args, _stream_ptr(self._device)))
        return (self.out, self.lse) if self._return_lse else self.out


def sdpa_overrideable(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                      attn_bias: Optional[torch.Tensor] = None, dropout_p: float = 0.0,
                      is_causal: bool = False, return_debug_mask: bool = False,
                      scale: Optional[float] = None):
    """The 9-tuple of ``_scaled_dot_product_fused_attention_overrideable``
    (torch_spyre/_inductor/decompositions.py:523-609): (output, logsumexp,
    cum_seq_q, cum_seq_k, max_q, max_k, philox_seed, philox_offset,
    debug_attn_mask), from the op's CUDA kernel.  GQA follows from the head
    counts; dropout raises ``Unsupported`` as the reference does."""
    if dropout_p > 0.0:
        raise Unsupported("Attention dropout not implemented")
    try:
        return _OVERRIDEABLE(query, key, value, attn_bias, dropout_p, is_causal, return_debug_mask, scale=scale)
    except RuntimeError as e:
        raise _lib.library_error(e) from None


_OVERRIDEABLE = torch.ops.aten._scaled_dot_product_fused_attention_overrideable.default


class sdpa_override(torch.overrides.TorchFunctionMode):
    """Inside this context, ``torch.nn.functional.scaled_dot_product_attention``
    calls this module can serve (CUDA float16 q / k / v, D in {64, 128},
    Hq a multiple of Hkv, no dropout, masks of float16 / float32 / bool)
    run the HIP kernels; any other call runs torch's own.

    The reference gets the same effect by making ``_fused_sdp_choice``
    answer "overrideable" for its device (torch_spyre/csrc/attn_utils.cpp:22-37);
    CUDA tensors keep torch's choice outside this context."""

    def __torch_function__(self, func, types, args=(), kwargs=None):
        kwargs = kwargs or {}
        if func is torch.nn.functional.scaled_dot_product_attention and _servable(*args, **kwargs):
            return scaled_dot_product_attention(*args, **kwargs)
        return func(*args, **kwargs)


def _servable(query, key, value, attn_mask=None, dropout_p=0.0, is_causal=False, scale=None,
              enable_gqa=False) -> bool:
    ts = (query, key, value)
    if not all(isinstance(t, torch.Tensor) and t.is_cuda and t.dtype == torch.float16 and t.dim() == 4 for t in ts):
        return False
    if query.shape[-1] not in (64, 128) or key.shape[-1] != query.shape[-1] or dropout_p > 0.0:
        return False
    # value must match key exactly and the batch must match query: torch
    # serves other shapes (another value head dim, broadcast batch dims)
    if value.shape != key.shape or query.shape[0] != key.shape[0]:
        return False
    if not (query.device == key.device == value.device):
        return False
    if key.shape[1] == 0 or query.shape[1] % key.shape[1] or (query.shape[1] != key.shape[1] and not enable_gqa):
        return False
    if attn_mask is not None and (is_causal or not isinstance(attn_mask, torch.Tensor)
                                  or attn_mask.dtype not in _MASK_KIND):
        return False
    return True
