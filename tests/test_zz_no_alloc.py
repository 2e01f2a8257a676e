"""spyre_paged_decode_attn_noalloc_f16: the decode entry point whose chunk
partials live in the library's own per-GPU scratch array instead of a
caller-provided workspace.

Checked through the C ABI against spyre_paged_decode_attn_f16 with a
workspace (the same kernels, so bit-identical output and LSE) on two calls
in a row, the second with a smaller batch and shorter contexts, both long
enough for several chunks (more than 4096 tokens per chunk at split 512),
so the scratch carries the partials and the arrival flags of the chunks'
merge.  A call whose partials exceed the scratch is refused before it
reaches the device.
"""

import pytest
import torch

from tests.conftest import SEED
from tests.test_attention_gpu import make_case

pytestmark = pytest.mark.gpu

PAGE = 64


def _ptr(t):
    return t.data_ptr() if t is not None else None


def _call(fn, cache, table, lens, q, out, lse, max_ctx, workspace=None, split=512):
    from torch_spyre_amd import _lib

    B, Hq, D = q.shape
    stream = torch.cuda.current_stream(q.device).cuda_stream
    common = (_ptr(q), _ptr(cache.k), _ptr(cache.v), _ptr(table), table.stride(0), _ptr(lens), _ptr(out),
              _ptr(lse))
    tail = (B, Hq, cache.Hkv, D, PAGE, cache.num_pages, max_ctx, split, 1.0 / D ** 0.5, stream)
    if workspace is None:
        rc = fn(*common, *tail)
    else:
        rc = fn(*common, _ptr(workspace), workspace.numel(), *tail)
    _lib.check(fn.__name__, rc)


@pytest.mark.parametrize("calls", [[(6, [20000, 9000, 4097, 130, 16000, 12345]), (3, [9000, 4500, 5000])]])
def test_noalloc_matches_workspace_entry(cuda, calls):
    from torch_spyre_amd import _lib

    L = _lib.lib()
    for i, (B, ctx) in enumerate(calls):
        cache, table, lens, q = make_case(cuda, B, 32, 8, 128, ctx, SEED + 90 + i)
        table, lens = table.to(cuda), lens.to(cuda)
        max_ctx = max(ctx)
        need = L.spyre_paged_decode_attn_workspace_bytes(B, 32, 8, 128, max_ctx, 512)
        assert 0 < need <= 16 << 20
        ws = torch.empty(need, dtype=torch.uint8, device=cuda)
        out_ref = torch.empty_like(q)
        lse_ref = torch.empty((B, 32), dtype=torch.float32, device=cuda)
        _call(L.spyre_paged_decode_attn_f16, cache, table, lens, q, out_ref, lse_ref, max_ctx, workspace=ws)
        out = torch.full_like(q, float("nan"))
        lse = torch.full((B, 32), float("nan"), dtype=torch.float32, device=cuda)
        _call(L.spyre_paged_decode_attn_noalloc_f16, cache, table, lens, q, out, lse, max_ctx)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), out_ref.view(torch.int16)), f"call {i}: output differs"
        assert torch.equal(lse.view(torch.int32), lse_ref.view(torch.int32)), f"call {i}: LSE differs"


def test_noalloc_refuses_oversized_call(cuda):
    """B 64, 32 / 8 heads, D 128 at 131072 tokens needs 34 MB of partials:
    refused with SPYRE_ENOSPC and a message naming both sizes."""
    from torch_spyre_amd import _lib

    L = _lib.lib()
    need = L.spyre_paged_decode_attn_workspace_bytes(64, 32, 8, 128, 131072, 512)
    assert need > 16 << 20
    dummy = torch.empty(16, dtype=torch.float16, device=cuda)
    p = dummy.data_ptr()
    rc = L.spyre_paged_decode_attn_noalloc_f16(p, p, p, p, 2048, p, p, None, 64, 32, 8, 128, PAGE, 1, 131072,
                                               512, 0.1, None)
    assert rc == _lib.SPYRE_ENOSPC
    msg = L.spyre_last_error().decode()
    assert str(need) in msg and str(16 << 20) in msg
