"""CPU: the C++ kernels of libspyre_torch.so are registered -- the spyre::
op schemas, their CUDA kernels and fake kernels, and the CUDA kernel of
aten::_scaled_dot_product_fused_attention_overrideable -- and there is no
CPU kernel (calls on CPU tensors raise).  No GPU is used."""

import pytest
import torch


@pytest.fixture(scope="module")
def tsa():
    import torch_spyre_amd

    return torch_spyre_amd


SCHEMAS = {
    "sdpa_fwd": "spyre::sdpa_fwd(Tensor query, Tensor key, Tensor value, Tensor? attn_mask=None, "
                "bool is_causal=False, float? scale=None, bool enable_gqa=False, bool return_lse=True) "
                "-> (Tensor, Tensor)",
    "paged_decode_attention": "spyre::paged_decode_attention(Tensor q, Tensor k_cache, Tensor v_cache, "
                              "Tensor block_table, Tensor context_lens, float scale, int split_tokens=512, "
                              "int max_context_len=-1) -> (Tensor, Tensor)",
    "kv_append": "spyre::kv_append(Tensor k_new, Tensor v_new, Tensor(a!) k_cache, Tensor(b!) v_cache, "
                 "Tensor block_table, Tensor positions) -> ()",
}


@pytest.mark.parametrize("name", sorted(SCHEMAS))
def test_schema_and_kernels(tsa, name):
    op = getattr(torch.ops.spyre, name).default
    assert str(op._schema) == SCHEMAS[name]
    assert torch._C._dispatch_has_kernel_for_dispatch_key(op.name(), "CUDA")
    assert not torch._C._dispatch_has_kernel_for_dispatch_key(op.name(), "CPU")
    assert torch._C._dispatch_has_kernel_for_dispatch_key(op.name(), "Meta")  # the fake kernel


def test_aten_overrideable_cuda_kernel(tsa):
    name = "aten::_scaled_dot_product_fused_attention_overrideable"
    assert torch._C._dispatch_has_kernel_for_dispatch_key(name, "CUDA")


def test_cpu_tensors_have_no_kernel(tsa):
    q = torch.zeros(1, 2, 1, 64, dtype=torch.float16)
    with pytest.raises(NotImplementedError):
        torch.ops.spyre.sdpa_fwd(q, q, q)


def test_fake_shapes(tsa):
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        q = torch.empty(2, 8, 5, 64, dtype=torch.float16, device="cuda")
        k = torch.empty(2, 2, 7, 64, dtype=torch.float16, device="cuda")
        out, lse = torch.ops.spyre.sdpa_fwd(q, k, k, None, False, None, True)
        assert out.shape == (2, 8, 5, 64) and out.stride() == (5 * 8 * 64, 64, 8 * 64, 1)
        assert lse.shape == (2, 8, 5) and lse.dtype == torch.float32
        out, lse = torch.ops.spyre.sdpa_fwd(q, k, k, None, False, None, True, False)
        assert lse.shape == (0, 8, 5)
