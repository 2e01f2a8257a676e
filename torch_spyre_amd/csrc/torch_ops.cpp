// PyTorch-ROCm kernels of the attention and KV-cache ops, calling the C ABI
// of libspyre_hip.so directly: the eager path of a reference caller
// (torch.ops.spyre.*, aten::_scaled_dot_product_fused_attention_overrideable)
// checks its tensors, allocates its outputs and workspace from the caching
// allocator and launches on the current stream without a Python frame in
// between.
//
//   spyre::sdpa_fwd                SDPA forward with logsumexp (any Sq)
//   aten::_scaled_dot_product_fused_attention_overrideable   CUDA kernel:
//       the 9-tuple of torch_spyre/_inductor/decompositions.py:523-609
//       (selected by _fused_sdp_choice, torch_spyre/csrc/attn_utils.cpp:22-37)
//   spyre::paged_decode_attention  paged split-KV decode (no reference counterpart)
//   spyre::kv_append               batched paged-cache write (no reference counterpart)
//
// Argument errors raise ValueError / TypeError (TORCH_CHECK_VALUE / _TYPE);
// a failure the library reports raises RuntimeError whose message starts
// "[spyre_hip <entry point> <code>]" (the Python layer re-raises it as
// SpyreHipError).  Dropout raises NotImplementedError, as the reference's
// decomposition refuses it (decompositions.py:578-580).

#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include <cmath>
#include <cstdint>

#include "../../include/spyre_hip.h"

namespace {

void* stream_of(const at::Tensor& t) {
  return static_cast<void*>(c10::hip::getCurrentHIPStream(t.device().index()).stream());
}

void check_rc(const char* fn, int rc) {
  if (rc != SPYRE_OK) {
    const char* msg = spyre_last_error();
    TORCH_CHECK(false, "[spyre_hip ", fn, " ", rc, "] ", msg ? msg : "");
  }
}

// fp16 CUDA [B, H, S, D] whose rows the kernels read as 16-byte vectors:
// feature stride 1, other strides multiples of 8, 16-byte aligned; anything
// else is copied into that form.
at::Tensor sdpa_operand(const at::Tensor& t, const char* name) {
  TORCH_CHECK_VALUE(t.is_cuda(), name, " must be a CUDA (HIP) tensor; there is no CPU path");
  TORCH_CHECK_VALUE(t.dim() == 4, name, " must be 4-D [B, H, S, D]");
  TORCH_CHECK_TYPE(t.scalar_type() == at::kHalf, name, " must be float16 (got ", t.scalar_type(), ")");
  const auto st = t.strides();
  const bool ready = st[3] == 1 && st[0] % 8 == 0 && st[1] % 8 == 0 && st[2] % 8 == 0 &&
                     reinterpret_cast<uintptr_t>(t.data_ptr()) % 16 == 0;
  // contiguous() would keep a tensor torch counts as contiguous (odd strides
  // on size-1 dims, an unaligned storage offset)
  return ready ? t : t.clone(at::MemoryFormat::Contiguous);
}

std::tuple<at::Tensor, at::Tensor> sdpa_fwd(const at::Tensor& query, const at::Tensor& key, const at::Tensor& value,
                                            const std::optional<at::Tensor>& attn_mask, bool is_causal,
                                            std::optional<double> scale, bool enable_gqa, bool return_lse) {
  const at::Tensor q = sdpa_operand(query, "query");
  const at::Tensor k = sdpa_operand(key, "key");
  const at::Tensor v = sdpa_operand(value, "value");
  const int64_t B = q.size(0), Hq = q.size(1), Sq = q.size(2), D = q.size(3);
  const int64_t Hkv = k.size(1), Skv = k.size(2);
  TORCH_CHECK_VALUE(v.sizes() == k.sizes() && k.size(0) == B && k.size(3) == D,
                    "key/value must be [B, Hkv, Skv, D] matching query");
  TORCH_CHECK_VALUE(q.device() == k.device() && q.device() == v.device(), "query, key and value on different devices");
  TORCH_CHECK_VALUE(Hq == Hkv || enable_gqa, "Hq != Hkv requires enable_gqa=True");
  TORCH_CHECK_VALUE(Hkv > 0 && Hq % Hkv == 0, "Hq=", Hq, " is not a multiple of Hkv=", Hkv);
  TORCH_CHECK_VALUE(!(is_causal && attn_mask.has_value()), "is_causal and attn_mask are exclusive");
  const c10::OptionalDeviceGuard guard(q.device());
  int kind = SPYRE_MASK_NONE;
  at::Tensor mask;
  int64_t mstrides[4] = {0, 0, 0, 0};
  if (attn_mask.has_value()) {
    at::Tensor m = *attn_mask;
    TORCH_CHECK_VALUE(m.device() == q.device(), "attn_mask must be on the query's device");
    switch (m.scalar_type()) {
      case at::kHalf: kind = SPYRE_MASK_F16; break;
      case at::kFloat: kind = SPYRE_MASK_F32; break;
      case at::kBool:
      case at::kByte: kind = SPYRE_MASK_BOOL; break;
      default: TORCH_CHECK_TYPE(false, "attn_mask dtype ", m.scalar_type(), " not supported (float16, float32, bool)");
    }
    mask = m.expand({B, Hq, Sq, Skv});
    if (mask.scalar_type() == at::kBool) mask = mask.view(at::kByte);
    for (int i = 0; i < 4; ++i) mstrides[i] = mask.stride(i);
  }
  const double s = scale.has_value() ? *scale : 1.0 / std::sqrt(static_cast<double>(D));
  const auto f16 = q.options();
  at::Tensor out = at::empty({B, Sq, Hq, D}, f16);
  at::Tensor lse = at::empty({return_lse ? B : 0, Hq, Sq}, f16.dtype(at::kFloat));
  const int64_t qs[3] = {q.stride(0), q.stride(1), q.stride(2)};
  const int64_t ks[3] = {k.stride(0), k.stride(1), k.stride(2)};
  const int64_t vs[3] = {v.stride(0), v.stride(1), v.stride(2)};
  // The call's workspace (none for causal calls without a mask).
  size_t need = 0;
  if (kind != SPYRE_MASK_NONE || !is_causal)
    need = spyre_sdpa_fwd_call_workspace_bytes(kind != SPYRE_MASK_NONE ? mask.data_ptr() : nullptr, kind,
                                               kind != SPYRE_MASK_NONE ? mstrides : nullptr, B, Hq, Hkv, Sq, Skv, D);
  at::Tensor ws = need ? at::empty({static_cast<int64_t>(need)}, f16.dtype(at::kByte)) : at::Tensor();
  check_rc("spyre_sdpa_fwd_f16",
           spyre_sdpa_fwd_f16(q.data_ptr(), qs, k.data_ptr(), ks, v.data_ptr(), vs,
                              kind != SPYRE_MASK_NONE ? mask.data_ptr() : nullptr, kind,
                              kind != SPYRE_MASK_NONE ? mstrides : nullptr, is_causal ? 1 : 0,
                              static_cast<float>(s), out.data_ptr(), return_lse ? lse.data_ptr<float>() : nullptr,
                              need ? ws.data_ptr() : nullptr, need, B, Hq, Hkv, Sq, Skv, D, stream_of(q)));
  return {out.transpose(1, 2), lse};
}

// aten::_scaled_dot_product_fused_attention_overrideable's CUDA kernel: the
// 9-tuple (output, logsumexp, cum_seq_q, cum_seq_k, max_q, max_k,
// philox_seed, philox_offset, debug_attn_mask) with a real logsumexp.
std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor, c10::SymInt, c10::SymInt, at::Tensor, at::Tensor, at::Tensor>
sdpa_overrideable(const at::Tensor& query, const at::Tensor& key, const at::Tensor& value,
                  const std::optional<at::Tensor>& attn_bias, double dropout_p, bool is_causal, bool return_debug_mask,
                  std::optional<double> scale) {
  TORCH_CHECK_NOT_IMPLEMENTED(dropout_p == 0.0, "Attention dropout not implemented");
  TORCH_CHECK_VALUE(query.dim() == 4 && key.dim() == 4, "query and key must be 4-D [B, H, S, D]");
  auto [out, lse] = sdpa_fwd(query, key, value, attn_bias, is_causal, scale, query.size(1) != key.size(1), true);
  // the philox placeholders, [1] fp16 each as the reference returns them
  // (decompositions.py:586-587): views of one allocation
  const at::Tensor ph = at::empty({2}, query.options().dtype(at::kHalf));
  return {out, lse, at::Tensor(), at::Tensor(), c10::SymInt(query.size(2)), c10::SymInt(key.size(2)),
          ph.narrow(0, 0, 1), ph.narrow(0, 1, 1), at::Tensor()};
}

constexpr int64_t kPage = 64;

// t must be a CUDA tensor on `dev`: a kernel launched there reads or writes
// it through its pointer (a host pointer would fault there).
void require_on(const at::Tensor& t, const c10::Device& dev, const char* name) {
  TORCH_CHECK_VALUE(t.is_cuda(), name, " must be a CUDA (HIP) tensor; there is no CPU path");
  TORCH_CHECK_VALUE(t.device() == dev, name, " is on ", t.device(), "; the call runs on ", dev);
}

int64_t check_cache(const at::Tensor& kc, const at::Tensor& vc, int64_t Hkv, int64_t D) {
  for (const at::Tensor* t : {&kc, &vc}) {
    TORCH_CHECK_VALUE(t->is_cuda(), "caches must be CUDA (HIP) tensors");
    TORCH_CHECK_VALUE(t->scalar_type() == at::kHalf && t->is_contiguous(), "caches must be contiguous float16");
  }
  const int64_t per_page = Hkv * D * kPage;
  TORCH_CHECK_VALUE(kc.numel() % per_page == 0 && kc.numel() == vc.numel(),
                    "caches must hold whole pages of ", per_page, " elements (Hkv=", Hkv, ", D=", D, ")");
  TORCH_CHECK_VALUE(kc.dim() < 2 || kc.size(1) == Hkv, "k_cache has ", kc.size(1), " KV heads, expected ", Hkv);
  return kc.numel() / per_page;
}

std::tuple<at::Tensor, at::Tensor> paged_decode_attention(const at::Tensor& q, const at::Tensor& k_cache,
                                                          const at::Tensor& v_cache, const at::Tensor& block_table,
                                                          const at::Tensor& context_lens, double scale,
                                                          int64_t split_tokens, int64_t max_context_len) {
  TORCH_CHECK_VALUE(q.is_cuda(), "q must be a CUDA (HIP) tensor; there is no CPU path");
  TORCH_CHECK_VALUE(q.scalar_type() == at::kHalf && q.dim() == 3 && q.is_contiguous(),
                    "q must be contiguous float16 [B, Hq, D]");
  const int64_t B = q.size(0), Hq = q.size(1), D = q.size(2);
  TORCH_CHECK_VALUE(k_cache.dim() >= 2, "k_cache must be [num_pages, Hkv, ...]");
  const int64_t Hkv = k_cache.size(1);
  TORCH_CHECK_VALUE(Hkv > 0 && Hq % Hkv == 0, "Hq=", Hq, " is not a multiple of Hkv=", Hkv);
  const int64_t num_pages = check_cache(k_cache, v_cache, Hkv, D);
  require_on(k_cache, q.device(), "k_cache");
  require_on(v_cache, q.device(), "v_cache");
  require_on(block_table, q.device(), "block_table");
  require_on(context_lens, q.device(), "context_lens");
  TORCH_CHECK_VALUE(block_table.scalar_type() == at::kInt && block_table.dim() == 2 && block_table.size(0) == B &&
                        block_table.stride(1) == 1 && block_table.is_cuda(),
                    "block_table must be a CUDA int32 [B, W] tensor with unit column stride");
  TORCH_CHECK_VALUE(context_lens.scalar_type() == at::kInt && context_lens.dim() == 1 && context_lens.size(0) == B &&
                        context_lens.is_contiguous() && context_lens.is_cuda(),
                    "context_lens must be a contiguous CUDA int32 [B] tensor");
  const c10::OptionalDeviceGuard guard(q.device());
  if (max_context_len < 0) max_context_len = B ? context_lens.max().item<int32_t>() : 0;  // synchronises
  TORCH_CHECK_VALUE(max_context_len <= block_table.size(1) * kPage, "max_context_len ", max_context_len,
                    " exceeds the block table's ", block_table.size(1), " pages");
  const size_t need = spyre_paged_decode_attn_workspace_bytes(B, Hq, Hkv, D, max_context_len, split_tokens);
  at::Tensor ws = at::empty({static_cast<int64_t>(std::max<size_t>(need, 4))}, q.options().dtype(at::kByte));
  at::Tensor out = at::empty_like(q);
  at::Tensor lse = at::empty({B, Hq}, q.options().dtype(at::kFloat));
  check_rc("spyre_paged_decode_attn_f16",
           spyre_paged_decode_attn_f16(q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
                                       block_table.data_ptr<int32_t>(), block_table.stride(0),
                                       context_lens.data_ptr<int32_t>(), out.data_ptr(), lse.data_ptr<float>(),
                                       ws.data_ptr(), ws.numel(), B, Hq, Hkv, D, kPage, num_pages, max_context_len,
                                       split_tokens, static_cast<float>(scale), stream_of(q)));
  return {out, lse};
}

void kv_append(const at::Tensor& k_new, const at::Tensor& v_new, const at::Tensor& k_cache, const at::Tensor& v_cache,
               const at::Tensor& block_table, const at::Tensor& positions) {
  for (const at::Tensor* t : {&k_new, &v_new}) {
    TORCH_CHECK_VALUE(t->is_cuda(), "k_new / v_new must be CUDA (HIP) tensors");
    TORCH_CHECK_VALUE(t->scalar_type() == at::kHalf && t->dim() == 3 && t->is_contiguous(),
                      "k_new / v_new must be contiguous float16 [B, Hkv, D]");
  }
  TORCH_CHECK_VALUE(v_new.sizes() == k_new.sizes(), "k_new and v_new shapes differ");
  const int64_t B = k_new.size(0), Hkv = k_new.size(1), D = k_new.size(2);
  const int64_t num_pages = check_cache(k_cache, v_cache, Hkv, D);
  require_on(v_new, k_new.device(), "v_new");
  require_on(k_cache, k_new.device(), "k_cache");
  require_on(v_cache, k_new.device(), "v_cache");
  require_on(block_table, k_new.device(), "block_table");
  require_on(positions, k_new.device(), "positions");
  TORCH_CHECK_VALUE(block_table.scalar_type() == at::kInt && block_table.dim() == 2 && block_table.size(0) == B &&
                        block_table.stride(1) == 1,
                    "block_table must be int32 [B, pages_per_seq] with unit column stride");
  TORCH_CHECK_VALUE(positions.scalar_type() == at::kInt && positions.dim() == 1 && positions.size(0) == B &&
                        positions.is_contiguous(),
                    "positions must be contiguous int32 [B]");
  const c10::OptionalDeviceGuard guard(k_new.device());
  check_rc("spyre_kv_append_f16",
           spyre_kv_append_f16(k_new.data_ptr(), v_new.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
                               block_table.data_ptr<int32_t>(), block_table.stride(0), block_table.size(1),
                               positions.data_ptr<int32_t>(), B, Hkv, D, kPage, num_pages, stream_of(k_new)));
}

}  // namespace

TORCH_LIBRARY_FRAGMENT(spyre, m) {
  m.def("sdpa_fwd(Tensor query, Tensor key, Tensor value, Tensor? attn_mask=None, bool is_causal=False, "
        "float? scale=None, bool enable_gqa=False, bool return_lse=True) -> (Tensor, Tensor)");
  m.def("paged_decode_attention(Tensor q, Tensor k_cache, Tensor v_cache, Tensor block_table, "
        "Tensor context_lens, float scale, int split_tokens=512, int max_context_len=-1) -> (Tensor, Tensor)");
  m.def("kv_append(Tensor k_new, Tensor v_new, Tensor(a!) k_cache, Tensor(b!) v_cache, Tensor block_table, "
        "Tensor positions) -> ()");
}

TORCH_LIBRARY_IMPL(spyre, CUDA, m) {
  m.impl("sdpa_fwd", &sdpa_fwd);
  m.impl("paged_decode_attention", &paged_decode_attention);
  m.impl("kv_append", &kv_append);
}

TORCH_LIBRARY_IMPL(aten, CUDA, m) {
  m.impl("_scaled_dot_product_fused_attention_overrideable", &sdpa_overrideable);
}
