// Batched KV-cache append into the paged stick-layout cache
// (spyre_kv_append_f16): the new token of every sequence is written into its
// page slot in one launch, with the positions read from device memory.
//
//   K cache [num_pages, Hkv, D/64, 64 tok, 64]: the token's D values land as
//     D/64 partial-stick writes of 128 contiguous bytes each;
//   V cache [num_pages, Hkv, D, 64 tok]: the token is one column of the
//     page's D sticks (the transposed, relayout-on-write half).
//
// Positions < 0 skip the sequence; positions past the block table's row and
// page ids outside [0, num_pages) are not written (dropped rather than faulting).

#include <hip/hip_runtime.h>

#include "spyre_common.h"

namespace {

constexpr int kPage = 64;

__global__ void kv_append_kernel(const _Float16* __restrict__ k_new,
                                 const _Float16* __restrict__ v_new, _Float16* __restrict__ kc,
                                 _Float16* __restrict__ vc, const int32_t* __restrict__ bt,
                                 int64_t bt_stride, int64_t pages_per_seq,
                                 const int32_t* __restrict__ pos, int Hkv, int D,
                                 int64_t num_pages) {
  const int h = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
  const int p = pos[b];
  if (p < 0 || p / kPage >= pages_per_seq) return;
  const int64_t page = bt[static_cast<int64_t>(b) * bt_stride + p / kPage];
  if (page < 0 || page >= num_pages) return;
  const int slot = p % kPage;
  const int64_t src = (static_cast<int64_t>(b) * Hkv + h) * D + d;
  const int64_t head = (page * Hkv + h) * static_cast<int64_t>(D) * kPage;
  kc[head + (d / 64) * (kPage * 64) + slot * 64 + (d % 64)] = k_new[src];
  vc[head + static_cast<int64_t>(d) * kPage + slot] = v_new[src];
}

}  // namespace

extern "C" int spyre_kv_append_f16(const void* k_new, const void* v_new, void* k_cache,
                                   void* v_cache, const int32_t* block_table, int64_t bt_stride,
                                   int64_t pages_per_seq, const int32_t* positions, int B, int Hkv,
                                   int D, int page_size, int64_t num_pages, void* stream) {
  spyre_hip::clear_error();
  SPYRE_REQUIRE(k_new && v_new && k_cache && v_cache && block_table && positions, SPYRE_EINVAL,
                "null pointer argument");
  SPYRE_REQUIRE(B >= 0 && Hkv > 0 && num_pages > 0 && bt_stride >= 0 && pages_per_seq >= 0,
                SPYRE_EINVAL,
                "bad sizes B=%d Hkv=%d num_pages=%lld", B, Hkv, static_cast<long long>(num_pages));
  SPYRE_REQUIRE(D == 64 || D == 128, SPYRE_EUNSUPPORTED, "head_dim %d not in {64, 128}", D);
  SPYRE_REQUIRE(page_size == kPage, SPYRE_EUNSUPPORTED, "page_size %d != %d", page_size, kPage);
  if (B == 0) return SPYRE_OK;
  kv_append_kernel<<<dim3(Hkv, B), D, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const _Float16*>(k_new), static_cast<const _Float16*>(v_new),
      static_cast<_Float16*>(k_cache), static_cast<_Float16*>(v_cache), block_table, bt_stride,
      pages_per_seq, positions, Hkv, D, num_pages);
  const hipError_t e = hipGetLastError();
  SPYRE_REQUIRE(e == hipSuccess, SPYRE_EHIP, "kv append launch failed: %s", hipGetErrorString(e));
  return SPYRE_OK;
}
