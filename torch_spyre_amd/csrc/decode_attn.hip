// Split-KV paged decode attention for gfx950 (spyre_paged_decode_attn_f16).
//
// Semantics (one query token per sequence, GQA q head h -> KV head h / g):
//   out[b,h,:] = softmax(scale * q[b,h,:] . K[b,h/g,t,:]^T)_t  V[b,h/g,t,:],  t < ctx[b]
// as torch_spyre/_inductor/decompositions.py:523-609 computes it (there with
// the scale split as sqrt(scale) on q and k; here applied once in fp32).
//
// Cache layout (64-token pages, one page = 16 KiB per KV head and tensor):
//   K  [num_pages, Hkv, D/64, 64 tok, 64]   sticks along D    (QK^T reduces over D)
//   V  [num_pages, Hkv, D, 64 tok]          sticks along tokens (PV reduces over tokens)
// so that the reduction dim of both products is contiguous and every MFMA
// operand is one 16-byte load straight from HBM into VGPRs.
//
// Pass 1 (decode_split_kernel): one workgroup of 4 wavefronts per
// (sequence, KV head, split of `split_pages` pages).  The pages of a split
// rotate through the 4 wavefronts (the KV carousel); each wavefront streams a
// whole page per iteration:
//   S^T[tok, head] = K[tok, :] Q^T[:, head]   4 x 4 MFMA 16x16x32 (M = 16 tokens)
//   online softmax in fp32 (exp2 domain), row max across the 4 lane groups
//   of a head by lane shuffles;
//   O^T[d, head] += V^T[d, tok] P^T[tok, head]   D/16 x 2 MFMA 16x16x32
// The q heads of one KV head (g of them, padded to the MFMA's 16 columns)
// form the dense N dimension, so K and V are read once for all g heads.
// The token order of the QK rows is permuted so that each lane's P values
// are exactly the 8 consecutive tokens the PV B operand needs (no shuffles).
// The 4 wavefronts' (m, l, O) are merged through LDS and the split's partial
// is written to the workspace.
//
// Pass 2 (decode_merge_kernel): per (sequence, q head) combine the splits'
// partials -- the split-KV merge -- and write fp16 out (+ optional LSE).

#include <hip/hip_runtime.h>

#include <cmath>

#include "spyre_common.h"

namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kPage = 64;
constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kCols = 16;  // MFMA N: q heads per KV head, padded
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

__device__ __forceinline__ float wave_xor(float x, int m) { return __shfl_xor(x, m, 64); }

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

struct SplitArgs {
  const _Float16* q;
  const _Float16* k;
  const _Float16* v;
  const int32_t* block_table;
  int64_t bt_stride;
  const int32_t* ctx_lens;
  float* ws;
  int64_t num_pages;
  int Hq, Hkv, g, max_splits, split_pages, max_ctx;
  float scale_log2;
};

// ---- Operand loads: whole cache lines, then a lane shuffle --------------
//
// An MFMA 16x16x32 operand gives each row 4 lanes x 16 B = 64 B per
// instruction, i.e. half of a 128-byte stick; loading operands directly
// would make every load instruction touch 16 half lines.  Instead each
// instruction reads 8 whole sticks (8 lanes per stick) and two such loads X
// (rows 0-7) and Y (rows 8-15) are turned into the two operands of the
// stick's halves:
//   X lane l: row l&7,     chunk (l&8) ? 4 + (l>>4) : (l>>4)
//   Y lane l: row 8+(l&7), chunk (l&8) ? (l>>4) : 4 + (l>>4)
//   op0 = bit3 ? Y : X                 -> lane l: row l&15, chunk l>>4
//   op1 = ror8(bit3 ? X : Y)           -> lane l: row l&15, chunk 4 + (l>>4)
// where ror8 is the DPP row rotation by 8 (lane l reads lane l^8 of its
// 16-lane row).  A chunk is 16 B = 8 halves of the row.

__device__ __forceinline__ f16x8 ror8(f16x8 x) {
  typedef int i32x4 __attribute__((ext_vector_type(4)));
  i32x4 v = __builtin_bit_cast(i32x4, x);
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = __builtin_amdgcn_mov_dpp(v[i], 0x128, 0xf, 0xf, false);
  return __builtin_bit_cast(f16x8, v);
}

__device__ __forceinline__ int chunk_x(int lane) { return (lane & 8) ? 4 + (lane >> 4) : (lane >> 4); }
__device__ __forceinline__ int chunk_y(int lane) { return (lane & 8) ? (lane >> 4) : 4 + (lane >> 4); }

// Builds the operand pair from the raw X / Y loads (in place).
__device__ __forceinline__ void shuffle_pair(f16x8& x, f16x8& y, bool bit3) {
  const f16x8 op0 = bit3 ? y : x;
  const f16x8 op1 = ror8(bit3 ? x : y);
  x = op0;
  y = op1;
}

// QK block jh = (j, h): MFMA row i <-> token 32j + 8(i/4) + 4h + i%4.
__device__ __forceinline__ int qk_token(int jh, int i) {
  return 32 * (jh >> 1) + 8 * (i >> 2) + 4 * (jh & 1) + (i & 3);
}

// Raw K loads of one page: for block jh and stick tile t, X -> ka[jh][2t],
// Y -> ka[jh][2t+1] (operands after shuffle_pair: d = 32 ds + 8 (l>>4)).
template <int D>
__device__ __forceinline__ void load_k(f16x8 (&ka)[4][D / 32], const _Float16* kp, int lane) {
  const int cx = chunk_x(lane), cy = chunk_y(lane), r = lane & 7;
#pragma unroll
  for (int jh = 0; jh < 4; ++jh) {
    const int tx = qk_token(jh, r), ty = qk_token(jh, 8 + r);
#pragma unroll
    for (int t = 0; t < D / 64; ++t) {
      const _Float16* tile = kp + t * (kPage * 64);
      ka[jh][2 * t] = __builtin_nontemporal_load(reinterpret_cast<const f16x8*>(tile + tx * 64 + cx * 8));
      ka[jh][2 * t + 1] = __builtin_nontemporal_load(reinterpret_cast<const f16x8*>(tile + ty * 64 + cy * 8));
    }
  }
}

// Raw V^T loads of one page: for d block db, X (d rows 16db + 0..7) ->
// va[db][0], Y (rows 16db + 8..15) -> va[db][1]; after shuffle_pair
// va[db][j] is the operand for tokens 32j + 8 (l>>4) .. +8.
template <int D>
__device__ __forceinline__ void load_v(f16x8 (&va)[D / 16][2], const _Float16* vp, int lane) {
  const int cx = chunk_x(lane), cy = chunk_y(lane), r = lane & 7;
#pragma unroll
  for (int db = 0; db < D / 16; ++db) {
    va[db][0] = __builtin_nontemporal_load(reinterpret_cast<const f16x8*>(vp + (16 * db + r) * kPage + cx * 8));
    va[db][1] = __builtin_nontemporal_load(reinterpret_cast<const f16x8*>(vp + (16 * db + 8 + r) * kPage + cy * 8));
  }
}

template <int D>
__global__ __launch_bounds__(kThreads, 2) void decode_split_kernel(SplitArgs a) {
  constexpr int DS = D / 32;  // QK K-steps
  constexpr int DB = D / 16;  // PV output blocks
  const int s = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int ctx = min(max(a.ctx_lens[b], 0), a.max_ctx);
  const int n_pages = (ctx + kPage - 1) / kPage;
  const int p0 = s * a.split_pages;
  if (p0 >= n_pages) return;
  const int p1 = min(p0 + a.split_pages, n_pages);
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int col = lane & 15, grp = lane >> 4;
  // This wavefront's pages: p0 + wave + kWaves * it, it < n_it.
  const int n_it = (p1 - p0 - wave + kWaves - 1) / kWaves;
  const int32_t* trow = a.block_table + static_cast<int64_t>(b) * a.bt_stride + p0 + wave;
  // One lane per page: the page ids of the next 64 iterations.
  int ids = lane < n_it ? trow[kWaves * lane] : 0;

  // Q^T operand: lane = (head col, d group grp); padded heads are zero.
  f16x8 qb[DS];
  {
    const bool ok = col < a.g;
    const _Float16* qr = a.q + (static_cast<int64_t>(b) * a.Hq + kvh * a.g + (ok ? col : 0)) * D;
#pragma unroll
    for (int ds = 0; ds < DS; ++ds) {
      f16x8 x = *reinterpret_cast<const f16x8*>(qr + 32 * ds + 8 * grp);
      qb[ds] = ok ? x : f16x8{};
    }
  }

  const int64_t page_elems = static_cast<int64_t>(a.Hkv) * D * kPage;
  const int64_t head_elems = static_cast<int64_t>(D) * kPage;
  float m_run = -INFINITY, l_run = 0.f;
  bool poisoned = false;  // a block-table entry was out of range
  f32x4 o[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) o[db] = f32x4{0.f, 0.f, 0.f, 0.f};

  if (n_it > 0) {
    // Page it's K/V base pointers (page id broadcast from lane it % 64).
    auto locate = [&](int it, const _Float16*& kp, const _Float16*& vp) {
      int64_t phys = __builtin_amdgcn_readlane(ids, it & 63);
      const bool bad = phys < 0 || phys >= a.num_pages;
      poisoned |= bad;
      if (bad) phys = 0;  // stay in bounds; the result is poisoned below
      kp = a.k + phys * page_elems + kvh * head_elems;
      vp = a.v + phys * page_elems + kvh * head_elems;
    };
    const _Float16 *kp, *vp;
    locate(0, kp, vp);
    f16x8 ka[4][DS];
    f16x8 va[DB][2];
    load_k<D>(ka, kp, lane);
    load_v<D>(va, vp, lane);

    for (int it = 0; it < n_it; ++it) {
      const int valid = min(kPage, ctx - (p0 + wave + kWaves * it) * kPage);
      const bool bit3 = (lane & 8) != 0;
#pragma unroll
      for (int jh = 0; jh < 4; ++jh)
#pragma unroll
        for (int t = 0; t < DS / 2; ++t) shuffle_pair(ka[jh][2 * t], ka[jh][2 * t + 1], bit3);
      f32x4 sc[4];
#pragma unroll
      for (int jh = 0; jh < 4; ++jh) {
        sc[jh] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ds = 0; ds < DS; ++ds)
          sc[jh] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[jh][ds], qb[ds], sc[jh], 0, 0, 0);
      }
      // The K registers are consumed: start the next page's K loads now, so
      // they are in flight during this page's softmax and PV.
      const bool more = it + 1 < n_it;
      if (more) {
        if (((it + 1) & 63) == 0) {
          const int nx = it + 1 + lane;
          ids = nx < n_it ? trow[kWaves * nx] : 0;
        }
        locate(it + 1, kp, vp);
        load_k<D>(ka, kp, lane);
      }

      // This lane holds head col's scores for tokens 32j + 8grp + 4h + v.
      float mx = -INFINITY;
#pragma unroll
      for (int jh = 0; jh < 4; ++jh)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int t = 32 * (jh >> 1) + 8 * grp + 4 * (jh & 1) + v;
          const float x = t < valid ? sc[jh][v] * a.scale_log2 : -INFINITY;
          sc[jh][v] = x;
          mx = fmaxf(mx, x);
        }
      mx = fmaxf(mx, wave_xor(mx, 16));
      mx = fmaxf(mx, wave_xor(mx, 32));
      const float m_new = fmaxf(m_run, mx);
      const float alpha = fast_exp2(m_run - m_new);
      float psum = 0.f;
      f16x8 pb[2];
#pragma unroll
      for (int jh = 0; jh < 4; ++jh)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const float pv = fast_exp2(sc[jh][v] - m_new);
          psum += pv;
          pb[jh >> 1][(jh & 1) * 4 + v] = static_cast<_Float16>(pv);
        }
      l_run = l_run * alpha + psum;
      m_run = m_new;
#pragma unroll
      for (int db = 0; db < DB; ++db) o[db] *= alpha;
#pragma unroll
      for (int db = 0; db < DB; ++db) shuffle_pair(va[db][0], va[db][1], bit3);
      if (valid < kPage) {
        // Tokens past the context may hold any bits (even NaN); zero them so
        // that 0 * V stays 0 in the PV product.
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
          for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 8; ++e)
              if (32 * j + 8 * grp + e >= valid) va[db][j][e] = static_cast<_Float16>(0.f);
      }
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          o[db] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va[db][j], pb[j], o[db], 0, 0, 0);
      if (more) load_v<D>(va, vp, lane);
    }
  }
  if (poisoned) l_run = NAN;  // propagates to the merged output: NaN, not a fault

  l_run += wave_xor(l_run, 16);
  l_run += wave_xor(l_run, 32);

  __shared__ float sm_m[kWaves][kCols], sm_l[kWaves][kCols];
  __shared__ float sm_o[kWaves][kCols][D];
  if (grp == 0) {
    sm_m[wave][col] = m_run;
    sm_l[wave][col] = l_run;
  }
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int v = 0; v < 4; ++v) sm_o[wave][col][16 * db + 4 * grp + v] = o[db][v];
  __syncthreads();

  const int64_t slot = (static_cast<int64_t>(b) * a.Hkv + kvh) * a.max_splits + s;
  float* wo = a.ws + slot * a.g * D;
  float* wm = a.ws + static_cast<int64_t>(gridDim.z) * a.Hkv * a.max_splits * a.g * D + slot * a.g * 2;
  for (int idx = threadIdx.x; idx < a.g * D; idx += kThreads) {
    const int h = idx / D, d = idx % D;
    float M = sm_m[0][h];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) M = fmaxf(M, sm_m[w][h]);
    float acc = 0.f, L = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float f = fast_exp2(sm_m[w][h] - M);  // waves without pages: exp2(-inf) = 0
      acc += sm_o[w][h][d] * f;
      L += sm_l[w][h] * f;
    }
    wo[h * D + d] = acc;
    if (d == 0) {
      wm[2 * h] = M;
      wm[2 * h + 1] = L;
    }
  }
}

struct MergeArgs {
  const float* ws;
  const int32_t* ctx_lens;
  _Float16* out;
  float* lse;
  int B, Hq, Hkv, g, max_splits, split_tokens, max_ctx;
};

template <int D>
__device__ __forceinline__ float block_reduce(float x, bool is_max, float* scratch) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const float y = __shfl_xor(x, m, 64);
    x = is_max ? fmaxf(x, y) : x + y;
  }
  const int w = threadIdx.x / 64;
  if ((threadIdx.x & 63) == 0) scratch[w] = x;
  __syncthreads();
  float r = scratch[0];
#pragma unroll
  for (int i = 1; i < D / 64; ++i) r = is_max ? fmaxf(r, scratch[i]) : r + scratch[i];
  __syncthreads();
  return r;
}

// Split-KV merge: one block of D threads per (q head, sequence).  The splits'
// weights exp2(m_s - M) are computed once per chunk of D splits into LDS,
// then each thread (one output feature) sums its column with 8-way unrolled
// independent loads.
template <int D>
__global__ __launch_bounds__(D) void decode_merge_kernel(MergeArgs a) {
  __shared__ float s_w[D];
  __shared__ float s_red[D / 64];
  const int h = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
  const int kvh = h / a.g, hh = h % a.g;
  const int ctx_raw = a.ctx_lens[b];
  const int ctx = min(max(ctx_raw, 0), a.max_ctx);
  const int ns = (ctx + a.split_tokens - 1) / a.split_tokens;
  _Float16* o = a.out + (static_cast<int64_t>(b) * a.Hq + h) * D;
  if (ns == 0) {  // empty context: zeros, as torch's CPU SDPA returns
    o[d] = static_cast<_Float16>(0.f);
    if (a.lse && d == 0) a.lse[static_cast<int64_t>(b) * a.Hq + h] = -INFINITY;
    return;
  }
  const int64_t slot0 = (static_cast<int64_t>(b) * a.Hkv + kvh) * a.max_splits;
  const float* wo = a.ws + slot0 * a.g * D + hh * D + d;
  const float* wm = a.ws + static_cast<int64_t>(a.B) * a.Hkv * a.max_splits * a.g * D + slot0 * a.g * 2 + hh * 2;
  const int64_t so = static_cast<int64_t>(a.g) * D;  // split stride of wo
  const int sm = 2 * a.g;                              // split stride of wm

  float mx = -INFINITY;
  for (int s = d; s < ns; s += D) mx = fmaxf(mx, wm[s * sm]);
  const float M = block_reduce<D>(mx, true, s_red);

  float acc = 0.f, lpart = 0.f;
  for (int c = 0; c < ns; c += D) {
    const int s = c + d;
    float w = 0.f;
    if (s < ns) {
      w = fast_exp2(wm[s * sm] - M);
      lpart += wm[s * sm + 1] * w;
    }
    s_w[d] = w;
    __syncthreads();
    const int n = min(D, ns - c);
    const float* col = wo + c * so;
    int j = 0;
    for (; j + 8 <= n; j += 8) {
      float x[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) x[u] = col[(j + u) * so];
#pragma unroll
      for (int u = 0; u < 8; ++u) acc += x[u] * s_w[j + u];
    }
    for (; j < n; ++j) acc += col[j * so] * s_w[j];
    __syncthreads();
  }
  const float L = block_reduce<D>(lpart, false, s_red);
  float r = acc / L;
  if (ctx_raw > a.max_ctx) r = NAN;  // caller broke the max_context_len contract
  o[d] = static_cast<_Float16>(r);
  if (a.lse && d == 0) a.lse[static_cast<int64_t>(b) * a.Hq + h] = (M + log2f(L)) * kLn2;
}

int64_t splits_for(int max_ctx, int split_tokens) {
  return max_ctx <= 0 ? 1 : (static_cast<int64_t>(max_ctx) + split_tokens - 1) / split_tokens;
}

}  // namespace

extern "C" size_t spyre_paged_decode_attn_workspace_bytes(int B, int Hq, int Hkv, int D,
                                                          int max_context_len, int split_tokens) {
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || D <= 0 || split_tokens <= 0 || Hq % Hkv) return 0;
  const int64_t g = Hq / Hkv;
  const int64_t ns = splits_for(max_context_len, split_tokens);
  return static_cast<size_t>(B) * Hkv * ns * g * (D + 2) * sizeof(float);
}

extern "C" int spyre_paged_decode_attn_f16(const void* q, const void* k_cache, const void* v_cache,
                                           const int32_t* block_table, int64_t bt_stride,
                                           const int32_t* context_lens, void* out, float* lse,
                                           void* workspace, size_t workspace_bytes, int B, int Hq,
                                           int Hkv, int D, int page_size, int64_t num_pages,
                                           int max_context_len, int split_tokens, float scale,
                                           void* stream) {
  spyre_hip::clear_error();
  SPYRE_REQUIRE(q && k_cache && v_cache && block_table && context_lens && out && workspace,
                SPYRE_EINVAL, "null pointer argument");
  SPYRE_REQUIRE(B > 0 && Hq > 0 && Hkv > 0 && Hq % Hkv == 0, SPYRE_EINVAL,
                "bad head counts B=%d Hq=%d Hkv=%d", B, Hq, Hkv);
  const int g = Hq / Hkv;
  SPYRE_REQUIRE(g <= kCols, SPYRE_EUNSUPPORTED, "GQA group %d > %d", g, kCols);
  SPYRE_REQUIRE(D == 64 || D == 128, SPYRE_EUNSUPPORTED, "head_dim %d not in {64, 128}", D);
  SPYRE_REQUIRE(page_size == kPage, SPYRE_EUNSUPPORTED, "page_size %d != %d", page_size, kPage);
  SPYRE_REQUIRE(split_tokens > 0 && split_tokens % kPage == 0, SPYRE_EINVAL,
                "split_tokens %d must be a positive multiple of %d", split_tokens, kPage);
  SPYRE_REQUIRE(max_context_len >= 0 && num_pages > 0 && bt_stride >= 0, SPYRE_EINVAL,
                "bad max_context_len / num_pages / bt_stride");
  SPYRE_REQUIRE(bt_stride * kPage >= max_context_len || B == 1, SPYRE_EINVAL,
                "block table rows (%lld pages) shorter than max_context_len %d",
                static_cast<long long>(bt_stride), max_context_len);
  const size_t need =
      spyre_paged_decode_attn_workspace_bytes(B, Hq, Hkv, D, max_context_len, split_tokens);
  SPYRE_REQUIRE(workspace_bytes >= need, SPYRE_ENOSPC, "workspace %zu < %zu bytes",
                workspace_bytes, need);
  const int max_splits = static_cast<int>(splits_for(max_context_len, split_tokens));
  hipStream_t st = static_cast<hipStream_t>(stream);

  SplitArgs sa{static_cast<const _Float16*>(q), static_cast<const _Float16*>(k_cache),
               static_cast<const _Float16*>(v_cache), block_table, bt_stride, context_lens,
               static_cast<float*>(workspace), num_pages, Hq, Hkv, g, max_splits,
               split_tokens / kPage, max_context_len, scale * kLog2e};
  MergeArgs ma{static_cast<const float*>(workspace), context_lens, static_cast<_Float16*>(out),
               lse, B, Hq, Hkv, g, max_splits, split_tokens, max_context_len};
  const dim3 g1(max_splits, Hkv, B), g2(Hq, B);
  if (D == 128) {
    decode_split_kernel<128><<<g1, kThreads, 0, st>>>(sa);
    decode_merge_kernel<128><<<g2, 128, 0, st>>>(ma);
  } else {
    decode_split_kernel<64><<<g1, kThreads, 0, st>>>(sa);
    decode_merge_kernel<64><<<g2, 64, 0, st>>>(ma);
  }
  const hipError_t e = hipGetLastError();
  SPYRE_REQUIRE(e == hipSuccess, SPYRE_EHIP, "decode attention launch failed: %s",
                hipGetErrorString(e));
  return SPYRE_OK;
}
