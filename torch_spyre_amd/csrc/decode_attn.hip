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
// so that the reduction dim of both products is contiguous: every MFMA
// operand is built from whole 128-byte sticks loaded straight into VGPRs.
//
// Pass 1 (decode_split_list_kernel; decode_split_kernel for batches over
// kMaxListSeqs): one workgroup of kWaves wavefronts per work item (sequence,
// KV head, chunk).  A sequence's pages are cut into as few chunks of at most
// kWaves * split_pages pages as cover it, in equal shares, and each
// wavefront streams an equal share (at most split_pages) of its chunk.  The
// pages rotate through the wavefront's operand registers -- the KV carousel:
// page i+1's K loads are issued as soon as page i's QK MFMAs have consumed
// their registers, its V loads as soon as PV has -- and each page is
//   S^T[tok, head] = K[tok, :] Q^T[:, head]   4 x D/32 MFMA 16x16x32 (M = 16 tokens)
//   online softmax in fp32 (exp2 domain), row max across the 4 lane groups
//   of a head by lane shuffles;
//   O^T[d, head] += V^T[d, tok] P^T[tok, head]   D/16 x 2 MFMA 16x16x32
// The q heads of one KV head (g of them, padded to the MFMA's 16 columns)
// form the dense N dimension, so K and V are read once for all g heads.
// The token order of the QK rows is permuted so that each lane's P values
// are exactly the 8 consecutive tokens the PV B operand needs.  The
// wavefronts' partials (unnormalised O, running max, row sum) meet in LDS
// behind one barrier, and every thread folds output elements over them in
// wavefront order (a pairwise tree cost four more barriers).  A sequence
// that fits one chunk (every sequence when max_context_len <= kWaves *
// split_tokens) is then finished by its workgroup: fp16 out and LSE are
// written directly and pass 2 is not launched.  Otherwise the chunk's
// partial goes to the workspace.
//
// Pass 2 (decode_merge_kernel): per (sequence, q head) with several chunks,
// combine the chunks' partials -- the split-KV merge -- and write fp16 out
// (+ optional LSE).  A one-call decode whose pass-1 grid fits one round of
// the device's workgroup slots (paged or dense K / V) merges the chunks in
// pass 1 instead: the workgroup that sees every chunk's arrival flag of its
// (sequence, KV head) combines them (merge_in_kernel).

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <mutex>
#include <type_traits>

#include "decode_dense.h"
#include "spyre_common.h"

namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kPage = 64;
constexpr int kWaves = 8;  // wavefronts per workgroup = per work item
constexpr int kThreads = kWaves * 64;
constexpr int kCols = 16;  // MFMA N: q heads per KV head, padded
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

__device__ __forceinline__ float wave_xor(float x, int m) { return __shfl_xor(x, m, 64); }

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// fp32 -> fp16 of a value already rounded to fp32.  The empty asm keeps the
// compiler from fusing the product before it into a mixed-precision FMA
// (one rounding instead of two), which it does in some kernels and not in
// others: the split and merge passes must round their outputs alike.
__device__ __forceinline__ _Float16 to_f16(float x) {
  asm volatile("" : "+v"(x));
  return static_cast<_Float16>(x);
}

struct SplitArgs {
  const _Float16* q;
  const _Float16* k;
  const _Float16* v;
  const int32_t* block_table;
  int64_t bt_stride;
  const int32_t* ctx_lens;
  float* ws;
  _Float16* out;  // null: every chunk writes its partial (two-pass mode)
  float* lse;
  int64_t num_pages;
  int B, Hq, Hkv, g, max_chunks, chunk_pages, max_ctx;
  float scale_log2;
  // Dense K / V (decode_dense_kernel): [B, Hkv, S, D] with feature stride 1
  // and these strides (elements), every sequence max_ctx tokens long; q
  // [B, Hq, D] with strides q_sb, q_sh.  block_table and ctx_lens unused.
  int64_t q_sb, q_sh, k_sb, k_sh, k_ss, v_sb, v_sh, v_ss;
  // Nonzero: this call's arrival-flag value (a new one per call); the
  // chunks of a sequence with several then merge inside the kernel
  // (run_item, merge_in_kernel), their flags after the partials in ws.
  // 0: the merge pass combines them.
  uint32_t ticket;
};

// Pages of a context and the number of chunks (of at most chunk_pages
// pages) it is cut into; an empty context still has one chunk, whose
// workgroup writes its zeros.
__host__ __device__ __forceinline__ int pages_of(int ctx) { return ctx / kPage + (ctx % kPage != 0); }
__host__ __device__ __forceinline__ int chunks_of(int ctx, int chunk_pages) {
  const int p = pages_of(ctx);
  return p == 0 ? 1 : p / chunk_pages + (p % chunk_pages != 0);
}

// Work-list mode handles batches up to this many sequences (their split
// counts are prefix-summed in LDS); larger batches use grid mode.
#ifndef SPYRE_DECODE_LIST_MAX
#define SPYRE_DECODE_LIST_MAX 1024
#endif
constexpr int kMaxListSeqs = SPYRE_DECODE_LIST_MAX;

// Wavefronts per SIMD the split kernels are compiled for: two pages of
// operands (the one being computed and the next one in flight) take the
// 256 VGPRs that two wavefronts per SIMD leave each.
constexpr int kWavesPerSimd = 2;

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

__host__ __device__ __forceinline__ int chunk_x(int lane) { return (lane & 8) ? 4 + (lane >> 4) : (lane >> 4); }
__host__ __device__ __forceinline__ int chunk_y(int lane) { return (lane & 8) ? (lane >> 4) : 4 + (lane >> 4); }

// ---- Dense route addresses (K / V as [tokens, D] rows) -------------------
//
// One 64-token run of a dense K / V head is read by these loads (lane l):
//   K load (jh, t, y): token dense_k_tok(l, y) + dense_k_dtok(jh), bytes
//     dense_k_col(l, y) + 128 t .. + 15 of the token's row (t < D / 64);
//   V load (j, i):     token dense_v_tok(l) + 32 j + i, bytes
//     dense_v_col<D>(l) .. + kDenseVBytes<D> - 1.
// Every byte lies inside the first 2 D bytes of its token's row.  The
// kernel and the host-side check (spyre_dense_decode_load_extent) use
// these same functions.
__host__ __device__ __forceinline__ int dense_k_tok(int lane, bool y) {
  const int r = lane & 7;
  return 8 * (r >> 2) + (r & 3) + (y ? 16 : 0);  // QK block 0's token of MFMA row r (X) or 8 + r (Y)
}
__host__ __device__ __forceinline__ int dense_k_dtok(int jh) { return 32 * (jh >> 1) + 4 * (jh & 1); }
__host__ __device__ __forceinline__ int dense_k_col(int lane, bool y) { return 16 * (y ? chunk_y(lane) : chunk_x(lane)); }
__host__ __device__ __forceinline__ int dense_v_tok(int lane) { return 8 * (lane >> 4); }
// D = 128: features 8f .. 8f + 7, f = l & 15 (16 bytes).  D = 64: features
// 8f + 4h .. + 3, f = l & 7, h = (l >> 3) & 1 (8 bytes): lanes 8-15 of a row
// start half a block on, so that MFMA row i's feature is 8 (i & 7) + 4 (i >> 3) + db.
template <int D>
__host__ __device__ __forceinline__ int dense_v_col(int lane) {
  return D == 128 ? 16 * (lane & 15) : 16 * (lane & 7) + 8 * ((lane >> 3) & 1);
}
template <int D>
constexpr int kDenseVBytes = D == 128 ? 16 : 8;

// Builds the operand pair from the raw X / Y loads (in place).
__device__ __forceinline__ void shuffle_pair(f16x8& x, f16x8& y, bool bit3) {
  const f16x8 op0 = bit3 ? y : x;
  const f16x8 op1 = ror8(bit3 ? x : y);
  x = op0;
  y = op1;
}

// Pages are read with buffer loads: a resource (base, size) per page in
// SGPRs, a 32-bit per-lane offset in a VGPR and the load-invariant part of
// the offset in an SGPR / immediate.  This keeps address registers to four
// VGPRs per wavefront, and the hardware clamps every access to the page.
typedef __amdgpu_buffer_rsrc_t Rsrc;
constexpr int kRsrcWord3 = 0x00020000;  // raw (untyped) buffer, 32-bit format
constexpr int kLoadNT = 2;              // non-temporal: K/V are streamed once

__device__ __forceinline__ Rsrc page_rsrc(const _Float16* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16*>(base), 0, bytes, kRsrcWord3);
}

__device__ __forceinline__ f16x8 bload(Rsrc r, int voff, int soff) {
  return __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, kLoadNT));
}

// The dense V operand registers of one token: 8 features (D = 128) or 4
// (D = 64).
template <int D>
using DenseV = typename std::conditional<D == 128, f16x8, f16x4>::type;

template <int D>
__device__ __forceinline__ DenseV<D> bload_v(Rsrc r, int voff, int soff) {
  if constexpr (D == 128)
    return bload(r, voff, soff);
  else
    return __builtin_bit_cast(f16x4, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, kLoadNT));
}

// Per-lane byte offsets of the raw loads (see the X / Y scheme above).
struct LoadOffsets {
  int kx, ky, vx, vy;
  __device__ __forceinline__ explicit LoadOffsets(int lane) {
    const int r = lane & 7, cx = chunk_x(lane), cy = chunk_y(lane);
    // QK block jh = (j, h): MFMA row i <-> token 32j + 8(i/4) + 4h + i%4;
    // this is block 0's token of row r.
    const int tx = dense_k_tok(lane, false);
    kx = (tx * 64 + cx * 8) * 2;
    ky = ((tx + 16) * 64 + cy * 8) * 2;     // row 8 + r is token tx + 16
    vx = (r * kPage + cx * 8) * 2;
    vy = ((8 + r) * kPage + cy * 8) * 2;
  }
  // Dense K / V (head_dim D), tokens k_row / v_row bytes apart: the K
  // loads as above (dense_k_*); vx is the dense V load's offset
  // (load_v_dense), vy unused.
  template <int D>
  __device__ __forceinline__ static LoadOffsets dense(int lane, int k_row, int v_row) {
    LoadOffsets lo(lane);
    lo.kx = dense_k_tok(lane, false) * k_row + dense_k_col(lane, false);
    lo.ky = dense_k_tok(lane, true) * k_row + dense_k_col(lane, true);
    lo.vx = dense_v_tok(lane) * v_row + dense_v_col<D>(lane);
    lo.vy = 0;
    return lo;
  }
};

// Raw K loads of one page: for block jh and stick tile t, X -> ka[jh][2t],
// Y -> ka[jh][2t+1] (operands after shuffle_pair: d = 32 ds + 8 (l>>4)).
template <int D>
__device__ __forceinline__ void load_k(f16x8 (&ka)[4][D / 32], Rsrc kr, const LoadOffsets& lo) {
#pragma unroll
  for (int jh = 0; jh < 4; ++jh) {
#pragma unroll
    for (int t = 0; t < D / 64; ++t) {
      const int so = ((32 * (jh >> 1) + 4 * (jh & 1)) * 64 + t * (kPage * 64)) * 2;
      ka[jh][2 * t] = bload(kr, lo.kx, so);
      ka[jh][2 * t + 1] = bload(kr, lo.ky, so);
    }
  }
}

// Dense K: the same X / Y stick loads, tokens k_row bytes apart (the
// token's two 128-byte sticks side by side instead of 8 KiB apart).  A
// 64-token window (WHOLE) keeps the token offset in the scalar operand:
// every load lies inside the window's rows.  A context shorter than 64
// tokens is read as one short run (WHOLE false) with the whole offset in
// the per-lane operand, which the buffer's range check covers (the range
// ends with the last token's 2 D bytes): no byte past the context is read,
// and the lanes of tokens past it load zeros (bytes inside the view when
// the token stride is below 2 D bytes).
template <int D, bool WHOLE>
__device__ __forceinline__ void load_k_dense(f16x8 (&ka)[4][D / 32], Rsrc kr, const LoadOffsets& lo, int k_row) {
#pragma unroll
  for (int jh = 0; jh < 4; ++jh)
#pragma unroll
    for (int t = 0; t < D / 64; ++t) {
      const int so = dense_k_dtok(jh) * k_row + t * 128;
      ka[jh][2 * t] = WHOLE ? bload(kr, lo.kx, so) : bload(kr, lo.kx + so, 0);
      ka[jh][2 * t + 1] = WHOLE ? bload(kr, lo.ky, so) : bload(kr, lo.ky + so, 0);
    }
}

// Dense V ([tokens, D], tokens v_row bytes apart): lane l (token group tg =
// l >> 4) loads its features (dense_v_col) of tokens 32j + 8tg + i into
// va[i][j], each instruction four whole token rows.  transposed_col turns a
// j's eight registers into the PV operands: MFMA db's row i is feature
// 8i + db (D = 128), or 8 (i & 7) + 4 (i >> 3) + db (D = 64, db < 4).
// Windows and short runs as load_k_dense.
template <int D, bool WHOLE>
__device__ __forceinline__ void load_v_dense(DenseV<D> (&va)[8][2], Rsrc vr, const LoadOffsets& lo, int v_row) {
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int so = (32 * j + i) * v_row;
      va[i][j] = WHOLE ? bload_v<D>(vr, lo.vx, so) : bload_v<D>(vr, lo.vx + so, 0);
    }
}

// Column a of the 8 x 8 block of 16-bit elements va[0..7][j]: element i is
// va[i][j][a] (the a-th loaded feature of token 32j + 8tg + i).
template <typename VT>
__device__ __forceinline__ f16x8 transposed_col(const VT (&va)[8][2], int j, int a) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  typedef uint32_t u32w __attribute__((ext_vector_type(sizeof(VT) / 4)));
  u32x4 x;
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const uint32_t lo = __builtin_bit_cast(u32w, va[2 * p][j])[a / 2];
    const uint32_t hi = __builtin_bit_cast(u32w, va[2 * p + 1][j])[a / 2];
    x[p] = (a & 1) ? ((lo >> 16) | (hi & 0xffff0000u)) : ((lo & 0xffffu) | (hi << 16));
  }
  return __builtin_bit_cast(f16x8, x);
}

// Raw V^T loads of one page: for d block db, X (d rows 16db + 0..7) ->
// va[db][0], Y (rows 16db + 8..15) -> va[db][1]; after shuffle_pair
// va[db][j] is the operand for tokens 32j + 8 (l>>4) .. +8.
template <int D>
__device__ __forceinline__ void load_v(f16x8 (&va)[D / 16][2], Rsrc vr, const LoadOffsets& lo) {
#pragma unroll
  for (int db = 0; db < D / 16; ++db) {
    const int so = 16 * db * kPage * 2;
    va[db][0] = bload(vr, lo.vx, so);
    va[db][1] = bload(vr, lo.vy, so);
  }
}

// Pages [p0, p0 + n_it) of sequence b, KV head kvh (context ctx tokens),
// streamed by one wavefront: the pages rotate through the operand registers
// (the next page's K loads are issued as soon as this page's QK MFMAs have
// consumed theirs).  Leaves the wavefront's partial in registers: lane
// (head col, group grp) holds O^T[d = 16db + 4grp + v][col] unnormalised in
// o[db][v], the running max m (log2 domain) and the row sum l of head col.
// n_it = 0 leaves the empty partial (0, -inf, 0).
// DENSE: "pages" are 64-token runs of dense K / V (SplitArgs' dense
// strides); lane (col, grp) then holds O^T[d][col] in o[db][v] for d the
// feature of PV row i = 4 grp + v of MFMA db (load_v_dense).
template <int D, bool DENSE = false>
__device__ __forceinline__ void stream_pages(const SplitArgs& a, int b, int kvh, int p0, int n_it,
                                             int ctx, int lane, f32x4 (&o)[D / 16], float& m_out,
                                             float& l_out) {
  constexpr int DS = D / 32;  // QK K-steps
  constexpr int DB = D / 16;  // PV output blocks
#pragma unroll
  for (int db = 0; db < DB; ++db) o[db] = f32x4{0.f, 0.f, 0.f, 0.f};
  m_out = -INFINITY;
  l_out = 0.f;
  if (n_it <= 0) return;
  const int col = lane & 15, grp = lane >> 4;
  const int32_t* trow = DENSE ? nullptr : a.block_table + static_cast<int64_t>(b) * a.bt_stride + p0;
  // One lane per page: the page ids of the next 64 pages.
  int ids = !DENSE && lane < n_it ? trow[lane] : 0;

  // Q^T operand: lane = (head col, d group grp); padded heads are zero.
  f16x8 qb[DS];
  {
    const bool ok = col < a.g;
    const int h = kvh * a.g + (ok ? col : 0);
    const _Float16* qr = DENSE ? a.q + b * a.q_sb + h * a.q_sh : a.q + (static_cast<int64_t>(b) * a.Hq + h) * D;
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

  // Page it's K/V resources (page id broadcast from lane it % 64).
  const int head_bytes = static_cast<int>(head_elems * 2);
  // Dense: run it is tokens 64 (p0 + it) .. + 63 of the sequence's K / V
  // head.  A short last run (ctx % 64 != 0, ctx >= 64) is read as the
  // 64-token window ending with the last token, whose first tokens (the
  // previous run's, already streamed) are masked out, so that every load of
  // the steady state lies inside the view.  Only a context below 64 tokens
  // is a short run: one run, loaded before the loop with the whole offset
  // per lane (load_k_dense).  A resource's range ends with the last row's
  // 2 D bytes (the host keeps 64 rows of either within 2^30 bytes, so no
  // offset wraps).
  const int k_row = DENSE ? static_cast<int>(a.k_ss * 2) : 0, v_row = DENSE ? static_cast<int>(a.v_ss * 2) : 0;
  // Run it's window: it starts lo_tok tokens before the run (0 but for a
  // short last run of dense K / V: the wave's run shift_it, shifted by
  // shift tokens), and its tokens [lo_tok, hi_tok) are the run's own.
  int shift_it = -1, shift = 0;
  if (DENSE && ctx >= kPage && ctx % kPage != 0 && p0 + n_it == pages_of(ctx)) {
    shift_it = n_it - 1;
    shift = kPage - ctx % kPage;
  }
  auto window = [&](int it, int& lo_tok, int& hi_tok) {
    lo_tok = it == shift_it ? shift : 0;
    hi_tok = min(kPage, ctx - (p0 + it) * kPage + lo_tok);
  };
  // Dense: the wave's first run; run it is run_bytes further on.
  const char* k0 = DENSE ? reinterpret_cast<const char*>(a.k + b * a.k_sb + kvh * a.k_sh) +
                               static_cast<int64_t>(p0) * kPage * k_row : nullptr;
  const char* v0 = DENSE ? reinterpret_cast<const char*>(a.v + b * a.v_sb + kvh * a.v_sh) +
                               static_cast<int64_t>(p0) * kPage * v_row : nullptr;
  auto locate = [&](int it, Rsrc& kr, Rsrc& vr) {
    if constexpr (DENSE) {
      int lo_tok, hi_tok;
      window(it, lo_tok, hi_tok);
      const char* kp = k0 + (static_cast<int64_t>(it) * kPage - lo_tok) * k_row;
      const char* vp = v0 + (static_cast<int64_t>(it) * kPage - lo_tok) * v_row;
      kr = page_rsrc(reinterpret_cast<const _Float16*>(kp), (hi_tok - 1) * k_row + 2 * D);
      vr = page_rsrc(reinterpret_cast<const _Float16*>(vp), (hi_tok - 1) * v_row + 2 * D);
    } else {
      int64_t phys = __builtin_amdgcn_readlane(ids, it & 63);
      const bool bad = phys < 0 || phys >= a.num_pages;
      poisoned |= bad;
      if (bad) phys = 0;  // stay in bounds; the result is poisoned below
      kr = page_rsrc(a.k + phys * page_elems + kvh * head_elems, head_bytes);
      vr = page_rsrc(a.v + phys * page_elems + kvh * head_elems, head_bytes);
    }
  };
  // Dense K / V: the wave streams its runs from a rotated start, run_of(it)
  // (the softmax does not depend on the order).  Heads of contiguous
  // [B, H, S, D] tensors lie a power of two apart, and without the rotation
  // every workgroup reads the same offset of its head at the same moment:
  // B 16 x 16 heads x 4096 tokens at D 64 took 50.2 us in run order and 44.1
  // rotated, B 32 x 32 / 8 heads x 4096 at D 128 85.7 and 84.4 (one box).
  // Paged runs keep their order (random page placement already spreads
  // them; rotating measured slower there).
  const int rot = DENSE && n_it > 1 ? static_cast<int>((static_cast<uint32_t>(b) * a.Hkv + kvh + p0 / n_it) % n_it) : 0;
  auto run_of = [&](int it) { return it + rot < n_it ? it + rot : it + rot - n_it; };
  const LoadOffsets lo = DENSE ? LoadOffsets::dense<D>(lane, k_row, v_row) : LoadOffsets(lane);
  // Loads of a whole run (a page, or a 64-token window of dense K / V).
  auto issue_k = [&](f16x8 (&ka)[4][DS], Rsrc kr) {
    if constexpr (DENSE) load_k_dense<D, true>(ka, kr, lo, k_row); else load_k<D>(ka, kr, lo);
  };
  // V registers: dense, 8 tokens x 2 halves of the run (DenseV<D> each);
  // paged, DB feature blocks x 2 token halves.
  using VT = typename std::conditional<DENSE, DenseV<D>, f16x8>::type;
  constexpr int VR = DENSE ? 8 : DB;
  auto issue_v = [&](VT (&va)[VR][2], Rsrc vr) {
    if constexpr (DENSE) load_v_dense<D, true>(va, vr, lo, v_row); else load_v<D>(va, vr, lo);
  };
  f16x8 ka[4][DS];
  VT va[VR][2];
  {
    Rsrc kr, vr;
    locate(run_of(0), kr, vr);
    if (DENSE && ctx < kPage) {
      if constexpr (DENSE) {  // the one short run
        load_k_dense<D, false>(ka, kr, lo, k_row);
        load_v_dense<D, false>(va, vr, lo, v_row);
      }
    } else {
      issue_k(ka, kr);
      issue_v(va, vr);
    }
  }
  const bool bit3 = (lane & 8) != 0;

  // Run it, whose operands are in ka / va.  (Two runs rotating through two
  // sets of registers at D = 64, where they fit, measured slower: 46.7 ->
  // 48.9 us for B 32 x 16 heads x 2048 tokens.)
  auto step = [&](int it) {
    int lo_tok, valid;  // this run's own window tokens: [lo_tok, valid)
    window(run_of(it), lo_tok, valid);
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
    // The K registers are consumed: start the next run's K loads into them
    // now, so they are in flight during this run's softmax and PV.
    const int nx = it + 1;
    const bool more = nx < n_it;
    Rsrc kr, vr;
    if (more) {
      if (!DENSE && (nx & 63) == 0) {  // the page ids of the next 64 runs
        const int q = nx + lane;
        ids = q < n_it ? trow[q] : 0;
      }
      locate(run_of(nx), kr, vr);
      issue_k(ka, kr);
    }

    // This lane holds head col's scores for tokens 32j + 8grp + 4h + v.
    // Tokens outside [lo_tok, valid) score -inf; a whole run (every run but
    // a sequence's last) skips the comparisons by a wave-uniform branch.
    float mx = -INFINITY;
    auto scale_scores = [&](auto edge) {
#pragma unroll
      for (int jh = 0; jh < 4; ++jh)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int t = 32 * (jh >> 1) + 8 * grp + 4 * (jh & 1) + v;
          float x = sc[jh][v] * a.scale_log2;
          if constexpr (decltype(edge)::value) x = t >= lo_tok && t < valid ? x : -INFINITY;
          sc[jh][v] = x;
          mx = fmaxf(mx, x);
        }
    };
    if (lo_tok > 0 || valid < kPage)
      scale_scores(std::true_type{});
    else
      scale_scores(std::false_type{});
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
    if constexpr (DENSE) {
      // va[i][j] holds window token 32j + 8grp + i.  Tokens below lo_tok
      // are the view's own and weigh 0; past a short context the loads were
      // out of range and gave zeros (token strides are 0 or at least 2 D
      // bytes; with 0 every token is the one row), so 0 * V stays 0.
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int db = 0; db < DB; ++db)
          o[db] = __builtin_amdgcn_mfma_f32_16x16x32_f16(transposed_col(va, j, db), pb[j], o[db], 0, 0, 0);
    } else {
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
    }
    if (more) issue_v(va, vr);
  };

  for (int it = 0; it < n_it; ++it) step(it);
  if (poisoned) l_run = NAN;  // propagates to the merged output: NaN, not a fault
  l_run += wave_xor(l_run, 16);
  l_run += wave_xor(l_run, 32);
  m_out = m_run;
  l_out = l_run;
}

// Chunks whose loads are issued together in a merge (one memory latency
// for up to this many chunks).
constexpr int kMergeChunk = 16;

// The merge of one output row's 4 features over a sequence's nch chunk
// partials, the split-KV merge of both the merge pass and the in-kernel
// merge: load_ml(s) / load_o(s) return chunk s's (m, l) and the row's 4
// features of O.  kMergeChunk chunks' loads go out together; past the last
// chunk the loads repeat it and add nothing.  Running (M, L, acc) as the
// online softmax rescales them; returns acc and leaves M, L.
template <typename LoadML, typename LoadO>
__device__ __forceinline__ f32x4 merge_row4(int nch, LoadML load_ml, LoadO load_o, float& M, float& L) {
  constexpr int G = kMergeChunk;
  M = -INFINITY;
  L = 0.f;
  f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int c = 0; c < nch; c += G) {
    f32x2 ml[G];
    f32x4 x[G];
#pragma unroll
    for (int u = 0; u < G; ++u) {
      const int s = min(c + u, nch - 1);
      ml[u] = load_ml(s);
      x[u] = load_o(s);
    }
    float mc = M;
#pragma unroll
    for (int u = 0; u < G; ++u)
      if (c + u < nch) mc = fmaxf(mc, ml[u][0]);
    const float r = fast_exp2(M - mc);  // first round: exp2(-inf) = 0
    L *= r;
    acc *= r;
#pragma unroll
    for (int u = 0; u < G; ++u) {
      // Explicit fused multiply-adds: every kernel that merges rounds alike.
      const float w = fast_exp2(ml[u][0] - mc);
      if (c + u < nch) {
        L = __builtin_fmaf(ml[u][1], w, L);
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[e] = __builtin_fmaf(x[u][e], w, acc[e]);
      }
    }
    M = mc;
  }
  return acc;
}

// Several chunks per sequence: after its chunk's partial (a device-scope
// store of every element) workgroup (b, c, kvh) stores an
// arrival flag (the call's ticket) from wavefront 0, waits for it, and reads
// the flags of every chunk of (b, kvh) with device-scope loads.  Of any two
// workgroups, the one whose flag store finished later reads the other's
// flag after it, so at least one sees all of them; every one that does
// merges the g rows of (b, kvh) over the chunks in order (to the same bits)
// and clears the flags, so replays of a captured call (one ticket) start
// clear and a new call's ticket matches no older call's flags.  Thread
// (row col, features 4 d4 .. + 3) merges by merge_row4 with device-scope
// loads, so its results match the merge pass's bit for bit.  bad: the
// context broke the max_context_len contract (NaN output).
template <int D, int W>
__device__ void merge_in_kernel(const SplitArgs& a, int b, int c, int kvh, int nch, bool bad, int wave,
                                int lane) {
  constexpr int kAuxDevice = 16;  // sc1: device scope
  constexpr int D4 = D / 4;
  const int64_t parts = static_cast<int64_t>(a.B) * a.Hkv * a.max_chunks;
  const int64_t slot0 = (static_cast<int64_t>(b) * a.Hkv + kvh) * a.max_chunks;
  const Rsrc wr = __builtin_amdgcn_make_buffer_rsrc(a.ws, 0, 0x7ffffff0, kRsrcWord3);
  const uint32_t fl_off = static_cast<uint32_t>((parts * a.g * (D + 2) + slot0) * 4);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();  // every partial store of the workgroup done
  __shared__ int s_merge;
  if (wave == 0) {
    if (lane == 0) __builtin_amdgcn_raw_buffer_store_b32(a.ticket, wr, fl_off + c * 4, 0, kAuxDevice);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    bool seen = true;
    for (int s2 = lane; s2 < nch; s2 += 64)
      seen = seen && __builtin_amdgcn_raw_buffer_load_b32(wr, fl_off + s2 * 4, 0, kAuxDevice) == a.ticket;
    const bool all = __all(seen);
    if (lane == 0) s_merge = all ? 1 : 0;
  }
  __syncthreads();
  if (!s_merge) return;
  const uint32_t ml_off = static_cast<uint32_t>(parts * a.g * D * 4);
  for (int u = static_cast<int>(threadIdx.x); u < a.g * D4; u += W * 64) {
    const int col = u / D4, d = 4 * (u - col * D4);
    const uint32_t part0 = static_cast<uint32_t>(slot0 * a.g + col);  // chunk s: part0 + s g
    float Mr, Lr;
    const f32x4 ac = merge_row4(
        nch,
        [&](int s) {
          const uint32_t part = part0 + static_cast<uint32_t>(s * a.g);
          return __builtin_bit_cast(f32x2, __builtin_amdgcn_raw_buffer_load_b64(wr, ml_off + part * 8, 0, kAuxDevice));
        },
        [&](int s) {
          const uint32_t part = part0 + static_cast<uint32_t>(s * a.g);
          return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, (part * D + d) * 4, 0, kAuxDevice));
        },
        Mr, Lr);
    const int64_t row = static_cast<int64_t>(b) * a.Hq + kvh * a.g + col;
    const float inv = bad ? NAN : 1.f / Lr;  // the merge pass's product, then NaN for a bad context
    f16x4 rv;
#pragma unroll
    for (int e = 0; e < 4; ++e) rv[e] = to_f16(ac[e] * inv);
    *reinterpret_cast<f16x4*>(a.out + row * D + d) = rv;
    if (a.lse && d == 0) a.lse[row] = (Mr + log2f(Lr)) * kLn2;
  }
  for (int s2 = static_cast<int>(threadIdx.x); s2 < nch; s2 += W * 64)
    __builtin_amdgcn_raw_buffer_store_b32(0u, wr, fl_off + s2 * 4, 0, kAuxDevice);
}

// Work item (sequence b, chunk c, KV head kvh), run by all kWaves
// wavefronts of the workgroup.  The wavefronts' partials are combined in LDS
// and the whole workgroup writes the result: fp16 out and LSE when the
// sequence has one chunk and out is given, else the chunk's partial (O per
// q head and feature; m, l) into the workspace for the merge pass -- or,
// with a ticket, for the merge in the same kernel (merge_in_kernel).
template <int D, bool DENSE = false, int W = kWaves>
__device__ __forceinline__ void run_item(const SplitArgs& a, int b, int c, int kvh, int wave,
                                         int lane) {
  constexpr int DB = D / 16;
  const int ctx_raw = DENSE ? a.max_ctx : a.ctx_lens[b];
  const int ctx = min(max(ctx_raw, 0), a.max_ctx);
  const int n_pages = pages_of(ctx);
  const int nch = chunks_of(ctx, a.chunk_pages);
  // Chunk c holds pages [cp0, cp1); wavefront w an equal share of them.
  const int cp0 = static_cast<int>(static_cast<int64_t>(c) * n_pages / nch);
  const int cp1 = static_cast<int>(static_cast<int64_t>(c + 1) * n_pages / nch);
  const int nc = cp1 - cp0;
  const int w0 = cp0 + static_cast<int>(static_cast<int64_t>(wave) * nc / W);
  const int w1 = cp0 + static_cast<int>(static_cast<int64_t>(wave + 1) * nc / W);
  f32x4 o[DB];
  float m, l;
  stream_pages<D, DENSE>(a, b, kvh, w0, w1 - w0, ctx, lane, o, m, l);
  // Every wavefront's partial goes to LDS once; then each thread folds
  // output elements over the W partials, in wavefront order.  Lane
  // (col, grp) holds O^T[d = 16 db + 4 grp + v][col] in o[db][v]; a row of
  // 16 columns is padded so that the fold's reads of columns < 4 (the usual
  // group size) fall in distinct banks.
  constexpr int kColPad = 4;
  __shared__ f32x4 s_o[W][DB][4][16 + kColPad];
  __shared__ float s_m[W][16], s_l[W][16];
  {
    const int col = lane & 15, grp = lane >> 4;
#pragma unroll
    for (int db = 0; db < DB; ++db) s_o[wave][db][grp][col] = o[db];
    if (grp == 0) {
      s_m[wave][col] = m;
      s_l[wave][col] = l;
    }
  }
  __syncthreads();
  const bool single = a.out && nch == 1;
  const bool bad = ctx_raw > a.max_ctx;  // caller broke the max_context_len contract
  const int64_t slot = (static_cast<int64_t>(b) * a.Hkv + kvh) * a.max_chunks + c;
  if (!single && a.ticket) {
    // The chunk's partial as 16-byte device-scope stores (sc1: written
    // through to memory; the merging workgroup may run on another XCD) of 4
    // consecutive features per thread, then the arrival flags.  The host
    // keeps the workspace below 2^31 bytes for this path.
    constexpr int D4 = D / 4;
    const Rsrc wr = __builtin_amdgcn_make_buffer_rsrc(a.ws, 0, 0x7ffffff0, kRsrcWord3);
    const uint32_t ml_off = static_cast<uint32_t>(static_cast<int64_t>(a.B) * a.Hkv * a.max_chunks * a.g * D * 4);
    for (int u = static_cast<int>(threadIdx.x); u < a.g * D4; u += W * 64) {
      const int col = u / D4, d0 = 4 * (u - col * D4);
      // Features d0 + e (e < 4), by the inverse of the feature map below:
      // paged, PV row i0 + e of MFMA db0 (one f32x4 of s_o); dense, PV row
      // i0 of MFMAs db0 + e.
      const int i0 = !DENSE ? d0 & 15 : D == 128 ? d0 >> 3 : (d0 >> 3) + 8 * ((d0 >> 2) & 1);
      const int db0 = !DENSE ? d0 >> 4 : D == 128 ? d0 & 7 : 0;
      const int grp = i0 >> 2;
      float M = -INFINITY;
#pragma unroll
      for (int w = 0; w < W; ++w) M = fmaxf(M, s_m[w][col]);
      float L = 0.f;
      f32x4 O = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int w = 0; w < W; ++w) {
        const float sc = M == -INFINITY ? 0.f : fast_exp2(s_m[w][col] - M);
        L = __builtin_fmaf(s_l[w][col], sc, L);  // as the per-element fold below
#pragma unroll
        for (int e = 0; e < 4; ++e)
          O[e] = __builtin_fmaf(DENSE ? s_o[w][db0 + e][grp][col][i0 & 3] : s_o[w][db0][grp][col][e], sc, O[e]);
      }
      const uint32_t part = static_cast<uint32_t>(slot * a.g + col);
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, O), wr, (part * D + d0) * 4, 0, 16);
      if (d0 == 0)
        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, f32x2{M, L}), wr, ml_off + part * 8, 0, 16);
    }
    merge_in_kernel<D, W>(a, b, c, kvh, nch, bad, wave, lane);
    return;
  }
  for (int e = static_cast<int>(threadIdx.x); e < a.g * D; e += W * 64) {
    // e -> (db, grp, col, v), v fastest, then col < g, then grp.
    const int v = e & 3;
    const int r = e >> 2;
    const int col = r % a.g, r2 = r / a.g;
    const int grp = r2 & 3, db = r2 >> 2;
    const int i = 4 * grp + v;  // PV row
    const int d = !DENSE ? 16 * db + i : D == 128 ? 8 * i + db : 8 * (i & 7) + 4 * (i >> 3) + db;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < W; ++w) M = fmaxf(M, s_m[w][col]);
    float L = 0.f, O = 0.f;
#pragma unroll
    for (int w = 0; w < W; ++w) {
      // Empty partials (m = -inf) weigh 0; all empty: M = -inf, L = O = 0.
      const float sc = M == -INFINITY ? 0.f : fast_exp2(s_m[w][col] - M);
      // Explicit fused multiply-adds: the partials of the vector path above
      // (chunks merged in the kernel) and of this one round alike.
      L = __builtin_fmaf(s_l[w][col], sc, L);
      O = __builtin_fmaf(s_o[w][db][grp][col][v], sc, O);
    }
    if (single) {
      const int64_t row = static_cast<int64_t>(b) * a.Hq + kvh * a.g + col;
      // Empty context: zeros, as torch's CPU SDPA returns.
      const float inv = ctx == 0 ? 0.f : (bad ? NAN : 1.f / L);
      a.out[row * D + d] = to_f16(O * inv);
      if (a.lse && d == 0) a.lse[row] = ctx == 0 ? -INFINITY : (M + log2f(L)) * kLn2;
    } else {
      a.ws[(slot * a.g + col) * D + d] = O;
      if (d == 0) {
        float* wm = a.ws + static_cast<int64_t>(a.B) * a.Hkv * a.max_chunks * a.g * D + (slot * a.g + col) * 2;
        wm[0] = M;
        wm[1] = L;
      }
    }
  }
}

// Grid mode: blockIdx = (chunk, KV head, sequence).  Chunks past a
// sequence's count return at once (the whole workgroup).
template <int D>
__global__ __launch_bounds__(kThreads, kWavesPerSimd) void decode_split_kernel(SplitArgs a) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64), lane = threadIdx.x % 64;
  const int b = blockIdx.z, c = blockIdx.x;
  const int ctx = min(max(a.ctx_lens[b], 0), a.max_ctx);
  if (c >= chunks_of(ctx, a.chunk_pages)) return;
  run_item<D>(a, b, c, blockIdx.y, wave, lane);
}

// Work-list mode: the items (sequence, chunk, KV head) that exist are
// numbered densely -- each workgroup prefix-sums the per-sequence chunk
// counts in LDS -- and workgroup x takes item x.  Real items come first, so
// no workgroup is spent on a chunk past a sequence's end until all real ones
// have been dispatched; ragged batches stay balanced.
template <int D>
__global__ __launch_bounds__(kThreads, kWavesPerSimd) void decode_split_list_kernel(SplitArgs a) {
  if (a.max_chunks == 1) {
    // Every sequence is one chunk (an empty one too): item x is (sequence
    // x / Hkv, chunk 0, KV head x % Hkv), with no prefix sum to wait for.
    const int item = blockIdx.x;
    if (item >= a.B * a.Hkv) return;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64), lane = threadIdx.x % 64;
    run_item<D>(a, item / a.Hkv, 0, item % a.Hkv, wave, lane);
    return;
  }
  __shared__ int s_pre[kMaxListSeqs > 0 ? kMaxListSeqs + 1 : 1];
  for (int i = threadIdx.x; i < a.B; i += kThreads) {
    const int c = min(max(a.ctx_lens[i], 0), a.max_ctx);
    s_pre[i + 1] = chunks_of(c, a.chunk_pages);
  }
  if (threadIdx.x == 0) s_pre[0] = 0;
  __syncthreads();
  if (threadIdx.x < 64) {  // inclusive scan of s_pre[1..B], 64 at a time
    const int lane = threadIdx.x;
    int carry = 0;
    for (int base = 1; base <= a.B; base += 64) {
      const int i = base + lane;
      int v = i <= a.B ? s_pre[i] : 0;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int t = __shfl_up(v, o, 64);
        if (lane >= o) v += t;
      }
      if (i <= a.B) s_pre[i] = v + carry;
      carry += __shfl(v, 63, 64);
    }
  }
  __syncthreads();
  // Everything below is workgroup-uniform; readfirstlane keeps it in
  // scalar registers.
  const int total = __builtin_amdgcn_readfirstlane(s_pre[a.B]) * a.Hkv;
  const int item = blockIdx.x;
  if (item >= total) return;  // the whole workgroup
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64), lane = threadIdx.x % 64;
  const int bs = item / a.Hkv, kvh = item - bs * a.Hkv;
  int lo = 0, hi = a.B;  // s_pre[lo] <= bs < s_pre[hi]
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (__builtin_amdgcn_readfirstlane(s_pre[mid]) <= bs) lo = mid; else hi = mid;
  }
  run_item<D>(a, lo, bs - __builtin_amdgcn_readfirstlane(s_pre[lo]), kvh, wave, lane);
}

// Dense decode: item x = ((b Hkv + kvh) max_chunks + c); every sequence has
// max_chunks chunks of its max_ctx tokens (grid = B Hkv max_chunks).  W
// wavefronts per item and workgroup: 8, or 4 where the eight-wavefront
// grid would take more than one round of the device (dense_decode_plan).
template <int D, int W = kWaves>
__global__ __launch_bounds__(W * 64, kWavesPerSimd) void decode_dense_kernel(SplitArgs a) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64), lane = threadIdx.x % 64;
  const int item = blockIdx.x;
  const int c = item % a.max_chunks, r = item / a.max_chunks;
  run_item<D, true, W>(a, r / a.Hkv, c, r % a.Hkv, wave, lane);
}

// Workgroup slots of the four-wavefront dense kernel on the current device
// (cached per device), 0 if the runtime cannot say.
int dense4_slots(int D) {
  static std::atomic<int> cache[64][2];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  std::atomic<int>& c = cache[dev][D == 128];
  int v = c.load(std::memory_order_relaxed);
  if (v > 0) return v;
  int cus = 0, per_cu = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  const hipError_t e =
      D == 128 ? hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, decode_dense_kernel<128, 4>, 4 * 64, 0)
               : hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, decode_dense_kernel<64, 4>, 4 * 64, 0);
  if (e != hipSuccess || cus <= 0 || per_cu <= 0) return 0;
  v = cus * per_cu;
  c.store(v, std::memory_order_relaxed);
  return v;
}

struct MergeArgs {
  const float* ws;
  const int32_t* ctx_lens;  // null: every sequence max_ctx tokens (dense K / V)
  _Float16* out;
  float* lse;
  int B, Hq, Hkv, g, max_chunks, chunk_pages, max_ctx;
  int skip_single;  // sequences of one chunk were finished by pass 1
};

// Split-KV merge: one block of D threads per (q head, sequence) over the
// sequence's chunk partials.  All loads of kMergeChunk chunks (m, l and the
// thread's O column) are issued together before any of them is used, so
// they cost one memory latency; chunks past the sequence's count are read
// (in bounds: the workspace holds max_chunks) and discarded by selects,
// never multiplied.

template <int D>
__global__ __launch_bounds__(D) void decode_merge_kernel(MergeArgs a) {
  const int h = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
  const int kvh = h / a.g, hh = h % a.g;
  const int ctx_raw = a.ctx_lens ? a.ctx_lens[b] : a.max_ctx;
  const int ctx = min(max(ctx_raw, 0), a.max_ctx);
  const int ns = chunks_of(ctx, a.chunk_pages);
  if (a.skip_single && ns == 1) return;
  const int64_t slot0 = (static_cast<int64_t>(b) * a.Hkv + kvh) * a.max_chunks;
  const float* wo = a.ws + slot0 * a.g * D + hh * D + d;
  const float* wm = a.ws + static_cast<int64_t>(a.B) * a.Hkv * a.max_chunks * a.g * D + slot0 * a.g * 2 + hh * 2;
  const int64_t so = static_cast<int64_t>(a.g) * D;  // chunk stride of wo
  const int sm = 2 * a.g;                              // chunk stride of wm
  _Float16* o = a.out + (static_cast<int64_t>(b) * a.Hq + h) * D;
  if (ctx == 0) {  // empty context: zeros, as torch's CPU SDPA returns
    o[d] = static_cast<_Float16>(0.f);
    if (a.lse && d == 0) a.lse[static_cast<int64_t>(b) * a.Hq + h] = -INFINITY;
    return;
  }
  // Running (M, L, acc) over the chunks, rescaled like the online softmax.
  float M = -INFINITY, L = 0.f, acc = 0.f;
  for (int c = 0; c < ns; c += kMergeChunk) {
    float m[kMergeChunk], l[kMergeChunk], x[kMergeChunk];
#pragma unroll
    for (int u = 0; u < kMergeChunk; ++u) {
      const int s = min(c + u, a.max_chunks - 1);
      m[u] = wm[s * sm];
      l[u] = wm[s * sm + 1];
      x[u] = wo[s * so];
    }
    float mc = M;
#pragma unroll
    for (int u = 0; u < kMergeChunk; ++u)
      if (c + u < ns) mc = fmaxf(mc, m[u]);
    const float r = fast_exp2(M - mc);  // first round: exp2(-inf) = 0
    L *= r;
    acc *= r;
#pragma unroll
    for (int u = 0; u < kMergeChunk; ++u) {
      const float w = fast_exp2(m[u] - mc);  // fused multiply-adds, as merge_row4
      if (c + u < ns) {
        L = __builtin_fmaf(l[u], w, L);
        acc = __builtin_fmaf(x[u], w, acc);
      }
    }
    M = mc;
  }
  float res = acc * (1.f / L);  // as the split kernel rounds it: one pass and two agree bit for bit
  if (ctx_raw > a.max_ctx) res = NAN;  // caller broke the max_context_len contract
  o[d] = to_f16(res);
  if (a.lse && d == 0) a.lse[static_cast<int64_t>(b) * a.Hq + h] = (M + log2f(L)) * kLn2;
}

// The same merge with one block per (KV head, sequence) of g D / 4 threads:
// thread (q head col, features 4 d4 .. + 3) merges by merge_row4, loading
// 16-byte pieces of O, and chunks past the sequence's count repeat its last
// chunk instead of reading other slots.  Per output element the arithmetic
// is decode_merge_kernel's, so the two give the same bits.  Needs a 16-byte
// aligned workspace.
template <int D>
__global__ __launch_bounds__(kCols * D / 4) void decode_merge_rows_kernel(MergeArgs a) {
  constexpr int D4 = D / 4;
  const int kvh = blockIdx.x, b = blockIdx.y;
  const int col = static_cast<int>(threadIdx.x) / D4, d = 4 * (static_cast<int>(threadIdx.x) % D4);
  const int ctx_raw = a.ctx_lens ? a.ctx_lens[b] : a.max_ctx;
  const int ctx = min(max(ctx_raw, 0), a.max_ctx);
  const int ns = chunks_of(ctx, a.chunk_pages);
  if (a.skip_single && ns == 1) return;
  const int64_t row = static_cast<int64_t>(b) * a.Hq + kvh * a.g + col;
  _Float16* o = a.out + row * D + d;
  if (ctx == 0) {  // empty context: zeros, as torch's CPU SDPA returns
    *reinterpret_cast<f16x4*>(o) = f16x4{0, 0, 0, 0};
    if (a.lse && d == 0) a.lse[row] = -INFINITY;
    return;
  }
  const int64_t slot0 = (static_cast<int64_t>(b) * a.Hkv + kvh) * a.max_chunks;
  const float* wo = a.ws + (slot0 * a.g + col) * D + d;
  const float* wm = a.ws + static_cast<int64_t>(a.B) * a.Hkv * a.max_chunks * a.g * D + (slot0 * a.g + col) * 2;
  const int64_t so = static_cast<int64_t>(a.g) * D;  // chunk stride of wo
  const int sm = 2 * a.g;                              // chunk stride of wm
  float M, L;
  const f32x4 acc = merge_row4(
      ns, [&](int s) { return *reinterpret_cast<const f32x2*>(wm + s * sm); },
      [&](int s) { return *reinterpret_cast<const f32x4*>(wo + s * so); }, M, L);
  const float inv = 1.f / L;
  const bool bad = ctx_raw > a.max_ctx;  // caller broke the max_context_len contract
  f16x4 rv;
#pragma unroll
  for (int e = 0; e < 4; ++e) rv[e] = to_f16(bad ? NAN : acc[e] * inv);
  *reinterpret_cast<f16x4*>(o) = rv;
  if (a.lse && d == 0) a.lse[row] = (M + log2f(L)) * kLn2;
}

// Chunks of the longest context: a chunk is kWaves wavefronts' shares of at
// most split_tokens tokens each.
int64_t max_chunks_for(int max_ctx, int split_tokens) {
  const int64_t chunk_tokens = static_cast<int64_t>(kWaves) * split_tokens;
  return max_ctx <= 0 ? 1 : (max_ctx + chunk_tokens - 1) / chunk_tokens;
}

}  // namespace

extern "C" size_t spyre_paged_decode_attn_workspace_bytes(int B, int Hq, int Hkv, int D,
                                                          int max_context_len, int split_tokens) {
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || D <= 0 || split_tokens <= 0 || Hq % Hkv) return 0;
  const int64_t g = Hq / Hkv;
  const int64_t nc = max_chunks_for(max_context_len, split_tokens);
  // The chunk partials (fp32 O per q head and feature, m, l), then an
  // arrival flag per (sequence, KV head, chunk) for the one-call entry.
  return static_cast<size_t>(B) * Hkv * nc * (g * (D + 2) + 1) * sizeof(float);
}

namespace {

// Split-kernel workgroups that run at once on the current device (CUs times
// workgroups per CU), cached per device; 0 if the runtime cannot say.
int split_slots(int D) {
  static std::atomic<int> cache[64][2];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  std::atomic<int>& c = cache[dev][D == 128];
  int v = c.load(std::memory_order_relaxed);
  if (v > 0) return v;
  int cus = 0, per_cu = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  const hipError_t e =
      D == 128 ? hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, decode_split_list_kernel<128>, kThreads, 0)
               : hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, decode_split_list_kernel<64>, kThreads, 0);
  if (e != hipSuccess || cus <= 0 || per_cu <= 0) return 0;
  v = cus * per_cu;
  c.store(v, std::memory_order_relaxed);
  return v;
}

// Pages per chunk.  The requested size cp0 (kWaves x split) may grow by up
// to a quarter when that packs the workgroups of max_context_len-long
// sequences into fewer rounds of the device's slots (cost = rounds x pages
// per chunk); larger chunks never need more workspace than cp0's.  Depends
// only on the call's sizes and the device, so the two passes of a two-pass
// call agree.
int balanced_chunk_pages(int64_t pairs, int max_ctx, int cp0, int slots) {
  const int64_t n = pages_of(max_ctx);
  if (slots <= 0 || n <= cp0) return cp0;
  auto cost = [&](int cp) {
    const int64_t nch = (n + cp - 1) / cp;
    const int64_t per = (n + nch - 1) / nch;  // pages of the largest chunk (equal shares)
    return (pairs * nch + slots - 1) / slots * per;
  };
  int best = cp0;
  int64_t best_cost = cost(cp0);
  for (int cp = cp0 + 1; cp <= cp0 + cp0 / 4; ++cp) {
    const int64_t c = cost(cp);
    if (c < best_cost) {
      best = cp;
      best_cost = c;
    }
  }
  return best;
}

struct Plan {
  SplitArgs sa;
  MergeArgs ma;
  dim3 g1, g2;
  int D;
  bool list;
  bool multi_chunk;  // some context may need more than one chunk
};

int plan_attn(const void* q, const void* k_cache, const void* v_cache, const int32_t* block_table,
              int64_t bt_stride, const int32_t* context_lens, void* out, float* lse, void* workspace,
              size_t workspace_bytes, int B, int Hq, int Hkv, int D, int page_size,
              int64_t num_pages, int max_context_len, int split_tokens, float scale, bool need_inputs,
              bool need_out, Plan& p) {
  SPYRE_REQUIRE(context_lens && workspace, SPYRE_EINVAL, "null pointer argument");
  SPYRE_REQUIRE(!need_inputs || (q && k_cache && v_cache && block_table), SPYRE_EINVAL,
                "null pointer argument");
  SPYRE_REQUIRE(!need_out || out, SPYRE_EINVAL, "null output pointer");
  SPYRE_REQUIRE(B > 0 && Hq > 0 && Hkv > 0 && Hq % Hkv == 0, SPYRE_EINVAL,
                "bad head counts B=%d Hq=%d Hkv=%d", B, Hq, Hkv);
  const int g = Hq / Hkv;
  SPYRE_REQUIRE(g <= kCols, SPYRE_EUNSUPPORTED, "GQA group %d > %d", g, kCols);
  SPYRE_REQUIRE(D == 64 || D == 128, SPYRE_EUNSUPPORTED, "head_dim %d not in {64, 128}", D);
  SPYRE_REQUIRE(page_size == kPage, SPYRE_EUNSUPPORTED, "page_size %d != %d", page_size, kPage);
  SPYRE_REQUIRE(split_tokens > 0 && split_tokens % kPage == 0, SPYRE_EINVAL,
                "split_tokens %d must be a positive multiple of %d", split_tokens, kPage);
  SPYRE_REQUIRE(max_context_len >= 0 && bt_stride >= 0, SPYRE_EINVAL,
                "bad max_context_len / bt_stride");
  SPYRE_REQUIRE(!need_inputs || num_pages > 0, SPYRE_EINVAL, "bad num_pages");
  SPYRE_REQUIRE(!need_inputs || B == 1 || bt_stride * kPage >= max_context_len, SPYRE_EINVAL,
                "block table rows (%lld pages) shorter than max_context_len %d",
                static_cast<long long>(bt_stride), max_context_len);
  const size_t need =
      spyre_paged_decode_attn_workspace_bytes(B, Hq, Hkv, D, max_context_len, split_tokens);
  SPYRE_REQUIRE(workspace_bytes >= need, SPYRE_ENOSPC, "workspace %zu < %zu bytes",
                workspace_bytes, need);
  SPYRE_REQUIRE(split_tokens <= (1 << 24), SPYRE_EUNSUPPORTED, "split_tokens %d > 2^24",
                split_tokens);
  const int64_t max_chunks = max_chunks_for(max_context_len, split_tokens);
  const int64_t items = static_cast<int64_t>(B) * Hkv * max_chunks;
  SPYRE_REQUIRE(items < (int64_t{1} << 31) && Hkv <= 65535 && B <= 65535,
                SPYRE_EUNSUPPORTED, "too many work items (B=%d Hkv=%d chunks=%lld)", B, Hkv,
                static_cast<long long>(max_chunks));
  const int chunk_pages = balanced_chunk_pages(static_cast<int64_t>(B) * Hkv, max_context_len,
                                               kWaves * (split_tokens / kPage), split_slots(D));
  p.sa = SplitArgs{static_cast<const _Float16*>(q), static_cast<const _Float16*>(k_cache),
                   static_cast<const _Float16*>(v_cache), block_table, bt_stride, context_lens,
                   static_cast<float*>(workspace), static_cast<_Float16*>(out), lse, num_pages, B,
                   Hq, Hkv, g, static_cast<int>(max_chunks), chunk_pages, max_context_len,
                   scale * kLog2e};
  p.ma = MergeArgs{static_cast<const float*>(workspace), context_lens, static_cast<_Float16*>(out),
                   lse, B, Hq, Hkv, g, static_cast<int>(max_chunks), chunk_pages, max_context_len, 0};
  p.D = D;
  p.list = B <= kMaxListSeqs;
  // List mode: an upper bound on the items; those past the real count are
  // numbered last and exit at once.  Grid mode: (chunk, KV head, sequence).
  p.g1 = p.list ? dim3(static_cast<unsigned>(items))
                : dim3(static_cast<unsigned>(max_chunks), Hkv, B);
  p.multi_chunk = max_chunks > 1;
  p.g2 = dim3(Hq, B);
  return SPYRE_OK;
}

// Whether a call of several chunks merges them inside the split kernel: its
// work list (at most B Hkv max_chunks items) fits one round of the current
// device's workgroup slots and the workspace (partials and flags) is
// addressable with 32-bit offsets.
bool merges_in_kernel(int B, int Hq, int Hkv, int D, int max_context_len, int split_tokens) {
  const int64_t slots = split_slots(D);
  return slots > 0 && static_cast<int64_t>(B) * Hkv * max_chunks_for(max_context_len, split_tokens) <= slots &&
         spyre_paged_decode_attn_workspace_bytes(B, Hq, Hkv, D, max_context_len, split_tokens) < (size_t{1} << 31);
}

int launch_split(const Plan& p, hipStream_t st) {
  if (p.list && p.D == 128)
    decode_split_list_kernel<128><<<p.g1, kThreads, 0, st>>>(p.sa);
  else if (p.list)
    decode_split_list_kernel<64><<<p.g1, kThreads, 0, st>>>(p.sa);
  else if (p.D == 128)
    decode_split_kernel<128><<<p.g1, kThreads, 0, st>>>(p.sa);
  else
    decode_split_kernel<64><<<p.g1, kThreads, 0, st>>>(p.sa);
  const hipError_t e = hipGetLastError();
  SPYRE_REQUIRE(e == hipSuccess, SPYRE_EHIP, "decode split launch failed: %s", hipGetErrorString(e));
  return SPYRE_OK;
}

int launch_merge(const Plan& p, hipStream_t st) {
  const unsigned rows_threads = static_cast<unsigned>(p.ma.g * p.D / 4);
  // Row vectors when the workspace is 16-byte aligned: ragged batch of 64
  // sequences 699.2 -> 695.3 us, B 32 x 32768 tokens 666.8 -> 665.2 (A/B on
  // one box, two alternations).
  const bool rows = reinterpret_cast<uintptr_t>(p.ma.ws) % 16 == 0;
  if (rows && p.D == 128)
    decode_merge_rows_kernel<128><<<dim3(p.ma.Hkv, p.ma.B), rows_threads, 0, st>>>(p.ma);
  else if (rows)
    decode_merge_rows_kernel<64><<<dim3(p.ma.Hkv, p.ma.B), rows_threads, 0, st>>>(p.ma);
  else if (p.D == 128)
    decode_merge_kernel<128><<<p.g2, 128, 0, st>>>(p.ma);
  else
    decode_merge_kernel<64><<<p.g2, 64, 0, st>>>(p.ma);
  const hipError_t e = hipGetLastError();
  SPYRE_REQUIRE(e == hipSuccess, SPYRE_EHIP, "decode merge launch failed: %s", hipGetErrorString(e));
  return SPYRE_OK;
}

}  // namespace

extern "C" int spyre_paged_decode_attn_split_f16(
    const void* q, const void* k_cache, const void* v_cache, const int32_t* block_table,
    int64_t bt_stride, const int32_t* context_lens, void* workspace, size_t workspace_bytes, int B,
    int Hq, int Hkv, int D, int page_size, int64_t num_pages, int max_context_len, int split_tokens,
    float scale, void* stream) {
  spyre_hip::clear_error();
  Plan p;
  int rc = plan_attn(q, k_cache, v_cache, block_table, bt_stride, context_lens, nullptr, nullptr,
                     workspace, workspace_bytes, B, Hq, Hkv, D, page_size, num_pages,
                     max_context_len, split_tokens, scale, true, false, p);
  if (rc != SPYRE_OK) return rc;
  return launch_split(p, static_cast<hipStream_t>(stream));
}

extern "C" int spyre_paged_decode_attn_merge_f16(const int32_t* context_lens, const void* workspace,
                                                 size_t workspace_bytes, void* out, float* lse, int B,
                                                 int Hq, int Hkv, int D, int max_context_len,
                                                 int split_tokens, void* stream) {
  spyre_hip::clear_error();
  Plan p;
  int rc = plan_attn(nullptr, nullptr, nullptr, nullptr, 0, context_lens, out, lse,
                     const_cast<void*>(workspace), workspace_bytes, B, Hq, Hkv, D, kPage, 1,
                     max_context_len, split_tokens, 1.f, false, true, p);
  if (rc != SPYRE_OK) return rc;
  return launch_merge(p, static_cast<hipStream_t>(stream));  // every sequence
}

extern "C" int spyre_paged_decode_attn_kernels(int B, int Hq, int Hkv, int D, int max_context_len,
                                               int split_tokens) {
  spyre_hip::clear_error();
  SPYRE_REQUIRE(B > 0 && Hq > 0 && Hkv > 0 && Hq % Hkv == 0 && (D == 64 || D == 128) && max_context_len >= 0 &&
                    split_tokens > 0 && split_tokens % kPage == 0,
                SPYRE_EINVAL, "bad decode sizes");
  if (max_chunks_for(max_context_len, split_tokens) <= 1) return 1;
  return merges_in_kernel(B, Hq, Hkv, D, max_context_len, split_tokens) ? 1 : 2;
}

extern "C" int spyre_paged_decode_attn_f16(const void* q, const void* k_cache, const void* v_cache,
                                           const int32_t* block_table, int64_t bt_stride,
                                           const int32_t* context_lens, void* out, float* lse,
                                           void* workspace, size_t workspace_bytes, int B, int Hq,
                                           int Hkv, int D, int page_size, int64_t num_pages,
                                           int max_context_len, int split_tokens, float scale,
                                           void* stream) {
  spyre_hip::clear_error();
  Plan p;
  int rc = plan_attn(q, k_cache, v_cache, block_table, bt_stride, context_lens, out, lse, workspace,
                     workspace_bytes, B, Hq, Hkv, D, page_size, num_pages, max_context_len,
                     split_tokens, scale, true, true, p);
  if (rc != SPYRE_OK) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  // Several chunks: merged inside the split kernel when its work list (at
  // most B Hkv max_chunks items) fits one round of the device's workgroup
  // slots and the workspace (partials and flags, moved as 16-byte pieces)
  // is 16-byte aligned and addressable with 32-bit offsets; else the merge
  // pass.  In longer lists each merging or
  // flag-setting workgroup holds its slot through its device-scope round
  // trips while the next item waits: B 4 x 64 / 8 heads x 131073 tokens
  // (33 chunks, 1056 items) measured 346.5 -> 355.5 us merged in the kernel,
  // B 1 x 32 / 8 x 131072 (264 items) 89.4 -> 88.3.
  const bool fused = p.multi_chunk && reinterpret_cast<uintptr_t>(workspace) % 16 == 0 &&
                     merges_in_kernel(B, Hq, Hkv, D, max_context_len, split_tokens);
  if (fused) p.sa.ticket = spyre_hip::next_call_ticket();
  if ((rc = launch_split(p, st)) != SPYRE_OK) return rc;
  if (!p.multi_chunk || fused) return SPYRE_OK;  // every output written
  p.ma.skip_single = 1;
  return launch_merge(p, st);
}

// ------------------------------------------------ dense K / V (SDPA decode) --

namespace spyre_hip {

uint32_t next_call_ticket() {
  static std::atomic<uint32_t> tickets{0};
  uint32_t t = tickets.fetch_add(1, std::memory_order_relaxed) + 1;
  if (t == 0) t = tickets.fetch_add(1, std::memory_order_relaxed) + 1;  // 0: a cleared flag
  return t;
}

DenseDecodePlan dense_decode_plan(int B, int Hq, int Hkv, int Skv, int D) {
  DenseDecodePlan p;
  if ((D != 64 && D != 128) || B <= 0 || B > 65535 || Hkv <= 0 || Hq % Hkv != 0 || Hq / Hkv > kCols || Skv <= 0)
    return p;
  const int slots = split_slots(D) > 0 ? split_slots(D) : 256;
  const int64_t pairs = static_cast<int64_t>(B) * Hkv;
  // Tokens per wavefront: 512 (as the paged default), halved down to one
  // page while the grid would leave workgroup slots empty.
  int split = 512;
  while (split > kPage && pairs * max_chunks_for(Skv, split) < slots) split /= 2;
  const int64_t nc0 = max_chunks_for(Skv, split);
  // At least half the slots busy: batch 3 x 4096 tokens (192 workgroups)
  // 26.2 -> 15.1 us against the LDS kernel's key split, batch 24 x 512
  // 27.8 -> 12.8 us.
  if (2 * pairs * nc0 < slots || pairs * nc0 >= (int64_t{1} << 31)) return p;
  // Four wavefronts per item, each with twice the runs, when the grid of
  // eight-wavefront items would take more than one round of the device and
  // the four-wavefront grid takes one (its workgroups hold half the waves,
  // so about twice as many are resident): every wavefront then streams as
  // long a share as in a one-round grid.
  const int64_t slots4 = dense4_slots(D);
  const int64_t nc4 = (static_cast<int64_t>(Skv) + 4 * split - 1) / (4 * split);
  const int W = split == 512 && pairs * nc0 > slots && slots4 > 0 && pairs * nc4 <= slots4 ? 4 : kWaves;
  p.waves = W;
  p.chunk_pages = balanced_chunk_pages(pairs, Skv, W * (split / kPage), W == 4 ? static_cast<int>(slots4) : slots);
  p.chunks = chunks_of(Skv, p.chunk_pages);
  // Several chunks: their fp32 partials (O per q head and feature; m, l),
  // then an arrival flag per chunk (uint32).
  p.ws_bytes = p.chunks > 1 ? static_cast<size_t>(pairs) * p.chunks * ((Hq / Hkv) * (D + 2) + 1) * sizeof(float) : 0;
  // The chunks merge in the kernel when its grid fits one round of the
  // device's slots (as for the paged kernel) and the workspace fits 32-bit
  // offsets; otherwise the merge pass.
  p.fused = p.chunks > 1 && pairs * p.chunks <= (W == 4 ? slots4 : slots) && p.ws_bytes < (size_t{1} << 31);
  p.ok = true;
  return p;
}

int dense_decode_launch(const DenseDecodePlan& plan, const void* q, const int64_t* q_strides, const void* k,
                        const int64_t* k_strides, const void* v, const int64_t* v_strides, void* out, float* lse,
                        void* workspace, int B, int Hq, int Hkv, int Skv, int D, float scale, void* stream) {
  SPYRE_REQUIRE(plan.ok && (D == 64 || D == 128), SPYRE_EUNSUPPORTED, "dense decode: call not covered");
  SPYRE_REQUIRE(plan.chunks == 1 || workspace, SPYRE_EINVAL, "dense decode: no workspace");
  for (int i = 0; i < 3; ++i)
    SPYRE_REQUIRE(k_strides[i] >= 0 && v_strides[i] >= 0, SPYRE_EUNSUPPORTED, "dense decode: negative stride");
  SPYRE_REQUIRE(k_strides[2] < (int64_t{1} << 23) && v_strides[2] < (int64_t{1} << 23), SPYRE_EUNSUPPORTED,
                "dense decode: token stride 2^23 elements or more");
  // Rows of whole tokens (a short context's loads of tokens past it are
  // then wholly out of range, load_k_dense), or one row for every token.
  SPYRE_REQUIRE((k_strides[2] == 0 || k_strides[2] >= D) && (v_strides[2] == 0 || v_strides[2] >= D),
                SPYRE_EUNSUPPORTED, "dense decode: token stride between 0 and head_dim");
  SplitArgs sa{};
  sa.q = static_cast<const _Float16*>(q);
  sa.k = static_cast<const _Float16*>(k);
  sa.v = static_cast<const _Float16*>(v);
  sa.ws = static_cast<float*>(workspace);
  sa.out = static_cast<_Float16*>(out);
  sa.lse = lse;
  sa.B = B;
  sa.Hq = Hq;
  sa.Hkv = Hkv;
  sa.g = Hq / Hkv;
  sa.max_chunks = plan.chunks;
  sa.chunk_pages = plan.chunk_pages;
  sa.max_ctx = Skv;
  sa.scale_log2 = scale * kLog2e;
  sa.q_sb = q_strides[0];
  sa.q_sh = q_strides[1];
  sa.k_sb = k_strides[0];
  sa.k_sh = k_strides[1];
  sa.k_ss = k_strides[2];
  sa.v_sb = v_strides[0];
  sa.v_sh = v_strides[1];
  sa.v_ss = v_strides[2];
  const bool fused = plan.fused;  // the chunks merge inside the kernel
  sa.ticket = fused ? next_call_ticket() : 0;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t items = static_cast<int64_t>(B) * Hkv * plan.chunks;
  const dim3 grid(static_cast<unsigned>(items));
  if (D == 128 && plan.waves == 4)
    decode_dense_kernel<128, 4><<<grid, 4 * 64, 0, st>>>(sa);
  else if (D == 128)
    decode_dense_kernel<128><<<grid, kThreads, 0, st>>>(sa);
  else if (plan.waves == 4)
    decode_dense_kernel<64, 4><<<grid, 4 * 64, 0, st>>>(sa);
  else
    decode_dense_kernel<64><<<grid, kThreads, 0, st>>>(sa);
  hipError_t e = hipGetLastError();
  SPYRE_REQUIRE(e == hipSuccess, SPYRE_EHIP, "dense decode launch failed: %s", hipGetErrorString(e));
  if (plan.chunks == 1 || fused) return SPYRE_OK;  // every sequence's output written
  const MergeArgs ma{sa.ws, nullptr, sa.out, lse, B, Hq, Hkv, sa.g, plan.chunks, plan.chunk_pages, Skv, 0};
  // The workspace is 16-byte aligned on this route (the SDPA entry checks).
  if (D == 128)
    decode_merge_rows_kernel<128><<<dim3(Hkv, B), sa.g * 128 / 4, 0, st>>>(ma);
  else
    decode_merge_rows_kernel<64><<<dim3(Hkv, B), sa.g * 64 / 4, 0, st>>>(ma);
  e = hipGetLastError();
  SPYRE_REQUIRE(e == hipSuccess, SPYRE_EHIP, "dense decode merge launch failed: %s", hipGetErrorString(e));
  return SPYRE_OK;
}

}  // namespace spyre_hip

// ------------------------------------------- dense route address check --

namespace {

// Every load of the dense route's run of `rows` tokens (64: a window,
// load_*_dense<D, true>; fewer: a short context, load_*_dense<D, false>):
// f(is_k, voffset, soffset, width) with the per-lane and scalar byte
// offsets the kernel passes.
template <typename F>
void for_each_dense_load(int D, int rows, int64_t k_row, int64_t v_row, F&& f) {
  const bool whole = rows == kPage;
  for (int lane = 0; lane < 64; ++lane) {
    for (int jh = 0; jh < 4; ++jh)
      for (int t = 0; t < D / 64; ++t)
        for (int y = 0; y < 2; ++y) {
          const int64_t base = dense_k_tok(lane, y) * k_row + dense_k_col(lane, y);  // LoadOffsets::dense
          const int64_t so = dense_k_dtok(jh) * k_row + 128 * t;
          f(true, whole ? base : base + so, whole ? so : 0, 16);
        }
    for (int j = 0; j < 2; ++j)
      for (int i = 0; i < 8; ++i) {
        const int col = D == 128 ? dense_v_col<128>(lane) : dense_v_col<64>(lane);
        const int w = D == 128 ? kDenseVBytes<128> : kDenseVBytes<64>;
        const int64_t base = dense_v_tok(lane) * v_row + col, so = (32 * j + i) * v_row;
        f(false, whole ? base : base + so, whole ? so : 0, w);
      }
  }
}

}  // namespace

extern "C" int spyre_dense_decode_load_extent(int D, int rows, int64_t k_row, int64_t v_row, int64_t* k_end,
                                              int64_t* v_end, int64_t* n_loads) {
  spyre_hip::clear_error();
  SPYRE_REQUIRE(D == 64 || D == 128, SPYRE_EINVAL, "head_dim %d not in {64, 128}", D);
  SPYRE_REQUIRE(rows >= 1 && rows <= kPage, SPYRE_EINVAL, "rows %d not in [1, %d]", rows, kPage);
  SPYRE_REQUIRE(k_row >= 0 && v_row >= 0 && k_end && v_end && n_loads, SPYRE_EINVAL, "bad arguments");
  // The resources' ranges (stream_pages' locate).  A load is counted as
  // touching memory unless its per-lane offset alone is out of range -- the
  // range check is not assumed to cover the scalar offset -- and then as
  // touching every byte up to voffset + soffset + width.
  const int64_t k_range = (rows - 1) * k_row + 2 * D, v_range = (rows - 1) * v_row + 2 * D;
  *k_end = *v_end = *n_loads = 0;
  for_each_dense_load(D, rows, k_row, v_row, [&](bool is_k, int64_t voff, int64_t soff, int w) {
    if (voff >= (is_k ? k_range : v_range)) return;  // out of range: zeros, no access
    int64_t& e = is_k ? *k_end : *v_end;
    e = std::max(e, voff + soff + w);
    ++*n_loads;
  });
  return SPYRE_OK;
}

// ------------------------------------------ the entry that allocates nothing --

// The chunk partials of spyre_paged_decode_attn_noalloc_f16.  Each GPU holds
// its own copy from the library's load to the end of the process.  In host
// code this name is a stand-in, not a device address: kernel arguments use
// the address scratch_address() returns for the current device.
static __device__ __align__(256) unsigned char scratch[SPYRE_DECODE_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;

// The current device's address of `scratch`, taken once per device (with
// that device current) by hipGetSymbolAddress; nullptr, with the error
// recorded, when the runtime cannot give it.
void* scratch_address() {
  static std::atomic<void*> addr[kMaxDevices];
  static std::mutex mu;
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    spyre_hip::set_error("no usable current device (%s, device %d)", hipGetErrorString(e), dev);
    return nullptr;
  }
  void* p = addr[dev].load(std::memory_order_acquire);
  if (p) return p;
  std::lock_guard<std::mutex> lock(mu);
  p = addr[dev].load(std::memory_order_relaxed);
  if (!p) {
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      spyre_hip::set_error("hipGetSymbolAddress of the decode scratch failed on device %d: %s", dev,
                           hipGetErrorString(e));
      return nullptr;
    }
    addr[dev].store(p, std::memory_order_release);
  }
  return p;
}

}  // namespace

extern "C" int spyre_paged_decode_attn_noalloc_f16(const void* q, const void* k_cache,
                                                   const void* v_cache, const int32_t* block_table,
                                                   int64_t bt_stride, const int32_t* context_lens,
                                                   void* out, float* lse, int B, int Hq, int Hkv,
                                                   int D, int page_size, int64_t num_pages,
                                                   int max_context_len, int split_tokens,
                                                   float scale, void* stream) {
  spyre_hip::clear_error();
  // Checked before any HIP call: a call that does not fit never touches the device.
  const size_t need =
      spyre_paged_decode_attn_workspace_bytes(B, Hq, Hkv, D, max_context_len, split_tokens);
  SPYRE_REQUIRE(need <= SPYRE_DECODE_SCRATCH_BYTES, SPYRE_ENOSPC,
                "decode needs %zu bytes of chunk partials, more than the %zu bytes of the "
                "library's scratch; pass a workspace to spyre_paged_decode_attn_f16 instead",
                need, static_cast<size_t>(SPYRE_DECODE_SCRATCH_BYTES));
  void* ws = scratch_address();
  if (!ws) return SPYRE_EHIP;
  // Nothing in the scratch needs clearing: the split pass writes every
  // partial a merge uses, the merge discards the rest by selects, and the
  // arrival flags of an in-kernel merge are cleared by the call that sets
  // them (a new call's ticket matches no flag an older call left).
  return spyre_paged_decode_attn_f16(q, k_cache, v_cache, block_table, bt_stride, context_lens, out,
                                     lse, ws, SPYRE_DECODE_SCRATCH_BYTES, B, Hq, Hkv, D, page_size,
                                     num_pages, max_context_len, split_tokens, scale, stream);
}
