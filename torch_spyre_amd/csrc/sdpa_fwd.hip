// Scaled dot-product attention forward for gfx950 (spyre_sdpa_fwd_f16):
// prefill and any Sq, with GQA, causal masking or an additive / boolean mask,
// and the natural-log logsumexp.
//
// Semantics (torch_spyre/_inductor/decompositions.py:523-609, with torch's
// CPU SDPA as the numerical reference):
//   out[b,h,i,:] = softmax_j(scale * q[b,h,i,:] . k[b,h/g,j,:] + bias[b,h,i,j]) v[b,h/g,j,:]
// bias = 0, or the mask (boolean masks keep where true), or for causal
// attention -inf where j > i (top-left aligned, triu(diagonal=1)).  A row
// whose keys are all masked gives zeros and LSE -inf (torch's CPU result;
// the reference's torch.softmax would give NaN there).
//
// Kernels, on the caller's stream:
//  * sdpa_fwd_lds_kernel serves calls without a mask (plain or causal) and
//    fp16 / boolean masks whose rows are whole 16-byte units.  A workgroup
//    of 8 wavefronts takes 256 queries of one (sequence, q head); wavefront w
//    takes 32.  Per 64-key step the K and V tiles (row-major, padded) move
//    from L2 straight into LDS (buffer loads with the LDS flag), once for all
//    8 wavefronts:
//       S^T[key, q] = K[key, :] Q^T[:, q]     2 x D/16 MFMA 32x32x16
//       online softmax in fp32 (exp2 domain), lazy rescaling of the max;
//       O^T[d, q] += V^T[d, key] P^T[key, q]  4 x D/32 MFMA 32x32x16
//    with the V^T operands read from the row-major V tile by transposing
//    LDS reads.  The loop is software-pipelined: step t's softmax overlaps
//    S(t+1).  A mask is staged per wavefront beside the tiles, a step ahead;
//    steps it blanks for the whole wavefront skip their softmax and P V.
//  * Other masks (fp32 biases, rows that are not whole 16-byte units):
//    1. v_token_sticks_kernel: V [B, Hkv, Skv, D] (rows may be strided) ->
//       Vt [B, Hkv, D, S64] in the workspace: V with its sticks along tokens
//       (the transpose-restick of each head), zero-padded to S64 = ceil(Skv
//       / 64) * 64, so the PV product's reduction dim (keys) is contiguous.
//    2. sdpa_fwd_kernel: one wavefront per 32 queries of one (sequence, q
//       head), four per workgroup, streaming 64 keys per step from L2:
//         S^T[key, q] = K[key, :] Q^T[:, q]   4 x D/32 x 2 MFMA 16x16x32
//         O^T[d, q] += Vt[d, key] P^T[key, q]   D/16 x 2 x 2 MFMA 16x16x32
//       reading the mask element by element through its broadcast strides.
// In both, the keys of the S rows are permuted so that each lane's P values
// are the 8 consecutive keys the PV operand needs (no lane exchange), and
// causal attention stops each wavefront at its last query's key.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <type_traits>

#include "decode_dense.h"
#include "spyre_common.h"
#include "transpose8.h"

namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
using spyre_hip::u32x4_t;

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kQ = 32;      // queries per wavefront (two MFMA column tiles)
constexpr int kKeys = 64;   // keys per step
constexpr int kStick = 64;  // Vt token padding: whole 64-key steps
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

__device__ __forceinline__ float wave_xor(float x, int m) { return __shfl_xor(x, m, 64); }
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// K and Vt are read with buffer loads: the (sequence, head) base and extent
// in SGPRs, a 32-bit per-lane byte offset in one VGPR, the load-invariant
// part in an SGPR / immediate.  Accesses past the extent read zeros.
typedef __amdgpu_buffer_rsrc_t Rsrc;
constexpr int kRsrcWord3 = 0x00020000;  // raw (untyped) buffer, 32-bit format
// 16 bytes per lane from buffer offset voff into LDS: lane l writes the 16
// bytes at dst + 16 l (dst wave-uniform).  Lanes whose offset lies past the
// buffer's range write zeros.
// ds_read_b64_tr_b16 at LDS element p (see the V operand reads below).
__device__ __forceinline__ short __attribute__((ext_vector_type(4))) tr_read4(const _Float16* p) {
  typedef short v4s __attribute__((ext_vector_type(4)));
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)(p));
}

__device__ __forceinline__ void load_lds16(Rsrc r, _Float16* dst, uint32_t voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)dst, 16, voff, 0, 0, 0);
}

// Range of the buffer descriptors whose bases move with the key step; the
// host keeps every head's K and Vt span within it.
constexpr uint32_t kBufRange = 0x7ffffff0u;

__device__ __forceinline__ Rsrc make_rsrc(const _Float16* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16*>(base), 0, bytes, kRsrcWord3);
}

__device__ __forceinline__ f16x8 bload(Rsrc r, int voff, int soff) {
  return __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}

// S^T block jh (16 keys of the step): MFMA row i <-> key 32(jh/2) + 8(i/4) + 4(jh%2) + i%4.
__device__ __forceinline__ int key_of(int jh, int i) {
  return 32 * (jh >> 1) + 8 * (i >> 2) + 4 * (jh & 1) + (i & 3);
}

// ---- 1. V -> token sticks -------------------------------------------------

struct VtArgs {
  const _Float16* v;
  int64_t sb, sh, ss;  // V strides (elements); d stride 1
  _Float16* vt;        // [B, Hkv, D, s64]
  int Hkv, Skv, s64, D;
  int64_t tiles;       // 64 x 64 tiles
};

// One wavefront per 64 tokens x 64 features: each lane loads an 8 x 8 block
// as eight 16-byte token rows, transposes it in registers and stores eight
// 16-byte feature rows of Vt.  Tokens past Skv are written as zeros.
__global__ __launch_bounds__(kThreads) void v_token_sticks_kernel(VtArgs a) {
  const int64_t tile = static_cast<int64_t>(blockIdx.x) * kWaves + threadIdx.x / 64;
  if (tile >= a.tiles) return;
  const int lane = threadIdx.x % 64;
  const int ts_n = a.s64 / 64, td_n = a.D / 64;
  const int ts = static_cast<int>(tile % ts_n);
  const int64_t r = tile / ts_n;
  const int td = static_cast<int>(r % td_n);
  const int64_t bh = r / td_n;
  const int64_t b = bh / a.Hkv, kvh = bh % a.Hkv;
  const int s0 = ts * 64 + (lane / 8) * 8, d0 = td * 64 + (lane % 8) * 8;
  const _Float16* src = a.v + b * a.sb + kvh * a.sh + d0;
  u32x4_t x[8], y[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const int s = s0 + t;
    x[t] = s < a.Skv ? *reinterpret_cast<const u32x4_t*>(src + s * a.ss) : u32x4_t{0, 0, 0, 0};
  }
  spyre_hip::transpose8x8_b16(x, y);
  _Float16* dst = a.vt + (bh * a.D + d0) * a.s64 + s0;
#pragma unroll
  for (int e = 0; e < 8; ++e) *reinterpret_cast<u32x4_t*>(dst + e * a.s64) = y[e];
}

// ---- 2. attention -----------------------------------------------------------

enum MaskKind { kNoMask = 0, kMaskF16 = 1, kMaskF32 = 2, kMaskBool = 3 };

struct FwdArgs {
  const _Float16* q;
  const _Float16* k;
  const _Float16* vt;
  int64_t q_sb, q_sh, q_ss;
  int64_t k_sb, k_sh, k_ss;
  int64_t vt_sb, vt_sh;
  uint32_t k_bytes, vt_bytes;  // extent of one (sequence, KV head) of K / Vt
  const void* mask;
  int64_t m_sb, m_sh, m_sq, m_sk;
  _Float16* out;  // [B, Sq, Hq, D]
  float* lse;     // [B, Hq, Sq] or null
  int B, Hq, Hkv, g, Sq, Skv, s64, mask_kind, causal;
  float scale_log2;
};

// Mask element types by kind.
template <int MK> struct MaskElem { using T = uint8_t; };
template <> struct MaskElem<kMaskF16> { using T = _Float16; };
template <> struct MaskElem<kMaskF32> { using T = float; };

// Additive bias (log2 domain) of mask element x.
template <int MK>
__device__ __forceinline__ float bias_of(typename MaskElem<MK>::T x) {
  if constexpr (MK == kMaskBool)
    return x ? 0.f : -INFINITY;
  else
    return static_cast<float>(x) * kLog2e;
}

// MK: mask kind (a separate kernel each, so the unmasked one carries no mask code).
template <int D, int MK>
__global__ __launch_bounds__(kThreads, 2) void sdpa_fwd_kernel(FwdArgs a) {
  constexpr int DS = D / 32;  // QK k-steps
  constexpr int DT = D / 16;  // O row tiles
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64), lane = threadIdx.x % 64;
  const int b = blockIdx.z, h = blockIdx.y;
  const int q0 = (blockIdx.x * kWaves + wave) * kQ;
  if (q0 >= a.Sq) return;
  const int kvh = h / a.g;
  const int col = lane & 15, grp = lane >> 4;
  const _Float16* qp = a.q + b * a.q_sb + h * a.q_sh;
  const Rsrc kr = make_rsrc(a.k + b * a.k_sb + kvh * a.k_sh, a.k_bytes);
  const Rsrc vr = make_rsrc(a.vt + b * a.vt_sb + kvh * a.vt_sh, a.vt_bytes);

  // Q^T operands: lane (query column col, feature group grp).
  f16x8 qb[2][DS];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int qi = q0 + 16 * nt + col;
#pragma unroll
    for (int ds = 0; ds < DS; ++ds)
      qb[nt][ds] = qi < a.Sq ? *reinterpret_cast<const f16x8*>(qp + qi * a.q_ss + 32 * ds + 8 * grp)
                             : f16x8{};
  }

  float m_run[2] = {-INFINITY, -INFINITY}, l_run[2] = {0.f, 0.f};
  f32x4 o[2][DT];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt)
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) o[nt][dt] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Mask rows of this lane's two query columns (clamped into the mask).
  using MT = typename MaskElem<MK>::T;
  const MT* mrow[2] = {nullptr, nullptr};
  if constexpr (MK != kNoMask) {
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const int qc = min(q0 + 16 * nt + col, a.Sq - 1);
      mrow[nt] = static_cast<const MT*>(a.mask) + b * a.m_sb + h * a.m_sh + qc * a.m_sq;
    }
  }
  const int m_sk = static_cast<int>(a.m_sk);

  // Per-lane byte offsets: K row key_of(jh, col) (+ 16-byte feature group),
  // Vt row col (+ 8 keys of group grp).  Keys past Skv are masked below;
  // their K rows are clamped to the last row.
  const int vt_lane = (col * a.s64 + 8 * grp) * 2;
  // Causal: no key past this wavefront's last query is needed.
  const int key_end = a.causal ? min(a.Skv, q0 + kQ) : a.Skv;
  for (int kb = 0; kb < key_end; kb += kKeys) {
    f16x8 ka[4][DS];
#pragma unroll
    for (int jh = 0; jh < 4; ++jh) {
      const int key = min(kb + key_of(jh, col), a.Skv - 1);
      const int voff = static_cast<int>(key * a.k_ss * 2) + 16 * grp;
#pragma unroll
      for (int ds = 0; ds < DS; ++ds) ka[jh][ds] = bload(kr, voff, 64 * ds);
    }
    f32x4 sc[4][2];
#pragma unroll
    for (int jh = 0; jh < 4; ++jh) {
      sc[jh][0] = sc[jh][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ds = 0; ds < DS; ++ds) {
        sc[jh][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[jh][ds], qb[0][ds], sc[jh][0], 0, 0, 0);
        sc[jh][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[jh][ds], qb[1][ds], sc[jh][1], 0, 0, 0);
      }
    }
    // The K registers are free: the Vt operands load during the softmax.
    f16x8 va[DT][2];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int j = 0; j < 2; ++j) va[dt][j] = bload(vr, vt_lane + kb * 2, (16 * dt * a.s64 + 32 * j) * 2);
    // Lane (query column, group grp) holds keys kb + 32j + 8grp + 4h + v.
    f16x8 pb[2][2];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const int qi = q0 + 16 * nt + col;
      float mx = -INFINITY;
#pragma unroll
      for (int jh = 0; jh < 4; ++jh)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int key = kb + 32 * (jh >> 1) + 8 * grp + 4 * (jh & 1) + v;
          bool keep = key < a.Skv && qi < a.Sq;
          if (a.causal) keep = keep && key <= qi;
          float x = sc[jh][nt][v] * a.scale_log2;
          if constexpr (MK != kNoMask) x += bias_of<MK>(mrow[nt][min(key, a.Skv - 1) * m_sk]);
          x = keep ? x : -INFINITY;
          sc[jh][nt][v] = x;
          mx = fmaxf(mx, x);
        }
      mx = fmaxf(mx, wave_xor(mx, 16));
      mx = fmaxf(mx, wave_xor(mx, 32));
      const float m_new = fmaxf(m_run[nt], mx);
      const float m_use = m_new == -INFINITY ? 0.f : m_new;  // all masked so far: p = 0
      const float alpha = fast_exp2(m_run[nt] - m_use);
      float psum = 0.f;
#pragma unroll
      for (int jh = 0; jh < 4; ++jh)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const float p = fast_exp2(sc[jh][nt][v] - m_use);
          psum += p;
          pb[nt][jh >> 1][(jh & 1) * 4 + v] = static_cast<_Float16>(p);
        }
      l_run[nt] = l_run[nt] * alpha + psum;
      m_run[nt] = m_new;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) o[nt][dt] *= alpha;
    }
    // O^T += Vt[d, keys] P^T[keys, q]; Vt is zero past Skv (up to s64).
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        o[0][dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va[dt][j], pb[0][j], o[0][dt], 0, 0, 0);
        o[1][dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va[dt][j], pb[1][j], o[1][dt], 0, 0, 0);
      }
  }

  // Lane (query column, group grp) holds O^T[d = 16dt + 4grp + v][q].
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    float l = l_run[nt];
    l += wave_xor(l, 16);
    l += wave_xor(l, 32);
    const int qi = q0 + 16 * nt + col;
    if (qi >= a.Sq) continue;
    _Float16* op = a.out + ((static_cast<int64_t>(b) * a.Sq + qi) * a.Hq + h) * D;
    const float inv = l > 0.f ? 1.f / l : 0.f;  // every key masked: zeros
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      f16x4 r;
#pragma unroll
      for (int v = 0; v < 4; ++v) r[v] = static_cast<_Float16>(o[nt][dt][v] * inv);
      *reinterpret_cast<f16x4*>(op + 16 * dt + 4 * grp) = r;
    }
    if (a.lse && grp == 0)
      a.lse[(static_cast<int64_t>(b) * a.Hq + h) * a.Sq + qi] =
          l > 0.f ? (m_run[nt] + log2f(l)) * kLn2 : -INFINITY;
  }
}

// ---- 3. attention with K/V tiles shared through LDS (no mask) -------------
//
// One workgroup of kWaves2 wavefronts per 256 queries of one (sequence, q
// head); wavefront w takes 32 of them.  Per 64-key step t the workgroup
// stages the K tile and the V tile, both [64 keys][D] as K and V lie in
// memory, in LDS, and every wavefront reads its MFMA operands from there:
//   S^T[key, q] = K Q^T   2 x D/16 MFMA 32x32x16 (M = 32 keys, N = 32 queries)
//   O^T[d, q] += V^T P^T  D/32 x 4 MFMA 32x32x16
// The V^T operand (8 consecutive keys of one feature per lane) comes from
// the row-major V tile through the transposing LDS read ds_read_b64_tr_b16,
// so V needs no relayout before the kernel.
// The loop is software-pipelined: K runs one step ahead of V, so while the
// VALU computes step t's softmax the matrix cores already compute step
// t+1's scores and then step t's P V.  Two LDS slots each hold K(t+1) /
// K(t+2) and V(t) / V(t+1); the next tiles travel from L2 straight into
// LDS during a step's math.  LDS rows are padded so that the rows one
// operand read touches fall in distinct bank groups.  Workgroups are
// numbered so that those of one (sequence, KV head) run on one XCD (one L2),
// and for causal attention each head's latest (heaviest) query block starts
// first.

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef short v4i16 __attribute__((ext_vector_type(4)));

constexpr int kWaves2 = 8;
constexpr int kThreads2 = kWaves2 * 64;
constexpr int kQW = 32;             // queries per wavefront
constexpr int kQB = kWaves2 * kQW;  // queries per workgroup
constexpr int kKT = 64;             // keys per step
static_assert(kStick % kKT == 0, "the Vt padding must cover whole steps");
constexpr int kPadH = 8;            // LDS row padding, halves (16 bytes)
constexpr int kPrefetch = 4;        // LDS operand reads in flight ahead of the MFMA using them

template <int D>
struct Lds2 {
  static constexpr int kRowK = D + kPadH;    // K tile row (one key), halves
  // V tile row: a transposed read serves 32 lanes at once, 4 rows x 4
  // 8-byte units in each of two column groups 32 bytes apart; a row step of
  // 16 (D = 128: 160 halves) or 48 (D = 64: 96 halves) banks mod 64 puts all
  // of them in distinct banks.
  static constexpr int kRowV = D + 32;
  static constexpr int kK = kKT * kRowK;
  static constexpr int kSlot = kK + kKT * kRowV;  // one slot: a K tile and a V tile
};

// S^T row rho of a 32-key half maps to key key32_of(rho) of that half: MFMA
// row tile i (8 rows) of lane half h holds rows 8i + 4h + v (i, v < 4); they
// are the keys 16(i/2) + 8h + 4(i%2) + v, i.e. the two 8-key runs the PV
// operand of half h needs.
__device__ __forceinline__ int key32_of(int rho) {
  const int i = rho >> 3, h = (rho >> 2) & 1, v = rho & 3;
  return 16 * (i >> 1) + 8 * h + 4 * (i & 1) + v;
}

// max(x of lane l, x of lane l ^ 32), in every lane.
__device__ __forceinline__ float max_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, x), __builtin_bit_cast(unsigned, x),
                                                  false, false);
  return fmaxf(__builtin_bit_cast(float, static_cast<unsigned>(r[0])),
               __builtin_bit_cast(float, static_cast<unsigned>(r[1])));
}

__device__ __forceinline__ float sum_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, x), __builtin_bit_cast(unsigned, x),
                                                  false, false);
  return __builtin_bit_cast(float, static_cast<unsigned>(r[0])) + __builtin_bit_cast(float, static_cast<unsigned>(r[1]));
}

struct Fwd2Args {
  const _Float16* q;
  const _Float16* k;
  const _Float16* v;
  const void* mask;          // fp16 bias or uint8 keep-mask, keys contiguous
  int64_t m_sb, m_sh, m_sq;  // elements
  uint32_t m_bytes;          // extent of one (sequence, q head) of the mask
  int64_t q_sb, q_sh, q_ss;
  int64_t k_sb, k_sh, k_ss;
  int64_t v_sb, v_sh, v_ss;
  _Float16* out;
  float* lse;
  int B, Hq, Hkv, g, Sq, Skv, causal, qblocks;
  // Rows per query: 1, or (calls without a mask, Sq < 256) the g q heads of
  // a KV head, which then share each K / V tile; gp = g / pack.
  int pack, gp;
  // Key split (calls without a mask or causal flag whose blocks would not
  // fill the device): block sp attends keys sp * split_keys .. + split_keys
  // - 1 and writes its fp32 partial (O, row max, row sum) to part; a merge
  // pass combines them.  nsplit == 1: no split.
  int nsplit, split_keys;
  float* part;
  // sdpa_decode_short_kernel's key split: this call's arrival-flag value
  // (nonzero, a new one per call).
  uint32_t ticket;
  uint32_t n_items;
  int xcd_remap;
  float scale_log2;
};

// A wavefront's mask block for one step: its 32 queries x the step's 64 keys,
// rows padded by 16 bytes, staged in LDS by buffer loads like the K / V
// tiles (whole 1 KB loads; units past the block arrive as zeros in a spare
// tail).
template <int MK> struct MaskTile {
  static constexpr int kRowU = 0, kDataU = 0, kLoads = 0, kBytes = 0, kEsz = 1;
};
template <> struct MaskTile<kMaskF16> {  // 128 + 16 bytes per row
  static constexpr int kRowU = 9, kDataU = 8, kLoads = 5, kBytes = kLoads * 1024, kEsz = 2;
};
template <> struct MaskTile<kMaskBool> {  // 64 + 16 bytes per row
  static constexpr int kRowU = 5, kDataU = 4, kLoads = 3, kBytes = kLoads * 1024, kEsz = 1;
};

// PRESCALED (|scale log2 e| <= 1, so q * that never overflows fp16): Q is
// multiplied by scale log2 e once, and every step's scores leave the MFMA
// already as exponents: the first QK MFMA starts from a tile holding -m
// (the running max), so P = exp2(S) needs no per-score FMA.  Otherwise the
// scale's sign is folded into Q and its magnitude into the exponent's FMA.
// SLOTS: K / V slots in LDS.  Two: each step's tiles are loaded one step
// ahead, a barrier per step.  Four (calls without a mask whose blocks have
// fewer than 256 rows, e.g. decode, where one wavefront computes and the
// step waits on its loads): loads two steps ahead, a barrier per two steps.
// HALF (blocks of at most 128 rows without a mask, e.g. decode): wavefronts
// 2r and 2r + 1 share row tile r and take one 32-key half of every step
// each; the pair's partials are folded in LDS at the end.
template <int D, bool PRESCALED, int MK, int SLOTS = 2, bool HALF = false>
__global__ __launch_bounds__(kThreads2) void sdpa_fwd_lds_kernel(Fwd2Args a) {
  static_assert(SLOTS == 2 || (SLOTS == 4 && MK == kNoMask), "four slots leave no room for a mask");
  static_assert(!HALF || MK == kNoMask, "half steps serve calls without a mask");
  using L = Lds2<D>;
  using MT = MaskTile<MK>;
  constexpr int DK = D / 16;  // QK k-steps
  constexpr int DM = D / 32;  // O row tiles
  // Two K / V slots, then (masked calls) two mask blocks per wavefront.
  __shared__ __align__(16) _Float16 lds[SLOTS * L::kSlot + kWaves2 * MT::kBytes];

  // item = ((b * Hkv + kvh) * qblocks + (qblocks - 1 - qb)) * gp + gi: the
  // blocks of one (sequence, KV head) are consecutive, latest query block
  // (longest, under causal masking) first across its g q heads.
  // With pack > 1 a block's rows are (query, q head) pairs of one KV head,
  // row = query * pack + head in group.
  uint32_t item = blockIdx.x;
  if (a.xcd_remap) item = (item % 8) * (a.n_items / 8) + item / 8;
  const int pack = MK == kNoMask ? a.pack : 1;
  const int sp = MK == kNoMask ? static_cast<int>(item % a.nsplit) : 0;
  if (MK == kNoMask) item /= a.nsplit;
  const int gi = static_cast<int>(item % a.gp);
  uint32_t r = item / a.gp;
  const int qb = a.qblocks - 1 - static_cast<int>(r % a.qblocks);
  r /= a.qblocks;
  const int kvh = static_cast<int>(r % a.Hkv);
  const int b = static_cast<int>(r / a.Hkv);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64), lane = threadIdx.x % 64;
  __builtin_assume(wave >= 0 && wave < kWaves2);  // lets the compiler drop always-true load guards
  const int hw = HALF ? (wave & 1) : 0;  // HALF: the key half of each step
  const int qw0 = qb * kQB, q0 = qw0 + (HALF ? (wave >> 1) : wave) * kQW;  // rows
  const int col = lane & 31, half = lane >> 5;
  const int qrow = q0 + col;
  const int qi = pack == 1 ? qrow : qrow / pack;  // this lane's query
  // Block gi of the KV head holds q heads gi * pack .. gi * pack + pack - 1.
  const int h = kvh * a.g + gi * pack + (qrow - qi * pack);
  const bool q_ok = qi < a.Sq;
  // The wavefront's first and last query, and the block's last.
  const int q_lo = pack == 1 ? q0 : q0 / pack;
  const int q_hi = pack == 1 ? q0 + kQW - 1 : (q0 + kQW - 1) / pack;
  const int qb_hi = pack == 1 ? qw0 + kQB - 1 : (qw0 + kQB - 1) / pack;

  // Q^T operand: lane (query column, half) holds features 16ks + 8half .. +8.
  f16x8 qv[DK];
  {
    const _Float16* qp = a.q + b * a.q_sb + h * a.q_sh + static_cast<int64_t>(min(qi, a.Sq - 1)) * a.q_ss + 8 * half;
#pragma unroll
    for (int ks = 0; ks < DK; ++ks) {
      qv[ks] = q_ok ? *reinterpret_cast<const f16x8*>(qp + 16 * ks) : f16x8{};
      if constexpr (PRESCALED) {
#pragma unroll
        for (int e = 0; e < 8; ++e) qv[ks][e] = static_cast<_Float16>(static_cast<float>(qv[ks][e]) * a.scale_log2);
      } else if (a.scale_log2 < 0.f) {
        qv[ks] = -qv[ks];  // the scale's sign, exactly
      }
    }
    // Wait for Q here, outside the loop: otherwise the first MFMA of every
    // step also waits for the next tiles' loads, which are then in flight.
#pragma unroll
    for (int ks = 0; ks < DK; ++ks) asm volatile("" : : "v"(qv[ks]));
  }
  const _Float16* kbase = a.k + b * a.k_sb + kvh * a.k_sh;
  const _Float16* vbase = a.v + b * a.v_sb + kvh * a.v_sh;

  // Tiles move from L2 straight into LDS (buffer loads with the LDS flag):
  // lane l of a load writes the 16 bytes at M0 + 16 l, so load i of a tile
  // fills its 16-byte units 64 i .. 64 i + 63, padded rows included.  Lane
  // l of load i fetches the unit's source; pad units and K / V rows past Skv
  // get an offset past the buffer's range and are written as zeros.  Per-lane
  // offsets are fixed for the whole loop; the step only moves the base.
  constexpr int kUK = L::kRowK / 8, kUV = L::kRowV / 8;  // 16-byte units per padded row
  constexpr int kNK = kKT * kUK / 64, kNV = kKT * kUV / 64;  // loads per tile
  static_assert(kKT * kUK % 64 == 0 && kKT * kUV % 64 == 0, "tiles must be whole loads");
  constexpr int kJK = (kNK + kWaves2 - 1) / kWaves2, kJV = (kNV + kWaves2 - 1) / kWaves2;
  constexpr uint32_t kOob = 0x80000000u;  // past kBufRange
  uint32_t k_off[kJK], v_off[kJV];
#pragma unroll
  for (int j = 0; j < kJK; ++j) {
    const int u = 64 * (wave + kWaves2 * j) + lane, row = u / kUK, ch = u % kUK;
    const bool pad = ch == kUK - 1;
    k_off[j] = pad ? kOob : (static_cast<uint32_t>(row) * static_cast<uint32_t>(a.k_ss) + 8 * ch) * 2;
  }
#pragma unroll
  for (int j = 0; j < kJV; ++j) {
    const int u = 64 * (wave + kWaves2 * j) + lane, row = u / kUV, ch = u % kUV;
    const bool pad = ch >= D / 8;  // kRowV / 8 - D / 8 pad units per row
    v_off[j] = pad ? kOob : (static_cast<uint32_t>(row) * static_cast<uint32_t>(a.v_ss) + 8 * ch) * 2;
  }
  // K / V tiles load in sequence (K(0), K(1), ... and V(0), V(1), ...), so
  // each has a running cursor: the next tile's first row and the bytes from
  // it to the end of row Skv - 1.  Rows past Skv lie past the descriptor's
  // range and arrive as zeros without a per-lane test (no unit straddles
  // the end: a row's units end within its stride); with a key stride of 0
  // every row reads row 0's bytes, finite values the key test masks.
  const _Float16* k_cur = kbase + static_cast<int64_t>(sp) * a.split_keys * a.k_ss;
  const _Float16* v_cur = vbase + static_cast<int64_t>(sp) * a.split_keys * a.v_ss;
  const int64_t k_tile = static_cast<int64_t>(kKT) * a.k_ss, v_tile = static_cast<int64_t>(kKT) * a.v_ss;
  // Bytes left as 32-bit values: the head's whole span fits one descriptor
  // (< 2 GiB, checked by the host), so a count clamped to kBufRange at the
  // start still covers every valid row and no row past Skv.
  auto left0 = [&](int64_t ss) {
    if (ss == 0) return static_cast<int32_t>(kBufRange);
    const int64_t all = static_cast<int64_t>(a.Skv) * ss * 2;
    return static_cast<int32_t>(min(all, static_cast<int64_t>(kBufRange)) - static_cast<int64_t>(sp) * a.split_keys * ss * 2);
  };
  int32_t k_left = left0(a.k_ss), v_left = left0(a.v_ss);
  const int32_t k_step = static_cast<int32_t>(min(2 * k_tile, static_cast<int64_t>(kBufRange)));
  const int32_t v_step = static_cast<int32_t>(min(2 * v_tile, static_cast<int64_t>(kBufRange)));
  auto range_of = [](int32_t left) { return static_cast<uint32_t>(max(left, 0)); };
  // The next K tile into slot `slot`.
  auto dma_k = [&](int slot) {
    const Rsrc r = make_rsrc(k_cur, range_of(k_left));
#pragma unroll
    for (int j = 0; j < kJK; ++j)
      if (wave + kWaves2 * j < kNK) load_lds16(r, lds + slot * L::kSlot + 512 * (wave + kWaves2 * j), k_off[j]);
    k_cur += k_tile;
    k_left -= k_step;
  };
  // The next V tile into slot `slot` (rows past Skv as zeros, so that a
  // masked key's P = 0 never meets stale bits).
  auto dma_v = [&](int slot) {
    const Rsrc r = make_rsrc(v_cur, range_of(v_left));
#pragma unroll
    for (int j = 0; j < kJV; ++j)
      if (wave + kWaves2 * j < kNV)
        load_lds16(r, lds + slot * L::kSlot + L::kK + 512 * (wave + kWaves2 * j), v_off[j]);
    v_cur += v_tile;
    v_left -= v_step;
  };
  // The wavefront's mask block of keys kb .. kb + 63 into its slot `slot`:
  // rows past Sq and bytes past the (sequence, head) slice arrive as zeros.
  // Offsets are from the wavefront's first query row; the descriptor's range
  // ends with the (sequence, head) slice.
  uint32_t m_off[MT::kLoads > 0 ? MT::kLoads : 1];
  const char* mbase = nullptr;
  uint32_t m_left = 0;  // bytes of the slice from row q0, key 0
  if constexpr (MK != kNoMask) {
    const int64_t row0 = static_cast<int64_t>(min(q0, a.Sq - 1)) * a.m_sq * MT::kEsz;
    mbase = static_cast<const char*>(a.mask) + (b * a.m_sb + h * a.m_sh) * MT::kEsz + row0;
    m_left = a.m_bytes - static_cast<uint32_t>(row0);
#pragma unroll
    for (int j = 0; j < MT::kLoads; ++j) {
      const int u = 64 * j + lane, row = u / MT::kRowU, ch = u % MT::kRowU;
      const bool ok = row < kQW && ch < MT::kDataU && q0 + row < a.Sq;
      m_off[j] = ok ? static_cast<uint32_t>((row * a.m_sq) * MT::kEsz + 16 * ch) : kOob;
    }
  }
  auto mask_block = [&](int slot) { return lds + SLOTS * L::kSlot + (slot * kWaves2 + wave) * (MT::kBytes / 2); };
  auto dma_m = [&](int kb, int slot) {
    if constexpr (MK != kNoMask) {
      const uint32_t done = static_cast<uint32_t>(kb) * MT::kEsz;  // < Skv esz <= m_left
      const Rsrc r = make_rsrc(reinterpret_cast<const _Float16*>(mbase + done), m_left - done);
#pragma unroll
      for (int j = 0; j < MT::kLoads; ++j) load_lds16(r, mask_block(slot) + 512 * j, m_off[j]);
    }
  };
  // The loads must have landed before the barrier that publishes them.
  auto dma_wait = [] { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); };

  // This block's keys: kb0 .. key_end - 1 (the whole row unless split).
  const int kb0 = sp * a.split_keys;
  const int key_end = a.causal ? min(a.Skv, qb_hi + 1) : (a.nsplit > 1 ? min(a.Skv, kb0 + a.split_keys) : a.Skv);
  const int n_tiles = (key_end - kb0 + kKT - 1) / kKT;
  // Step t has work for this wavefront unless all its keys are masked
  // (causal: keys past the wavefront's last query).
  auto active = [&](int t) { return t < n_tiles && q_lo < a.Sq && (!a.causal || kb0 + t * kKT <= q_hi); };
  // Only steps crossing Skv or the causal diagonal need the key test.
  auto edge = [&](int t) { return kb0 + t * kKT + kKT > a.Skv || (a.causal && kb0 + t * kKT + kKT - 1 > q_lo); };
  // |scale| (its sign is folded into Q), kept above 0 so that masked scores
  // (-inf) stay -inf; a scale of 0 then gives the uniform weights it should.
  const float scale_abs = fmaxf(fabsf(a.scale_log2), 1e-30f);
  float m_run = -INFINITY, l_run = 0.f;
  // PRESCALED: scores are carried relative to m_use (m_run, or 0 while no
  // finite score has been seen); neg_m_tile holds -m_use in every row.
  float m_use = 0.f;
  f32x16 neg_m_tile = f32x16{};
  f32x16 o[DM];
#pragma unroll
  for (int dm = 0; dm < DM; ++dm) o[dm] = f32x16{};

  // S^T half mt (keys 32mt .. 32mt + 31 of the step) from the K tile at kt.
  auto qk = [&](const _Float16* kt, int mt) {
    const _Float16* krow = kt + (mt * 32 + key32_of(col)) * L::kRowK + 8 * half;
    f32x16 acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(*reinterpret_cast<const f16x8*>(krow), qv[0],
                                                        PRESCALED ? neg_m_tile : f32x16{}, 0, 0, 0);
#pragma unroll
    for (int ks = 1; ks < DK; ++ks) {
      const f16x8 ka = *reinterpret_cast<const f16x8*>(krow + 16 * ks);
      acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka, qv[ks], acc, 0, 0, 0);
    }
    return acc;
  };
  // Lane (query column, half) holds S^T rows 8i + 4half + v of each 32-key
  // half (register 4i + v).  Masked scores become -inf.
  const int key_last = a.causal ? min(a.Skv - 1, qi) : a.Skv - 1;  // this lane's last visible key
  auto mask_step = [&](int t, f32x16 (&s)[2]) {
    const int kl = key_last - (kb0 + t * kKT) - 8 * half;  // key32_of adds 8 per lane half
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int rr = 0; rr < 16; ++rr) {
        const int kr = mt * 32 + key32_of(8 * (rr >> 2) + (rr & 3));  // key - t kKT - 8 half
        s[mt][rr] = kr <= kl ? s[mt][rr] : -INFINITY;
      }
  };
  // The step's mask from the wavefront's block in LDS: registers 4i + v of
  // half mt are keys 32 mt + 16 (i / 2) + 8 half + 4 (i % 2) + v of query
  // col, four consecutive keys per read.  A bias is added in the scores'
  // units (PRESCALED: log2 units, else divided by |scale|), a keep-mask
  // sends dropped scores to -inf.
  const float bias_mul = PRESCALED ? kLog2e : kLog2e / scale_abs;
  auto apply_mask = [&](int t, f32x16 (&s)[2]) {
    if constexpr (MK != kNoMask) {
      const char* row = reinterpret_cast<const char*>(mask_block(t & 1)) + col * (16 * MT::kRowU);
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int k4 = 32 * mt + 16 * (i >> 1) + 8 * half + 4 * (i & 1);
          if constexpr (MK == kMaskF16) {
            const f16x4 m4 = *reinterpret_cast<const f16x4*>(row + 2 * k4);
#pragma unroll
            for (int v = 0; v < 4; ++v) s[mt][4 * i + v] = __builtin_fmaf(static_cast<float>(m4[v]), bias_mul, s[mt][4 * i + v]);
          } else {
            const uint32_t m4 = *reinterpret_cast<const uint32_t*>(row + k4);
#pragma unroll
            for (int v = 0; v < 4; ++v)
              s[mt][4 * i + v] = ((m4 >> (8 * v)) & 0xffu) != 0 ? s[mt][4 * i + v] : -INFINITY;
          }
        }
    }
  };
  // The running max (log2 domain) moves only when a score of the step
  // exceeds it by more than 2^8, so P <= 256 (fine in fp16) and most steps
  // skip the rescale of O; O / l is exact whatever max is used.
  // PRESCALED: s holds exponents relative to m_use, and so does `ahead`
  // (the first half of the next step's scores, computed before this
  // update); a move of m_use shifts both, and the tile.
  // The step's row max in the units of m_run.
  auto row_max = [&](const f32x16 (&s)[2]) {
    float mx = -INFINITY;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int rr = 0; rr < 16; ++rr) mx = fmaxf(mx, s[mt][rr]);
    return PRESCALED ? max_xor32(mx) + m_use : max_xor32(mx) * scale_abs;
  };
  // ahead2: with a mask, the second half of S(t+1) is complete too.
  auto update_max = [&](f32x16 (&s)[2], f32x16& ahead, f32x16* ahead2, float mx) {
    if (__builtin_amdgcn_ballot_w64(mx > m_run + 8.f) != 0) {
      const float m_new = fmaxf(m_run, mx);
      const float alpha = m_new == -INFINITY ? 1.f : fast_exp2(m_run - m_new);
      l_run *= alpha;
#pragma unroll
      for (int dm = 0; dm < DM; ++dm) o[dm] *= alpha;
      m_run = m_new;
      if constexpr (PRESCALED) {
        const float m_use_new = m_new == -INFINITY ? m_use : m_new;  // lanes still without a score keep 0
        const float d = m_use_new - m_use;
        m_use = m_use_new;
#pragma unroll
        for (int rr = 0; rr < 16; ++rr) {
          s[0][rr] -= d;
          s[1][rr] -= d;
          ahead[rr] -= d;
          if (ahead2) (*ahead2)[rr] -= d;
          neg_m_tile[rr] = -m_use;
        }
      }
    }
  };
  // P (fp16) of half mt; the row sum adds the same fp16 values the PV
  // product uses.
  auto softmax_half = [&](const f32x16& s, float neg_m, f16x8 (&pb)[2]) {
    float psum = 0.f;
#pragma unroll
    for (int rr = 0; rr < 16; ++rr) {
      const float p = fast_exp2(PRESCALED ? s[rr] : __builtin_fmaf(s[rr], scale_abs, neg_m));  // masked: 0
      const int i = rr >> 2;
      pb[i >> 1][(i & 1) * 4 + (rr & 3)] = static_cast<_Float16>(p);
    }
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        psum = __builtin_amdgcn_fdot2(f16x2{pb[j][2 * e], pb[j][2 * e + 1]}, f16x2{1, 1}, psum, false);
    l_run += psum;
  };
  // P (fp16) of S^T registers 8j .. 8j + 7 of a half: the B operand of the
  // half's PV k-step j.  Returns the sum of the same fp16 values.
  auto softmax_q = [&](const f32x16& s, int j, float neg_m, f16x8& pb) -> float {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int rr = 8 * j + e;
      pb[e] = static_cast<_Float16>(fast_exp2(PRESCALED ? s[rr] : __builtin_fmaf(s[rr], scale_abs, neg_m)));
    }
    float psum = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      psum = __builtin_amdgcn_fdot2(f16x2{pb[2 * e], pb[2 * e + 1]}, f16x2{1, 1}, psum, false);
    return psum;
  };
  // A move of the running max to m_new = max(m_run, mx): O and l rescaled;
  // PRESCALED: S(t) and S(t+1) shifted with m_use, and the -m tile.
  auto rescale = [&](f32x16 (&s)[2], f32x16 (&ahead)[2], float mx) {
    const float m_new = fmaxf(m_run, mx);
    const float alpha = m_new == -INFINITY ? 1.f : fast_exp2(m_run - m_new);
    l_run *= alpha;
#pragma unroll
    for (int dm = 0; dm < DM; ++dm) o[dm] *= alpha;
    m_run = m_new;
    if constexpr (PRESCALED) {
      const float m_use_new = m_new == -INFINITY ? m_use : m_new;  // lanes still without a score keep 0
      const float d = m_use_new - m_use;
      m_use = m_use_new;
#pragma unroll
      for (int rr = 0; rr < 16; ++rr) {
        s[0][rr] -= d;
        s[1][rr] -= d;
        ahead[0][rr] -= d;
        ahead[1][rr] -= d;
        neg_m_tile[rr] = -m_use;
      }
    }
  };
  // The 2 DK + 4 DM MFMAs of a step in issue order, each with its LDS operand
  // fragment: 0 .. 2DK-1 the K operands of S(t+1) (half i / DK, k-step
  // i % DK), then the V^T operands of O^T += V^T P^T (two transposed reads
  // each), k-steps (half, j) = c / 2, c % 2 for c = (i - 2DK) / DM, O row tile
  // dm = (i - 2DK) % DM.
  // Each fragment is read kPrefetch MFMAs before its use: with reads issued
  // only just ahead, every MFMA waited out an LDS read.
  constexpr int kNF = 2 * DK + 4 * DM;
  // LDS element offsets of the Vt rows of the step's four 16-key columns,
  // hidden from the compiler: otherwise it pairs reads whose addresses are
  // 32 bytes apart and issues the earlier one late, beside the later one.
  uint32_t vtr;  // this lane's V tile element for the transposed reads, in the step's slot
  // Within each 16 lanes, lane s reads V[key 8 half + s / 4][d 16 (lane / 16 % 2) + 4 (s % 4)
  // .. + 3]; ds_read_b64_tr_b16 hands lane j of the 16 the four keys of column d + j.
  const uint32_t vtr_lane = static_cast<uint32_t>((8 * half + ((lane & 15) >> 2)) * L::kRowV +
                                                  16 * ((lane >> 4) & 1) + 4 * (lane & 3));
  auto tr4 = [&](uint32_t e) { return tr_read4(lds + e); };
  auto frag = [&](const _Float16* k1, int i) -> f16x8 {
    if (i < 2 * DK)  // the two halves' chains alternate: half i % 2, k-step i / 2
      return *reinterpret_cast<const f16x8*>(k1 + ((i % 2) * 32 + key32_of(col)) * L::kRowK + 8 * half +
                                             16 * (i / 2));
    i -= 2 * DK;
    // keys 16 (i / DM) + 8 half .. + 7 of feature 32 (i % DM) + col
    const uint32_t e = vtr + (16 * (i / DM)) * L::kRowV + 32 * (i % DM);
    const v4i16 lo = tr4(e), hi = tr4(e + 4 * L::kRowV);
    return __builtin_bit_cast(f16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  };
  // Keeps a region's operand reads interleaved one per MFMA (n of each).
  // Keeps a region's operand reads interleaved with its MFMAs i0 .. i1 - 1:
  // each MFMA, then the reads of the fragment kPrefetch ahead (two for a V
  // fragment).
  auto interleave_reads = [](int i0, int i1) {
    for (int i = i0; i < i1; ++i) {
      const int f = i + kPrefetch;
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
      if (f < 2 * DK)
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read (K)
      else if (f < kNF)
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // two (V, transposed)
    }
  };

  // Interleaves MFMAs i0 .. i1 - 1 with the rest of their region: after
  // each MFMA the reads of the fragment kPrefetch ahead, then te (after the
  // region's even MFMAs) or to (odd) transcendental and nv other VALU
  // instructions.
  auto interleave_mix = [](int i0, int i1, int te, int to, int nv) {
    for (int i = i0; i < i1; ++i) {
      const int f = i + kPrefetch;
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
      if (f < 2 * DK)
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read (K)
      else if (f < kNF)
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // two (V, transposed)
      const int nt = (i - i0) % 2 == 0 ? te : to;
      if (nt == 1) __builtin_amdgcn_sched_group_barrier(0x400, 1, 0);  // transcendental
      if (nt == 2) __builtin_amdgcn_sched_group_barrier(0x400, 2, 0);
      if (nv == 1) __builtin_amdgcn_sched_group_barrier(0x002, 1, 0);  // other VALU
      if (nv == 2) __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
      if (nv == 3) __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
      if (nv == 4) __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
    }
  };

  // HALF: the wavefront's S tile (keys 32 hw .. 32 hw + 31 of the step)
  // lives in slot 0 of cur / nxt; its fragments are K half hw (vi < DK) and
  // the V^T operands of keys 32 hw .. + 31 (vi - DK = j DM + dm).
  constexpr int kNFH = DK + 2 * DM;
  auto frag_h = [&](const _Float16* k1, int vi) -> f16x8 {
    if (vi < DK)
      return *reinterpret_cast<const f16x8*>(k1 + (hw * 32 + key32_of(col)) * L::kRowK + 8 * half + 16 * vi);
    const int i = vi - DK;
    const uint32_t e = vtr + (16 * (2 * hw + i / DM)) * L::kRowV + 32 * (i % DM);
    const v4i16 lo = tr4(e), hi = tr4(e + 4 * L::kRowV);
    return __builtin_bit_cast(f16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  };
  auto interleave_h = [](int i0, int i1) {
    for (int i = i0; i < i1; ++i) {
      const int f = i + kPrefetch;
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if (f < DK)
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      else if (f < kNFH)
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
  };
  auto step_h = [&](int t, f32x16& cur, f32x16& nxt) {
    const _Float16* k1 = lds + ((t + 1) % SLOTS) * L::kSlot;
    if constexpr (SLOTS == 2) {
      if (t + 2 < n_tiles) dma_k(t & 1);
      if (t + 1 < n_tiles) dma_v((t + 1) & 1);
    } else if ((t & 1) == 0) {
      if (t + 3 < n_tiles) dma_k((t + 3) % 4);
      if (t + 4 < n_tiles) dma_k(t % 4);
      if (t + 2 < n_tiles) dma_v((t + 2) % 4);
      if (t + 3 < n_tiles) dma_v((t + 3) % 4);
    }
    if (active(t)) {
      vtr = static_cast<uint32_t>((t % SLOTS) * L::kSlot + L::kK) + vtr_lane;
      asm volatile("" : "+v"(vtr));
      f16x8 fr[kNFH];
#pragma unroll
      for (int i = 0; i < kPrefetch; ++i) fr[i] = frag_h(k1, i);
      auto mfma = [&](int i, const f16x8& b, f32x16& acc) {
        acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(fr[i], b, acc, 0, 0, 0);
        if (i + kPrefetch < kNFH) fr[i + kPrefetch] = frag_h(k1, i + kPrefetch);
      };
      if (edge(t)) {  // the key test on this half
        const int kl = key_last - (kb0 + t * kKT) - 32 * hw - 8 * half;
#pragma unroll
        for (int rr = 0; rr < 16; ++rr)
          cur[rr] = key32_of(8 * (rr >> 2) + (rr & 3)) <= kl ? cur[rr] : -INFINITY;
      }
      nxt = PRESCALED ? neg_m_tile : f32x16{};
#pragma unroll
      for (int ks = 0; ks < DK; ++ks) mfma(ks, qv[ks], nxt);
      interleave_h(0, DK);
      float mx = -INFINITY;
#pragma unroll
      for (int rr = 0; rr < 16; ++rr) mx = fmaxf(mx, cur[rr]);
      mx = PRESCALED ? max_xor32(mx) + m_use : max_xor32(mx) * scale_abs;
      if (__builtin_amdgcn_ballot_w64(mx > m_run + 8.f) != 0) {
        const float m_new = fmaxf(m_run, mx);
        const float alpha = m_new == -INFINITY ? 1.f : fast_exp2(m_run - m_new);
        l_run *= alpha;
#pragma unroll
        for (int dm = 0; dm < DM; ++dm) o[dm] *= alpha;
        m_run = m_new;
        if constexpr (PRESCALED) {
          const float m_use_new = m_new == -INFINITY ? m_use : m_new;
          const float d = m_use_new - m_use;
          m_use = m_use_new;
#pragma unroll
          for (int rr = 0; rr < 16; ++rr) {
            cur[rr] -= d;
            nxt[rr] -= d;
            neg_m_tile[rr] = -m_use;
          }
        }
      }
      const float neg_m = m_run == -INFINITY ? 0.f : -m_run;
      f16x8 p[2];
      softmax_half(cur, neg_m, p);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int dm = 0; dm < DM; ++dm) mfma(DK + j * DM + dm, p[j], o[dm]);
      interleave_h(DK, kNFH);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (SLOTS == 2 || (t & 1)) {
      dma_wait();
      __syncthreads();
    }
  };

  // Step t: LDS holds K(t+1) in slot (t+1)&1 and V(t) in slot t&1, cur
  // holds S(t); the step loads K(t+2) and V(t+1) and leaves S(t+1) in nxt.
  // The MFMAs of S(t+1) and of step t's P V overlap step t's softmax: each
  // scheduling region pairs one MFMA group with one VALU group.  At a
  // wavefront's last active step S(t+1) reads a stale K slot and is never
  // used.
  auto step = [&](int t, f32x16 (&cur)[2], f32x16 (&nxt)[2]) {
    const _Float16* k1 = lds + ((t + 1) % SLOTS) * L::kSlot;
    if constexpr (SLOTS == 2) {
      // K(t+2) replaces K(t) (read during step t-1), V(t+1) replaces
      // V(t-1); both land during this step's math.
      if (t + 2 < n_tiles) dma_k(t & 1);
      if (t + 1 < n_tiles) dma_v((t + 1) & 1);
      if (t + 1 < n_tiles) dma_m(kb0 + (t + 1) * kKT, (t + 1) & 1);
    } else if ((t & 1) == 0) {
      // Steps t, t + 1 read K(t+1), K(t+2), V(t), V(t+1) (slot = tile % 4);
      // K(t+3), K(t+4), V(t+2), V(t+3) fill the other four slot halves,
      // whose last readers were steps t - 2 and t - 1, and land by the
      // barrier after step t + 1.
      if (t + 3 < n_tiles) dma_k((t + 3) % 4);
      if (t + 4 < n_tiles) dma_k(t % 4);
      if (t + 2 < n_tiles) dma_v((t + 2) % 4);
      if (t + 3 < n_tiles) dma_v((t + 3) % 4);
    }
    if (active(t)) {
      vtr = static_cast<uint32_t>((t % SLOTS) * L::kSlot + L::kK) + vtr_lane;
      asm volatile("" : "+v"(vtr));
      f16x8 fr[kNF];
#pragma unroll
      for (int i = 0; i < kPrefetch; ++i) fr[i] = frag(k1, i);
      // MFMA i, then the read of fragment i + kPrefetch.
      auto mfma = [&](int i, const f16x8& b, f32x16& acc) {
        acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(fr[i], b, acc, 0, 0, 0);
        if (i + kPrefetch < kNF) fr[i + kPrefetch] = frag(k1, i + kPrefetch);
      };
      if constexpr (MK == kNoMask) {
        if (edge(t)) mask_step(t, cur);
        // Region A: the 2 DK MFMAs of S(t+1) beside P(t) of half 0, computed
        // against the running max as it stands.  The max matters only as a
        // bound: while every lane's sum of a half's P stays <= 2^8, so does
        // every P, and nothing moves.  Otherwise (and at a wavefront's first
        // scores) the branch below takes the row max, rescales and redoes
        // P -- so the common step computes no max at all.
        nxt[0] = PRESCALED ? neg_m_tile : f32x16{};
        nxt[1] = PRESCALED ? neg_m_tile : f32x16{};
#pragma unroll
        for (int ks = 0; ks < DK; ++ks) {
          mfma(2 * ks, qv[ks], nxt[0]);
          mfma(2 * ks + 1, qv[ks], nxt[1]);
        }
        // P(t) of half 0 goes beside region A and P(t) of half 1 beside
        // the PV MFMAs of half 0 (region B1), so both regions carry VALU
        // work; each half has its own bound check.
        f16x8 p0[2], p1[2];
        float neg_m = m_run == -INFINITY ? 0.f : -m_run;
        float ps = softmax_q(cur[0], 0, neg_m, p0[0]) + softmax_q(cur[0], 1, neg_m, p0[1]);
        asm volatile("" : "+v"(p0[0]), "+v"(p0[1]), "+v"(ps));
        interleave_mix(0, 2 * DK, 1, 1, 1);
        if (__builtin_amdgcn_ballot_w64(!(ps <= 256.f) || m_run == -INFINITY) != 0) {
          rescale(cur, nxt, row_max(cur));
          neg_m = m_run == -INFINITY ? 0.f : -m_run;
          ps = softmax_q(cur[0], 0, neg_m, p0[0]) + softmax_q(cur[0], 1, neg_m, p0[1]);
        }
        l_run += ps;
        // Region B1: the PV MFMAs of half 0 beside P(t) of half 1.
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int dm = 0; dm < DM; ++dm) mfma(2 * DK + j * DM + dm, p0[j], o[dm]);
        ps = softmax_q(cur[1], 0, neg_m, p1[0]) + softmax_q(cur[1], 1, neg_m, p1[1]);
        asm volatile("" : "+v"(p1[0]), "+v"(p1[1]), "+v"(ps));
        interleave_mix(2 * DK, 2 * DK + 2 * DM, 2, 2, 2);
        if (__builtin_amdgcn_ballot_w64(!(ps <= 256.f)) != 0) {
          // Half 1 holds a score above the bound: move the max to half 1's
          // row max.  O (half 0's product included) and l are relative to
          // the old max and scale with it.
          float mx = -INFINITY;
#pragma unroll
          for (int rr = 0; rr < 16; ++rr) mx = fmaxf(mx, cur[1][rr]);
          rescale(cur, nxt, PRESCALED ? max_xor32(mx) + m_use : max_xor32(mx) * scale_abs);
          neg_m = m_run == -INFINITY ? 0.f : -m_run;
          ps = softmax_q(cur[1], 0, neg_m, p1[0]) + softmax_q(cur[1], 1, neg_m, p1[1]);
        }
        l_run += ps;
        // Region B2: the PV MFMAs of half 1.
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int dm = 0; dm < DM; ++dm) mfma(2 * DK + 2 * DM + j * DM + dm, p1[j], o[dm]);
        interleave_reads(2 * DK + 2 * DM, kNF);
      } else {

        // A mask can leave a step nothing to add: every score of the
        // wavefront's block -inf or more than 32 below its row's running
        // max, so every P rounds to 0 in fp16.  Such a step computes only
        // S(t+1); S(t+1) is therefore computed whole before the softmax.
        apply_mask(t, cur);
        if (edge(t)) mask_step(t, cur);
        const float mx = row_max(cur);
        const bool live = __builtin_amdgcn_ballot_w64(mx > -INFINITY && mx >= m_run - 32.f) != 0;
        nxt[0] = PRESCALED ? neg_m_tile : f32x16{};
        nxt[1] = PRESCALED ? neg_m_tile : f32x16{};
#pragma unroll
        for (int ks = 0; ks < DK; ++ks) {
          mfma(2 * ks, qv[ks], nxt[0]);
          mfma(2 * ks + 1, qv[ks], nxt[1]);
        }
        interleave_reads(0, 2 * DK);
        if (live) {
          update_max(cur, nxt[0], &nxt[1], mx);
          const float neg_m = m_run == -INFINITY ? 0.f : -m_run;
          f16x8 p0[2], p1[2];
          softmax_half(cur[0], neg_m, p0);
#pragma unroll
          for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int dm = 0; dm < DM; ++dm) mfma(2 * DK + j * DM + dm, p0[j], o[dm]);
          softmax_half(cur[1], neg_m, p1);
          interleave_reads(2 * DK, 2 * DK + 2 * DM);
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int dm = 0; dm < DM; ++dm) mfma(2 * DK + 2 * DM + j * DM + dm, p1[j], o[dm]);
        }
      }
    }
    if (SLOTS == 2 || (t & 1)) {
      dma_wait();
      __syncthreads();
    }
  };

  // Prologue: K(0), V(0) in slot 0 and K(1) in slot 1 (four slots: also
  // V(1) and K(2)), then S(0).  A step
  // writes nxt only when it is active, and a step is active only if the one
  // before it is, so S is never read unwritten.
  f32x16 sa[2], sb[2];
  if (n_tiles > 0) {
    dma_k(0);
    dma_v(0);
    dma_m(kb0, 0);
  }
  if (n_tiles > 1) dma_k(1);
  if constexpr (SLOTS == 4) {
    if (n_tiles > 1) dma_v(1);
    if (n_tiles > 2) dma_k(2);
  }
  dma_wait();
  __syncthreads();
  if (active(0)) {
    if constexpr (HALF) {
      sa[0] = qk(lds, hw);
    } else {
      sa[0] = qk(lds, 0);
      sa[1] = qk(lds, 1);
    }
  }
  __syncthreads();  // step 0 overwrites K(0)
  // Two steps per iteration, S(t) alternating between sa and sb.
  for (int t = 0; t < n_tiles; t += 2) {
    if constexpr (HALF) {
      step_h(t, sa[0], sb[0]);
      if (t + 1 < n_tiles) step_h(t + 1, sb[0], sa[0]);
    } else {
      step(t, sa, sb);
      if (t + 1 < n_tiles) step(t + 1, sb, sa);
    }
  }
  if constexpr (HALF) {
    // Fold each pair: wavefront 2r + 1 leaves O, m, l (per lane) in LDS,
    // 2r weights both by exp2(m - max) (a half that saw no key weighs 0).
    dma_wait();
    __syncthreads();  // every wavefront is done with the tiles
    constexpr int kRec = DM * 16 + 2;
    float* rec = reinterpret_cast<float*>(lds) + ((wave >> 1) * 64 + lane) * kRec;
    if (hw == 1) {
#pragma unroll
      for (int dm = 0; dm < DM; ++dm)
#pragma unroll
        for (int k = 0; k < 16; ++k) rec[dm * 16 + k] = o[dm][k];
      rec[DM * 16] = m_run;
      rec[DM * 16 + 1] = l_run;
    }
    __syncthreads();
    if (hw == 1) return;
    const float m1 = rec[DM * 16], l1 = rec[DM * 16 + 1];
    const float M = fmaxf(m_run, m1);
    const float w0 = m_run == -INFINITY ? 0.f : fast_exp2(m_run - M);
    const float w1 = m1 == -INFINITY ? 0.f : fast_exp2(m1 - M);
#pragma unroll
    for (int dm = 0; dm < DM; ++dm)
#pragma unroll
      for (int k = 0; k < 16; ++k) o[dm][k] = o[dm][k] * w0 + rec[dm * 16 + k] * w1;
    l_run = l_run * w0 + l1 * w1;
    m_run = M;
  }

  const float l = sum_xor32(l_run);
  if (!q_ok) return;
  if (MK == kNoMask && a.nsplit > 1) {
    // The partial: O unnormalised (relative to m_run), then m_run and l.
    const int64_t prow = ((static_cast<int64_t>(b) * a.Hq + h) * a.Sq + qi) * a.nsplit + sp;
    float* po = a.part + prow * D;
#pragma unroll
    for (int dm = 0; dm < DM; ++dm)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        *reinterpret_cast<f32x4*>(po + 32 * dm + 8 * i + 4 * half) =
            f32x4{o[dm][4 * i], o[dm][4 * i + 1], o[dm][4 * i + 2], o[dm][4 * i + 3]};
    if (half == 0) {
      float* pml = a.part + static_cast<int64_t>(a.B) * a.Hq * a.Sq * a.nsplit * D + 2 * prow;
      pml[0] = m_run;
      pml[1] = l;
    }
    return;
  }
  _Float16* op = a.out + ((static_cast<int64_t>(b) * a.Sq + qi) * a.Hq + h) * D;
  const float inv = l > 0.f ? 1.f / l : 0.f;
  // Lane (query column, half) holds O^T rows d = 32dm + 8i + 4half + v.
#pragma unroll
  for (int dm = 0; dm < DM; ++dm)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f16x4 rv;
#pragma unroll
      for (int v = 0; v < 4; ++v) rv[v] = static_cast<_Float16>(o[dm][4 * i + v] * inv);
      *reinterpret_cast<f16x4*>(op + 32 * dm + 8 * i + 4 * half) = rv;
    }
  if (a.lse && half == 0)
    a.lse[(static_cast<int64_t>(b) * a.Hq + h) * a.Sq + qi] = l > 0.f ? (m_run + log2f(l)) * kLn2 : -INFINITY;
}

// ---- 4. short decode: a block's keys all in flight at once ----------------
//
// Calls without a mask or causal flag whose block holds one row tile (the g
// q heads of a KV head times Sq <= 32 rows) and at most kWaves2 * KW keys
// (KW = 64 keys at D = 64, 32 at D = 128): wavefront w loads keys
// kb + w KW .. + KW - 1 of K and V into its own LDS slice, all loads issued
// at kernel start, and computes its partial of the rows over them (S^T =
// K Q^T, softmax, O^T = V^T P^T as in sdpa_fwd_lds_kernel, the V^T operands
// through transposing LDS reads).  The W partials are then folded in LDS:
// the call is one round of loads and one kernel.  Longer key runs are split
// across blocks, which merge inside the kernel (below).  W = 8 wavefronts,
// or 4 when a split needs at most half the device's compute units at 8: the
// blocks then use every unit, each loading half the keys.
template <int D>
struct ShortLds {
  static constexpr int kKW = D == 64 ? 64 : 32;          // keys per wavefront
  static constexpr int kRowK = D + kPadH;                // K row, halves (padded)
  static constexpr int kUK = kRowK / 8;                  // 16-byte units per K row
  static constexpr int kNK = (kKW * kUK + 63) / 64;      // loads per K slice
  static constexpr int kNV = kKW * D / 8 / 64;           // loads per V slice (rows of D halves)
  static constexpr int kSliceB = (kNK + kNV) * 1024;     // bytes per wavefront
  static constexpr int kFoldF = D / 2 + 4;               // per-lane record of a partial: O^T, m, l (16-byte aligned)
  static_assert(kKW * D / 8 % 64 == 0, "V slices must be whole loads");
  static_assert(64 * kFoldF * 4 <= kSliceB, "a wavefront's fold records fit its own slice");
};

template <int D, bool PRESCALED, int W>
__global__ __launch_bounds__(W * 64) void sdpa_decode_short_kernel(Fwd2Args a) {
  using L = ShortLds<D>;
  constexpr int DK = D / 16, DM = D / 32;
  constexpr int KW = L::kKW, MT = KW / 32;  // 32-key S^T tiles per wavefront
  constexpr int NT = W * 64;                // threads
  // W slices; a four-wavefront block asks for more than half a compute
  // unit's 160 KiB, so that no unit runs two blocks while another idles.
  constexpr int kLdsB = W * L::kSliceB > 82 * 1024 ? W * L::kSliceB : 82 * 1024;
  __shared__ __align__(16) _Float16 lds[kLdsB / 2];

  // item = ((b * Hkv + kvh) * gp + gi) * nsplit + sp (one query block).
  uint32_t item = blockIdx.x;
  if (a.xcd_remap) item = (item % 8) * (a.n_items / 8) + item / 8;
  const int sp = static_cast<int>(item % a.nsplit);
  item /= a.nsplit;
  const int gi = static_cast<int>(item % a.gp);
  const uint32_t r = item / a.gp;
  const int kvh = static_cast<int>(r % a.Hkv);
  const int b = static_cast<int>(r / a.Hkv);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64), lane = threadIdx.x % 64;
  __builtin_assume(wave >= 0 && wave < W);
  const int col = lane & 31, half = lane >> 5;
  const int pack = a.pack;
  const int qi = col / pack;  // this lane's row: query qi, q head h
  const int h = kvh * a.g + gi * pack + (col - qi * pack);
  const bool q_ok = qi < a.Sq;

  // This wavefront's keys: kw .. kw + KW - 1, those below key_end visible.
  const int kb0 = sp * a.split_keys;
  const int key_end = a.nsplit > 1 ? min(a.Skv, kb0 + a.split_keys) : a.Skv;
  const int kw = kb0 + wave * KW;
  const int rows_here = min(key_end - kw, KW);  // <= 0: no key for this wavefront
  // Q^T operand: lane (row, half) holds features 16ks + 8half .. +8; loaded
  // first, so that scaling it waits for Q alone.
  f16x8 qv[DK];
  {
    const _Float16* qp = a.q + b * a.q_sb + h * a.q_sh + static_cast<int64_t>(min(qi, a.Sq - 1)) * a.q_ss + 8 * half;
#pragma unroll
    for (int ks = 0; ks < DK; ++ks) qv[ks] = q_ok ? *reinterpret_cast<const f16x8*>(qp + 16 * ks) : f16x8{};
  }
  _Float16* slice = lds + wave * (L::kSliceB / 2);
  constexpr uint32_t kOob = 0x80000000u;
  if (rows_here > 0) {
    const Rsrc rk = make_rsrc(a.k + b * a.k_sb + kvh * a.k_sh + static_cast<int64_t>(kw) * a.k_ss, kBufRange);
    const Rsrc rv = make_rsrc(a.v + b * a.v_sb + kvh * a.v_sh + static_cast<int64_t>(kw) * a.v_ss, kBufRange);
#pragma unroll
    for (int j = 0; j < L::kNK; ++j) {
      const int u = 64 * j + lane, row = u / L::kUK, ch = u % L::kUK;
      const bool ok = row < rows_here && ch < D / 8;  // pads, rows past the keys or the slice: zeros
      load_lds16(rk, slice + 512 * j,
                 ok ? (static_cast<uint32_t>(row) * static_cast<uint32_t>(a.k_ss) + 8 * ch) * 2 : kOob);
    }
#pragma unroll
    for (int j = 0; j < L::kNV; ++j) {
      const int u = 64 * j + lane, row = u / (D / 8), ch = u % (D / 8);
      load_lds16(rv, slice + 512 * (L::kNK + j),
                 row < rows_here ? (static_cast<uint32_t>(row) * static_cast<uint32_t>(a.v_ss) + 8 * ch) * 2 : kOob);
    }
  }
#pragma unroll
  for (int ks = 0; ks < DK; ++ks) {
    if constexpr (PRESCALED) {
#pragma unroll
      for (int e = 0; e < 8; ++e) qv[ks][e] = static_cast<_Float16>(static_cast<float>(qv[ks][e]) * a.scale_log2);
    } else if (a.scale_log2 < 0.f) {
      qv[ks] = -qv[ks];
    }
  }
  const float scale_abs = fmaxf(fabsf(a.scale_log2), 1e-30f);
  // The wavefront's own slice: its loads landing is all it waits for.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  float m = -INFINITY, l = 0.f;  // m: the rows' max over the slice (log2 units)
  f32x16 o[DM];
#pragma unroll
  for (int dm = 0; dm < DM; ++dm) o[dm] = f32x16{};
  if (rows_here > 0) {
    // S^T tile mt: keys 32mt .. 32mt + 31 of the slice; lane (row, half)
    // holds keys key32_of(8i + 4half + v) in register 4i + v.
    f32x16 s[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const _Float16* krow = slice + (mt * 32 + key32_of(col)) * L::kRowK + 8 * half;
      s[mt] = f32x16{};
#pragma unroll
      for (int ks = 0; ks < DK; ++ks)
        s[mt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(*reinterpret_cast<const f16x8*>(krow + 16 * ks), qv[ks], s[mt],
                                                       0, 0, 0);
    }
    // Keys past the run (and past Skv) are masked; scores in log2 units.
    const int kl = key_end - 1 - kw - 8 * half;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int rr = 0; rr < 16; ++rr) {
        const int kr = mt * 32 + key32_of(8 * (rr >> 2) + (rr & 3));
        const float x = PRESCALED ? s[mt][rr] : s[mt][rr] * scale_abs;
        s[mt][rr] = kr <= kl ? x : -INFINITY;
      }
    float mx = -INFINITY;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int rr = 0; rr < 16; ++rr) mx = fmaxf(mx, s[mt][rr]);
    m = max_xor32(mx);  // the row's max over both lane halves (finite: key kw is visible)
    // P (fp16) and its row sum over the same fp16 values; pb[mt][j] is the
    // PV operand of keys 32mt + 16j + 8half .. + 7.
    f16x8 pb[MT][2];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
#pragma unroll
        for (int e = 0; e < 8; ++e) pb[mt][j][e] = static_cast<_Float16>(fast_exp2(s[mt][8 * j + e] - m));
#pragma unroll
        for (int e = 0; e < 4; ++e)
          l = __builtin_amdgcn_fdot2(f16x2{pb[mt][j][2 * e], pb[mt][j][2 * e + 1]}, f16x2{1, 1}, l, false);
      }
    // O^T += V^T P^T: V^T operands by transposing reads of the V slice (rows
    // of D halves).
    const uint32_t vtr = static_cast<uint32_t>(wave * (L::kSliceB / 2) + L::kNK * 512) +
                         static_cast<uint32_t>((8 * half + ((lane & 15) >> 2)) * D + 16 * ((lane >> 4) & 1) +
                                               4 * (lane & 3));
#pragma unroll
    for (int c = 0; c < KW / 16; ++c)
#pragma unroll
      for (int dm = 0; dm < DM; ++dm) {
        const uint32_t e = vtr + 16 * c * D + 32 * dm;
        const v4i16 lo = tr_read4(lds + e), hi = tr_read4(lds + e + 4 * D);
        const f16x8 va = __builtin_bit_cast(f16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
        o[dm] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pb[c >> 1][c & 1], o[dm], 0, 0, 0);
      }
  }

  // Fold: every wavefront's partial (O^T relative to m, then m and l) to
  // LDS, one 16-byte aligned record per lane, over its own slice -- free once
  // its P.V operands are read, so no barrier comes before the records.
  // Lanes of padding rows (qi >= Sq: a decode tile holds g of its 32 rows)
  // write nothing.
  constexpr int kF = L::kFoldF;
  auto rec_of = [&](int w, int ln) { return reinterpret_cast<float*>(lds + w * (L::kSliceB / 2)) + ln * kF; };
  if (q_ok) {
    float* mine = rec_of(wave, lane);
#pragma unroll
    for (int dm = 0; dm < DM; ++dm)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        *reinterpret_cast<f32x4*>(mine + dm * 16 + 4 * i) =
            f32x4{o[dm][4 * i], o[dm][4 * i + 1], o[dm][4 * i + 2], o[dm][4 * i + 3]};
    *reinterpret_cast<f32x2*>(mine + D / 2) = f32x2{m, l};
  }
  __syncthreads();
  // Thread t folds units u = t, t + 512, ... of the valid rows: row j (tile
  // column j) = u / (D / 4), features d = 4 (u % (D / 4)) .. d + 3, over the
  // W partials in wavefront order -- only units of real rows get a thread
  // (a decode tile of g rows: g D / 4 threads), each read 16 bytes or a
  // broadcast.  Lane (column j, half) holds value k = 16 (d / 32) + 4 (d %
  // 32 / 8) + d % 4 of feature d, half = d / 4 % 2.
  constexpr int D4 = D / 4;
  const int nv = pack * a.Sq;  // valid rows: tile columns 0 .. nv - 1
  // Key split: the block's partial of every valid row (O unnormalised
  // relative to M, then M and the row sum) goes to the workspace, then an
  // arrival flag; the block that sees every split's flag merges the rows
  // itself -- one kernel per call.  Partials and flags move with
  // device-scope (sc1) accesses: stores write through to memory and count as
  // done only once there, loads read memory, never a stale line of another
  // XCD's L2 -- no cache-wide write-back or invalidate (as a release /
  // acquire fence would issue, at ~20 us a call here) is needed.
  typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
  constexpr int kAuxDevice = 16;  // sc1: device scope
  const int64_t rows = static_cast<int64_t>(a.B) * a.Hq * a.Sq;
  const Rsrc pr = __builtin_amdgcn_make_buffer_rsrc(a.part, 0, kBufRange, kRsrcWord3);
  const uint32_t ml_off = static_cast<uint32_t>(rows * a.nsplit * D * 4);  // bytes: (M, l) pairs
  for (int u = static_cast<int>(threadIdx.x); u < nv * D4; u += NT) {
    const int j = u / D4, d = 4 * (u - j * D4);
    const int ln = j + 32 * ((d >> 2) & 1), k = 16 * (d >> 5) + 4 * ((d >> 3) & 3);
    f32x2 mlw[W];  // m and half 0's l of row j
    float l1[W];   // half 1's l
    f32x4 val[W];
#pragma unroll
    for (int w = 0; w < W; ++w) {
      mlw[w] = *reinterpret_cast<const f32x2*>(rec_of(w, j) + D / 2);
      l1[w] = rec_of(w, j + 32)[D / 2 + 1];
      val[w] = *reinterpret_cast<const f32x4*>(rec_of(w, ln) + k);
    }
    float M = -INFINITY, lsum = 0.f;
#pragma unroll
    for (int w = 0; w < W; ++w) M = fmaxf(M, mlw[w][0]);
    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < W; ++w) {
      const float wt = mlw[w][0] == -INFINITY ? 0.f : fast_exp2(mlw[w][0] - M);  // a slice without keys weighs 0
      lsum += (mlw[w][1] + l1[w]) * wt;
      acc += val[w] * wt;
    }
    const int jq = j / pack, jh = kvh * a.g + gi * pack + (j - jq * pack);
    const int64_t r = (static_cast<int64_t>(b) * a.Hq + jh) * a.Sq + jq;
    if (a.nsplit == 1) {
      const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
      f16x4 rv;
#pragma unroll
      for (int e = 0; e < 4; ++e) rv[e] = static_cast<_Float16>(acc[e] * inv);
      *reinterpret_cast<f16x4*>(a.out + ((static_cast<int64_t>(b) * a.Sq + jq) * a.Hq + jh) * D + d) = rv;
      if (a.lse && d == 0) a.lse[r] = lsum > 0.f ? (M + log2f(lsum)) * kLn2 : -INFINITY;
    } else {
      const uint32_t prow = static_cast<uint32_t>(r * a.nsplit + sp);
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, acc), pr, (prow * D + d) * 4, 0, kAuxDevice);
      if (d == 0)
        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2_t, f32x2{M, lsum}), pr, ml_off + prow * 8, 0,
                                              kAuxDevice);
    }
  }
  if (a.nsplit == 1) return;

  // Arrival: every wavefront's partial stores done, then wavefront 0 stores
  // the flag (this call's ticket), waits for it, and reads every split's
  // flag of the group.  Of any two blocks, the one whose flag store finished
  // later reads the other's flag after it, so at least one block sees all of
  // them.  Every block that does merges the rows, to the same bits (splits
  // in a fixed order).  Mergers clear the flags, so replays of a captured
  // call (one ticket) start clear; a new call's ticket matches no older
  // call's flags.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  __shared__ int s_merge;
  // The group's flags (item: its (sequence, KV head, head group) index).
  const uint32_t fl_off = ml_off + static_cast<uint32_t>(rows * a.nsplit * 8) + item * a.nsplit * 4;
  if (wave == 0) {
    if (lane == 0) __builtin_amdgcn_raw_buffer_store_b32(a.ticket, pr, fl_off + sp * 4, 0, kAuxDevice);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    bool seen = true;
    for (int s2 = lane; s2 < a.nsplit; s2 += 64)
      seen = seen && __builtin_amdgcn_raw_buffer_load_b32(pr, fl_off + s2 * 4, 0, kAuxDevice) == a.ticket;
    const bool all = __all(seen);
    if (lane == 0) s_merge = all ? 1 : 0;
  }
  __syncthreads();
  if (!s_merge) return;

  // Merge: thread (row j, features 4 d4 .. + 3) over every split in order,
  // G splits' loads in flight at once, without a branch: past the last
  // split the loads repeat it (a valid address) and, like splits with l = 0
  // (no visible key), carry no weight.
  constexpr int RP = NT / D4, G = 16;
  const int d4 = static_cast<int>(threadIdx.x) % D4;
  const uint32_t last = static_cast<uint32_t>(a.nsplit - 1);
  for (int j = static_cast<int>(threadIdx.x) / D4; j < nv; j += RP) {
    const int jq = j / pack, jh = kvh * a.g + gi * pack + (j - jq * pack);
    const int64_t r = (static_cast<int64_t>(b) * a.Hq + jh) * a.Sq + jq;
    const uint32_t r0 = static_cast<uint32_t>(r * a.nsplit);
    float Mr = -INFINITY, Lr = 0.f;
    f32x4 ac = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < a.nsplit; s0 += G) {
      f32x2 ml[G];
      f32x4 ov[G];
#pragma unroll
      for (int jj = 0; jj < G; ++jj) {
        const uint32_t s2 = min(static_cast<uint32_t>(s0 + jj), last);
        ml[jj] = __builtin_bit_cast(f32x2, __builtin_amdgcn_raw_buffer_load_b64(pr, ml_off + (r0 + s2) * 8, 0, kAuxDevice));
        ov[jj] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(pr, ((r0 + s2) * D + 4 * d4) * 4, 0,
                                                                                 kAuxDevice));
      }
      float mv[G];  // the split's max, or -inf when it carries no weight
#pragma unroll
      for (int jj = 0; jj < G; ++jj) mv[jj] = s0 + jj < a.nsplit && ml[jj][1] > 0.f ? ml[jj][0] : -INFINITY;
      float Mn = Mr;
#pragma unroll
      for (int jj = 0; jj < G; ++jj) Mn = fmaxf(Mn, mv[jj]);
      if (Mn == -INFINITY) continue;  // nothing visible yet
      const float c = fast_exp2(Mr - Mn);  // Mr = -inf: c = 0
      Lr *= c;
      ac *= c;
#pragma unroll
      for (int jj = 0; jj < G; ++jj) {
        const float w = fast_exp2(mv[jj] - Mn);  // -inf: 0
        Lr += ml[jj][1] * w;
        ac += ov[jj] * w;
      }
      Mr = Mn;
    }
    const float inv = Lr > 0.f ? 1.f / Lr : 0.f;
    f16x4 rv;
#pragma unroll
    for (int e = 0; e < 4; ++e) rv[e] = static_cast<_Float16>(ac[e] * inv);
    *reinterpret_cast<f16x4*>(a.out + ((static_cast<int64_t>(b) * a.Sq + jq) * a.Hq + jh) * D + 4 * d4) = rv;
    if (a.lse && d4 == 0) a.lse[r] = Lr > 0.f ? (Mr + log2f(Lr)) * kLn2 : -INFINITY;
  }
  for (int s2 = static_cast<int>(threadIdx.x); s2 < a.nsplit; s2 += NT)
    __builtin_amdgcn_raw_buffer_store_b32(0u, pr, fl_off + s2 * 4, 0, kAuxDevice);
}

// Combines a key split's partials per (sequence, q head, query): one
// workgroup per row.  Thread (sl, d4) folds splits sl, sl + SL, ... of
// features 4 d4 .. 4 d4 + 3, G of them loaded at once (every load issued
// before the first is used); the SL folds of a feature are then combined
// through LDS.  Splits with l = 0 (no visible key) carry no weight; a row
// with none gives zeros and LSE -inf.  (One work-item per 4 features of a
// row, looping over the splits, took 5-7 us for 32 splits of 32 rows: the
// whole merge ran on 4 compute units.)
struct MergeArgs {
  const float* part;
  _Float16* out;
  float* lse;
  int Hq, Sq, D, nsplit;
  int64_t rows;  // B * Hq * Sq
};

template <int D>
__global__ __launch_bounds__(256) void sdpa_split_merge_kernel(MergeArgs a) {
  constexpr int D4 = D / 4, SL = 256 / D4, G = 4;
  __shared__ float s_m[SL], s_l[SL];
  __shared__ f32x4 s_acc[SL][D4];
  const int64_t r = blockIdx.x;
  const int d4 = static_cast<int>(threadIdx.x) % D4, sl = static_cast<int>(threadIdx.x) / D4;
  const float* pml = a.part + a.rows * a.nsplit * D + 2 * r * a.nsplit;
  const float* po = a.part + r * a.nsplit * D + 4 * d4;
  float M = -INFINITY, L = 0.f;
  f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int s0 = sl; s0 < a.nsplit; s0 += SL * G) {
    f32x2 ml[G];
    f32x4 ov[G];
#pragma unroll
    for (int j = 0; j < G; ++j) {
      const int sp = s0 + j * SL;
      const bool in = sp < a.nsplit;
      ml[j] = in ? *reinterpret_cast<const f32x2*>(pml + 2 * sp) : f32x2{-INFINITY, 0.f};
      ov[j] = in ? *reinterpret_cast<const f32x4*>(po + static_cast<int64_t>(sp) * D) : f32x4{0.f, 0.f, 0.f, 0.f};
    }
    float Mn = M;
#pragma unroll
    for (int j = 0; j < G; ++j)
      if (ml[j][1] > 0.f) Mn = fmaxf(Mn, ml[j][0]);
    if (Mn == -INFINITY) continue;  // nothing visible yet
    const float c = exp2f(M - Mn);  // M = -inf: c = 0
    L *= c;
    acc *= c;
#pragma unroll
    for (int j = 0; j < G; ++j) {
      if (!(ml[j][1] > 0.f)) continue;
      const float w = exp2f(ml[j][0] - Mn);
      L += ml[j][1] * w;
      acc += ov[j] * w;
    }
    M = Mn;
  }
  if (d4 == 0) {
    s_m[sl] = M;
    s_l[sl] = L;
  }
  s_acc[sl][d4] = acc;
  __syncthreads();
  if (sl != 0) return;
  M = -INFINITY;
#pragma unroll
  for (int t = 0; t < SL; ++t)
    if (s_l[t] > 0.f) M = fmaxf(M, s_m[t]);
  L = 0.f;
  acc = f32x4{0.f, 0.f, 0.f, 0.f};
  if (M != -INFINITY) {
#pragma unroll
    for (int t = 0; t < SL; ++t) {
      if (!(s_l[t] > 0.f)) continue;
      const float w = exp2f(s_m[t] - M);
      L += s_l[t] * w;
      acc += s_acc[t][d4] * w;
    }
  }
  const int d = 4 * d4;
  const int64_t qi = r % a.Sq, bh = r / a.Sq;
  const int64_t h = bh % a.Hq, b = bh / a.Hq;
  const float inv = L > 0.f ? 1.f / L : 0.f;
  f16x4 rv;
#pragma unroll
  for (int v = 0; v < 4; ++v) rv[v] = static_cast<_Float16>(acc[v] * inv);
  *reinterpret_cast<f16x4*>(a.out + ((b * a.Sq + qi) * a.Hq + h) * D + d) = rv;
  if (a.lse && d == 0) a.lse[r] = L > 0.f ? (M + log2f(L)) * kLn2 : -INFINITY;
}

// The same merge for many rows and few splits (chunked prefill: thousands
// of rows, 2-16 splits): D / 4 threads per row, each merging its 4 features
// over every split with the loads of 8 splits in flight at once, 256 / (D /
// 4) rows per block.  (The kernel above gives each row a block and spreads
// its splits over the block: right for decode's few rows and many splits;
// with one block per row of 8 splits its blocks take 9.9 us for 8192 rows,
// whose partials are 34 MB.)
template <int D>
__global__ __launch_bounds__(256) void sdpa_split_merge_rows_kernel(MergeArgs a) {
  constexpr int D4 = D / 4, RPB = 256 / D4, G = 8;
  const int d4 = static_cast<int>(threadIdx.x) % D4;
  const int64_t r = static_cast<int64_t>(blockIdx.x) * RPB + static_cast<int>(threadIdx.x) / D4;
  if (r >= a.rows) return;
  const float* pml = a.part + a.rows * a.nsplit * D + 2 * r * a.nsplit;
  const float* po = a.part + r * a.nsplit * D + 4 * d4;
  float M = -INFINITY, L = 0.f;
  f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < a.nsplit; s0 += G) {
    f32x2 ml[G];
    f32x4 ov[G];
#pragma unroll
    for (int j = 0; j < G; ++j) {
      const int sp = s0 + j;
      const bool in = sp < a.nsplit;
      ml[j] = in ? *reinterpret_cast<const f32x2*>(pml + 2 * sp) : f32x2{-INFINITY, 0.f};
      // Non-temporal: each partial is read once (chunked prefill, B 4 x 128
      // queries x 4096 keys, 56.2 -> 55.3 us a call; B 8 x 64 x 4096 56.7 ->
      // 52.9 us; one box, two alternations).
      ov[j] = in ? __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(po + static_cast<int64_t>(sp) * D))
                 : f32x4{0.f, 0.f, 0.f, 0.f};
    }
    float Mn = M;
#pragma unroll
    for (int j = 0; j < G; ++j)
      if (ml[j][1] > 0.f) Mn = fmaxf(Mn, ml[j][0]);
    if (Mn == -INFINITY) continue;  // nothing visible yet
    const float c = exp2f(M - Mn);  // M = -inf: c = 0
    L *= c;
    acc *= c;
#pragma unroll
    for (int j = 0; j < G; ++j) {
      if (!(ml[j][1] > 0.f)) continue;
      const float w = exp2f(ml[j][0] - Mn);
      L += ml[j][1] * w;
      acc += ov[j] * w;
    }
    M = Mn;
  }
  const int d = 4 * d4;
  const int64_t qi = r % a.Sq, bh = r / a.Sq;
  const int64_t h = bh % a.Hq, b = bh / a.Hq;
  const float inv = L > 0.f ? 1.f / L : 0.f;
  f16x4 rv;
#pragma unroll
  for (int v = 0; v < 4; ++v) rv[v] = static_cast<_Float16>(acc[v] * inv);
  *reinterpret_cast<f16x4*>(a.out + ((b * a.Sq + qi) * a.Hq + h) * D + d) = rv;
  if (a.lse && d == 0) a.lse[r] = L > 0.f ? (M + log2f(L)) * kLn2 : -INFINITY;
}

int device_cus();

// Key split of a call without a mask or causal flag: splits enough that the
// grid gives every compute unit a block, each split at least 8 steps (512
// keys; shorter splits lose more to the merge pass than they gain) -- or,
// when the unsplit grid would use at most an eighth of the compute units,
// at least four steps (256 keys): such calls are bound by the latency of
// each block's chain of steps more than by the merge (2 x 8 heads x 256
// queries x 256 keys: 18.7 us split into 64-key runs, 15.6 unsplit or in
// 256-key runs; 64 queries x 1024 keys: 12.7 split in 256-key runs, 14.3
// unsplit).  Returns nsplit; split_keys is a multiple of 64.
int plan_split(int64_t blocks, int Skv, int* split_keys) {
  *split_keys = Skv;
  const int64_t cus = device_cus() > 0 ? device_cus() : 256;
  const int min_keys = blocks * 8 <= cus ? 4 * kKT : 512;
  if (blocks >= cus || Skv < 2 * min_keys) return 1;
  const int64_t ns = std::min<int64_t>((cus + blocks - 1) / blocks, Skv / min_keys);
  if (ns <= 1) return 1;
  const int64_t keys = ((Skv + ns - 1) / ns + kKT - 1) / kKT * kKT;
  *split_keys = static_cast<int>(keys);
  return static_cast<int>((Skv + keys - 1) / keys);
}

size_t split_bytes(int64_t rows, int nsplit, int D) {
  return nsplit > 1 ? static_cast<size_t>(rows) * nsplit * (D + 2) * sizeof(float) : 0;
}

int pack_heads(int B, int Hkv, int g, int Sq);

int64_t blocks_for(int B, int Hkv, int g, int Sq, int pack) {
  return static_cast<int64_t>(B) * Hkv * (g / pack) * ((static_cast<int64_t>(pack) * Sq + kQB - 1) / kQB);
}

// The grid of a call without a mask: short query runs pack all g q heads of
// a KV head into one block's rows and split the keys until the grid fills
// the device, if the workspace (ws_bytes) holds the split's partials;
// otherwise the heads are packed only as far as the unsplit grid still
// fills the device (pack_heads).
struct GridPlan {
  int pack = 1, nsplit = 1, split_keys = 0;
  size_t part_bytes = 0;
  bool short_decode = false;  // sdpa_decode_short_kernel
  int waves = kWaves2;         // its wavefronts per block
};

GridPlan plan_grid(int B, int Hq, int Hkv, int Sq, int Skv, int D, bool causal, size_t ws_bytes) {
  GridPlan gp;
  const int g = Hq / Hkv;
  gp.split_keys = Skv;
  // Short decode: one row tile (the g q heads of a KV head times Sq <= 32
  // rows) whose keys fit one block (kWaves2 slices), or a split of them
  // over blocks that all run in one round of the device.
  if (!causal && Sq > 0 && static_cast<int64_t>(g) * Sq <= 32) {
    const int kw = D == 64 ? ShortLds<64>::kKW : ShortLds<128>::kKW;
    const int64_t cus = device_cus() > 0 ? device_cus() : 256;
    int waves = kWaves2;
    int ns = std::max(1, (Skv + waves * kw - 1) / (waves * kw));
    // A split over at most half the units at eight wavefronts: four-wavefront
    // blocks of half the keys, twice as many, one per unit (batch-1 GQA, 4096
    // keys at D 128: 256 blocks of 128 keys instead of 128 of 256).
    if (ns > 1 && static_cast<int64_t>(B) * Hkv * 2 * ns <= cus) {
      waves = 4;
      ns = (Skv + waves * kw - 1) / (waves * kw);
    }
    // the partials, then one arrival flag per (sequence, KV head, split)
    const size_t pb = ns > 1 ? split_bytes(static_cast<int64_t>(B) * Hq * Sq, ns, D) +
                                   static_cast<size_t>(B) * Hkv * ns * sizeof(uint32_t)
                             : 0;
    if (static_cast<int64_t>(B) * Hkv * ns <= cus && (ns == 1 || ws_bytes >= pb)) {
      gp.pack = g;
      gp.nsplit = ns;
      gp.split_keys = ns > 1 ? waves * kw : Skv;
      gp.part_bytes = pb;
      gp.short_decode = true;
      gp.waves = waves;
      return gp;
    }
  }
  if (!causal && Sq > 0) {
    const int p0 = Sq < kQB ? g : 1;
    int keys = Skv;
    const int ns = plan_split(blocks_for(B, Hkv, g, Sq, p0), Skv, &keys);
    const size_t pb = split_bytes(static_cast<int64_t>(B) * Hq * Sq, ns, D);
    if (ns > 1 && ws_bytes >= pb) {
      gp.pack = p0;
      gp.nsplit = ns;
      gp.split_keys = keys;
      gp.part_bytes = pb;
      return gp;
    }
  }
  gp.pack = pack_heads(B, Hkv, g, Sq);
  return gp;
}

// Decode calls (one query per sequence, no mask, no causal flag) too large
// for the short-decode kernel whose grid of (sequence, KV head, chunk) items
// fills at least half the device: they stream K / V through the split-KV
// decode kernels (decode_attn.hip), whose operands come straight from
// memory into registers -- no LDS tiles, no barrier per step.
spyre_hip::DenseDecodePlan dense_route(int B, int Hq, int Hkv, int Sq, int Skv, int D, bool causal, int mask_kind) {
  if (mask_kind != kNoMask || causal || Sq != 1) return {};
  if (plan_grid(B, Hq, Hkv, Sq, Skv, D, false, SIZE_MAX).short_decode) return {};
  return spyre_hip::dense_decode_plan(B, Hq, Hkv, Skv, D);
}

template <int W>
void launch_short_w(const Fwd2Args& f2, int D, bool prescaled, hipStream_t st) {
  const dim3 grid(f2.n_items);
  if (D == 128 && prescaled)
    sdpa_decode_short_kernel<128, true, W><<<grid, W * 64, 0, st>>>(f2);
  else if (D == 128)
    sdpa_decode_short_kernel<128, false, W><<<grid, W * 64, 0, st>>>(f2);
  else if (prescaled)
    sdpa_decode_short_kernel<64, true, W><<<grid, W * 64, 0, st>>>(f2);
  else
    sdpa_decode_short_kernel<64, false, W><<<grid, W * 64, 0, st>>>(f2);
}

void launch_short(const Fwd2Args& f2, int D, bool prescaled, int waves, hipStream_t st) {
  if (waves == 4)
    launch_short_w<4>(f2, D, prescaled, st);
  else
    launch_short_w<kWaves2>(f2, D, prescaled, st);
}

template <int MK, int SLOTS = 2, bool HALF = false>
void launch_lds(const Fwd2Args& f2, int D, bool prescaled, hipStream_t st) {
  const dim3 grid(f2.n_items);
  if (D == 128 && prescaled)
    sdpa_fwd_lds_kernel<128, true, MK, SLOTS, HALF><<<grid, kThreads2, 0, st>>>(f2);
  else if (D == 128)
    sdpa_fwd_lds_kernel<128, false, MK, SLOTS, HALF><<<grid, kThreads2, 0, st>>>(f2);
  else if (prescaled)
    sdpa_fwd_lds_kernel<64, true, MK, SLOTS, HALF><<<grid, kThreads2, 0, st>>>(f2);
  else
    sdpa_fwd_lds_kernel<64, false, MK, SLOTS, HALF><<<grid, kThreads2, 0, st>>>(f2);
}

// A copy of a mask with 16-byte rows: [bm][hm][qm][pitch bytes], keys past
// Skv zero.  One work-item per 16-byte unit; the source is read element by
// element through its strides (any alignment of its rows).
struct MaskPadArgs {
  const char* src;
  char* dst;
  int64_t sb, sh, sq, sk;  // source strides, elements
  int64_t n_units;         // bm * hm * qm * units
  int hm, qm, units, Skv, esz;
};

__global__ __launch_bounds__(256) void mask_pad_kernel(MaskPadArgs a) {
  const int64_t u = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (u >= a.n_units) return;
  const int64_t row = u / a.units;
  const int cu = static_cast<int>(u - row * a.units);
  const int q = static_cast<int>(row % a.qm);
  const int64_t bh = row / a.qm;
  const int h = static_cast<int>(bh % a.hm);
  const int64_t b = bh / a.hm;
  const int64_t base = b * a.sb + h * a.sh + q * a.sq;
  uint32_t w[4] = {0u, 0u, 0u, 0u};
  if (a.esz == 2) {
    const uint16_t* src = reinterpret_cast<const uint16_t*>(a.src);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int key = cu * 8 + e;
      const uint32_t x = key < a.Skv ? src[base + key * a.sk] : 0u;
      w[e >> 1] |= x << (16 * (e & 1));
    }
  } else {
    const uint8_t* src = reinterpret_cast<const uint8_t*>(a.src);
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int key = cu * 16 + e;
      const uint32_t x = key < a.Skv ? src[base + key * a.sk] : 0u;
      w[e >> 2] |= x << (8 * (e & 3));
    }
  }
  *reinterpret_cast<uint4*>(a.dst + u * 16) = make_uint4(w[0], w[1], w[2], w[3]);
}

bool aligned16(const void* p);

// How a call's mask reaches the kernels:
//  kRouteNone    no mask;
//  kRouteStaged  fp16 / bool, rows of whole 16-byte units: the main kernel
//                stages it as it lies;
//  kRouteCopied  other fp16 / bool masks: copied with 16-byte rows into the
//                workspace first (mask_pad_kernel), then staged;
//  kRouteVt      fp32 masks (or a copy whose slice would pass 2 GiB): the
//                per-wavefront kernel, V through the workspace.
enum MaskRoute { kRouteNone, kRouteStaged, kRouteCopied, kRouteVt };

struct MaskPlan {
  MaskRoute route = kRouteNone;
  int64_t span = 0;                      // bytes of one (sequence, head) slice as staged
  int64_t bm = 1, hm = 1, qm = 1, pitch = 0;  // kRouteCopied: extents kept, row pitch (bytes)
  size_t copy_bytes = 0;
};

MaskPlan plan_mask(const void* mask, int kind, const int64_t* ms, int B, int Hq, int Sq, int Skv) {
  MaskPlan p;
  if (kind == kNoMask) return p;
  if (kind == kMaskF32) {
    p.route = kRouteVt;
    return p;
  }
  const int64_t esz = kind == kMaskF16 ? 2 : 1;
  if (Sq == 0 || Skv == 0) {  // nothing of the mask is read
    p.route = kRouteStaged;
    return p;
  }
  // Staged as it lies only if every slice ends on a whole 16-byte unit: the
  // kernel loads whole units and the descriptor's range ends with the slice,
  // so a unit straddling the end would arrive as zeros, valid keys included.
  const int64_t span = ((static_cast<int64_t>(Sq) - 1) * ms[2] + Skv) * esz;
  if (ms[3] == 1 && aligned16(mask) && (ms[0] * esz) % 16 == 0 && (ms[1] * esz) % 16 == 0 &&
      (ms[2] * esz) % 16 == 0 && (Skv * esz) % 16 == 0 && span <= kBufRange) {
    p.route = kRouteStaged;
    p.span = span;
    return p;
  }
  p.bm = ms[0] != 0 ? B : 1;
  p.hm = ms[1] != 0 ? Hq : 1;
  p.qm = ms[2] != 0 ? Sq : 1;
  p.pitch = (static_cast<int64_t>(Skv) * esz + 15) / 16 * 16;
  p.span = p.qm * p.pitch;  // whole rows: the copy holds the last row's padding
  if (p.span > kBufRange) {
    p.route = kRouteVt;
    return p;
  }
  p.route = kRouteCopied;
  p.copy_bytes = static_cast<size_t>(p.bm * p.hm * p.qm * p.pitch);
  return p;
}

// Compute units of the current device, cached per device; 0 if the runtime
// cannot say.
int device_cus() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  int v = cache[dev].load(std::memory_order_relaxed);
  if (v > 0) return v;
  if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) return 0;
  cache[dev].store(v, std::memory_order_relaxed);
  return v;
}

// Rows per query for a call without a mask: the largest divisor p of g whose
// packed grid (B Hkv (g / p) ceil(p Sq / 256) blocks) still gives every
// compute unit a block, so packing never idles units.
int pack_heads(int B, int Hkv, int g, int Sq) {
  if (Sq >= kQB || g == 1) return 1;
  const int64_t cus = device_cus() > 0 ? device_cus() : 256;
  for (int p = g; p > 1; --p) {
    if (g % p) continue;
    const int64_t blocks = static_cast<int64_t>(B) * Hkv * (g / p) * ((static_cast<int64_t>(p) * Sq + kQB - 1) / kQB);
    if (blocks >= cus) return p;
  }
  return 1;
}

int64_t s64_of(int Skv) { return (static_cast<int64_t>(Skv) + kStick - 1) / kStick * kStick; }

bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

}  // namespace

extern "C" size_t spyre_sdpa_fwd_workspace_bytes(int B, int Hkv, int Skv, int D) {
  if (B <= 0 || Hkv <= 0 || Skv < 0 || D <= 0) return 0;
  return static_cast<size_t>(B) * Hkv * D * s64_of(Skv) * sizeof(_Float16);
}

extern "C" size_t spyre_sdpa_fwd_call_workspace_bytes(const void* attn_mask, int mask_kind,
                                                      const int64_t* mask_strides, int B, int Hq, int Hkv,
                                                      int Sq, int Skv, int D) {
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv || Sq < 0 || Skv < 0 || (D != 64 && D != 128)) return 0;
  if (mask_kind == kNoMask) {  // a key split's partials (calls without the causal flag)
    const size_t split = plan_grid(B, Hq, Hkv, Sq, Skv, D, false, SIZE_MAX).part_bytes;
    const spyre_hip::DenseDecodePlan dp = dense_route(B, Hq, Hkv, Sq, Skv, D, false, mask_kind);
    return dp.ok ? std::max(split, dp.ws_bytes) : split;  // the split for calls the decode route refuses
  }
  if (!mask_strides || mask_kind < kNoMask || mask_kind > kMaskBool) return 0;
  const MaskPlan mp = plan_mask(attn_mask, mask_kind, mask_strides, B, Hq, Sq, Skv);
  if (mp.route == kRouteCopied) return mp.copy_bytes;
  return mp.route == kRouteVt ? spyre_sdpa_fwd_workspace_bytes(B, Hkv, Skv, D) : 0;
}

extern "C" int spyre_sdpa_fwd_f16(const void* q, const int64_t* q_strides, const void* k,
                                  const int64_t* k_strides, const void* v, const int64_t* v_strides,
                                  const void* attn_mask, int mask_kind, const int64_t* mask_strides,
                                  int is_causal, float scale, void* out, float* lse,
                                  void* workspace, size_t workspace_bytes, int B, int Hq, int Hkv,
                                  int Sq, int Skv, int D, void* stream) {
  spyre_hip::clear_error();
  SPYRE_REQUIRE(q_strides && k_strides && v_strides, SPYRE_EINVAL, "null stride argument");
  SPYRE_REQUIRE((Sq == 0 || (q && out)) && (Skv == 0 || (k && v)), SPYRE_EINVAL,
                "null pointer argument");
  SPYRE_REQUIRE(B > 0 && Hq > 0 && Hkv > 0 && Hq % Hkv == 0 && Sq >= 0 && Skv >= 0, SPYRE_EINVAL,
                "bad shape B=%d Hq=%d Hkv=%d Sq=%d Skv=%d", B, Hq, Hkv, Sq, Skv);
  SPYRE_REQUIRE(D == 64 || D == 128, SPYRE_EUNSUPPORTED, "head_dim %d not in {64, 128}", D);
  SPYRE_REQUIRE(mask_kind >= kNoMask && mask_kind <= kMaskBool, SPYRE_EINVAL, "bad mask kind %d",
                mask_kind);
  SPYRE_REQUIRE(mask_kind == kNoMask || (attn_mask && mask_strides), SPYRE_EINVAL,
                "mask pointer / strides missing");
  SPYRE_REQUIRE(!(is_causal && mask_kind != kNoMask), SPYRE_EINVAL,
                "is_causal and an attention mask are exclusive");
  SPYRE_REQUIRE(B <= 65535 && Hq <= 65535, SPYRE_EUNSUPPORTED, "B or Hq above 65535");
  // 16-byte rows: every operand row is read as whole 16-byte vectors.
  SPYRE_REQUIRE(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(out), SPYRE_EINVAL,
                "q, k, v, out must be 16-byte aligned");
  for (int i = 0; i < 3; ++i)
    SPYRE_REQUIRE(q_strides[i] % 8 == 0 && k_strides[i] % 8 == 0 && v_strides[i] % 8 == 0 &&
                      q_strides[i] >= 0 && k_strides[i] >= 0 && v_strides[i] >= 0,
                  SPYRE_EINVAL, "q/k/v strides must be non-negative multiples of 8 elements");
  if (mask_kind != kNoMask) {
    for (int i = 0; i < 4; ++i)
      SPYRE_REQUIRE(mask_strides[i] >= 0, SPYRE_EINVAL, "negative mask stride");
    SPYRE_REQUIRE(static_cast<int64_t>(Skv) * mask_strides[3] < (int64_t{1} << 31), SPYRE_EUNSUPPORTED,
                  "mask row spans 2^31 elements or more");
    const uintptr_t esz = mask_kind == kMaskF32 ? 4 : mask_kind == kMaskF16 ? 2 : 1;
    SPYRE_REQUIRE(reinterpret_cast<uintptr_t>(attn_mask) % esz == 0, SPYRE_EINVAL,
                  "mask pointer not aligned to its element");
  }
  // The mask's route (plan_mask); a masked call whose workspace holds V's
  // relayout but not the mask's copy takes the per-wavefront kernel.
  MaskPlan mp = plan_mask(attn_mask, mask_kind, mask_strides, B, Hq, Sq, Skv);
  if (mp.route == kRouteCopied && (!workspace || workspace_bytes < mp.copy_bytes || !aligned16(workspace)))
    mp.route = kRouteVt;
  const size_t need = mp.route == kRouteVt       ? spyre_sdpa_fwd_workspace_bytes(B, Hkv, Skv, D)
                      : mp.route == kRouteCopied ? mp.copy_bytes
                                                 : 0;
  SPYRE_REQUIRE(need == 0 || (workspace && workspace_bytes >= need && aligned16(workspace)),
                SPYRE_ENOSPC, "workspace %zu < %zu bytes (or misaligned)", workspace_bytes, need);
  const bool lds_path = mp.route != kRouteVt;
  if (Sq == 0) return SPYRE_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int s64 = static_cast<int>(s64_of(Skv));
  const void* mask_ptr = attn_mask;
  int64_t m_sb = 0, m_sh = 0, m_sq = 0;
  if (mask_kind != kNoMask) {
    m_sb = mask_strides[0];
    m_sh = mask_strides[1];
    m_sq = mask_strides[2];
  }
  if (mp.route == kRouteCopied) {
    const int esz = mask_kind == kMaskF16 ? 2 : 1;
    MaskPadArgs pa{static_cast<const char*>(attn_mask), static_cast<char*>(workspace), mask_strides[0],
                   mask_strides[1], mask_strides[2], mask_strides[3],
                   static_cast<int64_t>(mp.copy_bytes / 16), static_cast<int>(mp.hm), static_cast<int>(mp.qm),
                   static_cast<int>(mp.pitch / 16), Skv, esz};
    const int64_t blocks = (pa.n_units + 255) / 256;
    SPYRE_REQUIRE(blocks < (int64_t{1} << 31), SPYRE_EUNSUPPORTED, "mask too large");
    mask_pad_kernel<<<dim3(static_cast<unsigned>(blocks)), 256, 0, st>>>(pa);
    const hipError_t e = hipGetLastError();
    SPYRE_REQUIRE(e == hipSuccess, SPYRE_EHIP, "mask copy launch failed: %s", hipGetErrorString(e));
    const int64_t pe = mp.pitch / esz;  // row pitch, elements
    mask_ptr = workspace;
    m_sq = mp.qm > 1 ? pe : 0;
    m_sh = mp.hm > 1 ? mp.qm * pe : 0;
    m_sb = mp.bm > 1 ? mp.hm * mp.qm * pe : 0;
  }
  if (Skv > 0 && !lds_path) {
    VtArgs va{static_cast<const _Float16*>(v), v_strides[0], v_strides[1], v_strides[2],
              static_cast<_Float16*>(workspace), Hkv, Skv, s64, D,
              static_cast<int64_t>(B) * Hkv * (s64 / 64) * (D / 64)};
    const int64_t blocks = (va.tiles + kWaves - 1) / kWaves;
    SPYRE_REQUIRE(blocks < (int64_t{1} << 31), SPYRE_EUNSUPPORTED, "V too large");
    v_token_sticks_kernel<<<dim3(static_cast<unsigned>(blocks)), kThreads, 0, st>>>(va);
    const hipError_t e = hipGetLastError();
    SPYRE_REQUIRE(e == hipSuccess, SPYRE_EHIP, "V restick launch failed: %s", hipGetErrorString(e));
  }
  FwdArgs fa{};
  fa.q = static_cast<const _Float16*>(q);
  fa.k = static_cast<const _Float16*>(k);
  fa.vt = static_cast<const _Float16*>(workspace);
  fa.q_sb = q_strides[0];
  fa.q_sh = q_strides[1];
  fa.q_ss = q_strides[2];
  fa.k_sb = k_strides[0];
  fa.k_sh = k_strides[1];
  fa.k_ss = k_strides[2];
  fa.vt_sb = static_cast<int64_t>(Hkv) * D * s64;
  fa.vt_sh = static_cast<int64_t>(D) * s64;
  // Buffer extents (bytes) of one head: K and V rows 0..Skv-1, Vt [D, s64].
  const int64_t k_span = Skv > 0 ? ((static_cast<int64_t>(Skv) - 1) * k_strides[2] + D) * 2 : 0;
  const int64_t v_span = Skv > 0 ? ((static_cast<int64_t>(Skv) - 1) * v_strides[2] + D) * 2 : 0;
  const int64_t vt_span = static_cast<int64_t>(D) * s64 * 2;
  SPYRE_REQUIRE(k_span <= kBufRange && v_span <= kBufRange && vt_span <= kBufRange, SPYRE_EUNSUPPORTED,
                "one head of K or V spans 2 GiB or more");
  fa.k_bytes = static_cast<uint32_t>(k_span);
  fa.vt_bytes = static_cast<uint32_t>(vt_span);
  fa.mask = attn_mask;
  fa.mask_kind = mask_kind;
  if (mask_kind != kNoMask) {
    fa.m_sb = mask_strides[0];
    fa.m_sh = mask_strides[1];
    fa.m_sq = mask_strides[2];
    fa.m_sk = mask_strides[3];
  }
  fa.out = static_cast<_Float16*>(out);
  fa.lse = lse;
  fa.B = B;
  fa.Hq = Hq;
  fa.Hkv = Hkv;
  fa.g = Hq / Hkv;
  fa.Sq = Sq;
  fa.Skv = Skv;
  fa.s64 = s64;
  fa.causal = is_causal ? 1 : 0;
  fa.scale_log2 = scale * kLog2e;
  if (lds_path) {
    const spyre_hip::DenseDecodePlan dp = dense_route(B, Hq, Hkv, Sq, Skv, D, is_causal != 0, mask_kind);
    if (dp.ok && k_strides[2] < (int64_t{1} << 23) && v_strides[2] < (int64_t{1} << 23) &&
        (k_strides[2] == 0 || k_strides[2] >= D) && (v_strides[2] == 0 || v_strides[2] >= D) &&
        (dp.ws_bytes == 0 || (workspace && aligned16(workspace) && workspace_bytes >= dp.ws_bytes)))
      return spyre_hip::dense_decode_launch(dp, q, q_strides, k, k_strides, v, v_strides, out, lse, workspace, B,
                                            Hq, Hkv, Skv, D, scale, stream);
    // K/V tiles (and mask blocks) shared through LDS.
    Fwd2Args f2{};
    f2.q = fa.q;
    f2.k = fa.k;
    f2.v = static_cast<const _Float16*>(v);
    f2.q_sb = fa.q_sb;
    f2.q_sh = fa.q_sh;
    f2.q_ss = fa.q_ss;
    f2.k_sb = fa.k_sb;
    f2.k_sh = fa.k_sh;
    f2.k_ss = fa.k_ss;
    f2.v_sb = v_strides[0];
    f2.v_sh = v_strides[1];
    f2.v_ss = v_strides[2];
    f2.out = fa.out;
    f2.lse = fa.lse;
    f2.B = B;
    f2.Hq = Hq;
    f2.Hkv = Hkv;
    f2.g = fa.g;
    f2.Sq = Sq;
    f2.Skv = Skv;
    f2.causal = fa.causal;
    // Without a mask, short query runs pack q heads of a KV head into one
    // block's rows, so they share each K / V tile (decode: one block per
    // (sequence, KV head) instead of g mostly idle ones).
    // And (plan_grid) a key split when the blocks would not fill the device
    // and the workspace holds its partials.
    GridPlan gpl;
    if (mask_kind == kNoMask)
      gpl = plan_grid(B, Hq, Hkv, Sq, Skv, D, is_causal != 0, workspace && aligned16(workspace) ? workspace_bytes : 0);
    f2.pack = gpl.pack;
    f2.gp = fa.g / f2.pack;
    f2.qblocks = static_cast<int>((static_cast<int64_t>(f2.pack) * Sq + kQB - 1) / kQB);
    f2.nsplit = gpl.nsplit;
    f2.split_keys = gpl.nsplit > 1 ? gpl.split_keys : Skv;
    f2.part = gpl.nsplit > 1 ? static_cast<float*>(workspace) : nullptr;
    const int64_t items = blocks_for(B, Hkv, fa.g, Sq, f2.pack) * f2.nsplit;
    SPYRE_REQUIRE(items < (int64_t{1} << 31), SPYRE_EUNSUPPORTED, "too many query blocks");
    f2.n_items = static_cast<uint32_t>(items);
    f2.xcd_remap = items % 8 == 0;
    f2.scale_log2 = fa.scale_log2;
    // |scale log2 e| <= 1: q times it stays within fp16, so Q is prescaled.
    const bool prescaled = fabsf(f2.scale_log2) <= 1.f;
    f2.mask = mask_ptr;
    f2.m_sb = m_sb;
    f2.m_sh = m_sh;
    f2.m_sq = m_sq;
    f2.m_bytes = static_cast<uint32_t>(mp.span);
    if (gpl.short_decode) {
      // One row tile, its keys all in flight at once; a key split merges in
      // the same kernel.
      f2.ticket = spyre_hip::next_call_ticket();
      launch_short(f2, D, prescaled, gpl.waves, st);
    } else if (mask_kind == kMaskF16) {
      launch_lds<kMaskF16>(f2, D, prescaled, st);
    } else if (mask_kind == kMaskBool) {
      launch_lds<kMaskBool>(f2, D, prescaled, st);
    } else if (static_cast<int64_t>(f2.pack) * Sq <= kQB / 2) {
      launch_lds<kNoMask, 4, true>(f2, D, prescaled, st);  // half steps: two wavefronts per row tile
    } else if (static_cast<int64_t>(f2.pack) * Sq < kQB) {
      launch_lds<kNoMask, 4>(f2, D, prescaled, st);  // blocks with fewer rows than wavefronts can fill
    } else {
      launch_lds<kNoMask>(f2, D, prescaled, st);
    }
    if (f2.nsplit > 1 && !gpl.short_decode) {
      const hipError_t e0 = hipGetLastError();
      SPYRE_REQUIRE(e0 == hipSuccess, SPYRE_EHIP, "sdpa launch failed: %s", hipGetErrorString(e0));
      MergeArgs ma{f2.part, f2.out, f2.lse, Hq, Sq, D, f2.nsplit, static_cast<int64_t>(B) * Hq * Sq};
      SPYRE_REQUIRE(ma.rows < (int64_t{1} << 31), SPYRE_EUNSUPPORTED, "too many rows");
      // Rows of their own threads once they fill 256 blocks and the splits
      // are few; otherwise a block per row over its splits.
      const int64_t rpb = 256 / (D / 4);
      if (f2.nsplit <= 16 && ma.rows >= 256 * rpb) {
        const dim3 mgrid(static_cast<unsigned>((ma.rows + rpb - 1) / rpb));
        if (D == 128)
          sdpa_split_merge_rows_kernel<128><<<mgrid, 256, 0, st>>>(ma);
        else
          sdpa_split_merge_rows_kernel<64><<<mgrid, 256, 0, st>>>(ma);
      } else {
        const dim3 mgrid(static_cast<unsigned>(ma.rows));
        if (D == 128)
          sdpa_split_merge_kernel<128><<<mgrid, 256, 0, st>>>(ma);
        else
          sdpa_split_merge_kernel<64><<<mgrid, 256, 0, st>>>(ma);
      }
    }
  } else {
    const dim3 grid((Sq + kWaves * kQ - 1) / (kWaves * kQ), Hq, B);
    auto launch = [&](auto mk) {
      constexpr int MK = decltype(mk)::value;
      if (D == 128)
        sdpa_fwd_kernel<128, MK><<<grid, kThreads, 0, st>>>(fa);
      else
        sdpa_fwd_kernel<64, MK><<<grid, kThreads, 0, st>>>(fa);
    };
    switch (mask_kind) {
      case kMaskF16: launch(std::integral_constant<int, kMaskF16>{}); break;
      case kMaskF32: launch(std::integral_constant<int, kMaskF32>{}); break;
      default: launch(std::integral_constant<int, kMaskBool>{}); break;
    }
  }
  const hipError_t e = hipGetLastError();
  SPYRE_REQUIRE(e == hipSuccess, SPYRE_EHIP, "sdpa launch failed: %s", hipGetErrorString(e));
  return SPYRE_OK;
}
