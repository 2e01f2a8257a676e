// GPU executor of DMA loop nests (spyre_dma_copy).
//
// A loop nest says: for every index tuple i, dst[off_d + i.sd] = src[off_s + i.ss].
// The host normalises it (drops unit loops, merges loops that are contiguous
// on both sides) and picks one of four kinds of kernel:
//
//  * stick tile: one loop is a whole 128-byte stick, unit-stride on both
//               sides, and two others continue it contiguously, one in dst
//               (A) and one in src (B) -- row-major <-> sticks.  A workgroup
//               moves a tile of 32 x 32 sticks (128 KiB): it loads 32 runs
//               of 32 sticks (4 KiB contiguous in src), stages them in LDS
//               and stores 32 runs of 32 sticks (4 KiB contiguous in dst).
//               With all of a workgroup's loads issued before its stores and
//               one such workgroup per CU, the chip reads in one phase and
//               writes in the next, which HBM serves better than the mixed
//               read/write stream of small per-lane copies.
//  * vec:       one loop is unit-stride on both sides.  Each lane moves four
//               items of up to 16 bytes (loads issued before stores); eight
//               lanes cover one 128-byte stick, so every wavefront touches
//               whole cache lines on both sides.
//  * transpose: one loop is unit-stride in src and another in dst (the stick
//               moves to another dim, e.g. transpose-restick).  A wavefront
//               owns four 64x64 tiles of 2-byte elements (8x8 blocks of
//               16 bytes); its loads (all 32 first) go straight into LDS,
//               each lane then reads one 8x8 block per tile, transposes it
//               in registers and stores eight 16-byte column segments.
//               Loads and stores are both 128-byte-line coalesced.  4-byte
//               elements, and nests with more than three outer loops, use
//               a register-only form of the same tiling.
//  * scalar:    anything else, element by element.
//
// Stick tiles and 2-byte transposes have a stepped form for nests of whole
// tiles whose spans fit 32-bit buffer offsets (the common case): the tile
// index is decomposed once, in 32-bit arithmetic, over only the loops
// longer than one, from a kernel argument block sized to those loops, and
// nothing is predicated.
//
// Index decomposition uses multiply-high division by loop-invariant divisors
// (Granlund & Montgomery, "Division by Invariant Integers using
// Multiplication", PLDI 1994, round-up variant), valid for 0 <= n, d < 2^31.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstring>
#include <type_traits>
#include <vector>

#include "spyre_common.h"
#include "transpose8.h"

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

struct FastDiv {
  uint32_t d, mul, shift;
};

FastDiv make_fastdiv(uint32_t d) {
  uint32_t l = 0;
  while ((uint64_t{1} << l) < d) ++l;
  const uint64_t m = ((uint64_t{1} << 32) * ((uint64_t{1} << l) - d)) / d + 1;
  return FastDiv{d, static_cast<uint32_t>(m), l};
}

// Reads a kernel argument into scalar registers here and keeps it there.
// Arguments are read from memory where they are used (the compiler may
// re-read rather than hold them); one first needed after the load phase of
// a bandwidth-bound kernel would wait behind the whole chip's traffic.  The
// empty asm makes the value opaque, so it cannot be re-read.
template <typename T>
__device__ __forceinline__ T pinned(T x) {
  asm volatile("" : "+s"(x));
  return x;
}

__device__ __forceinline__ uint32_t fdiv(uint32_t n, const FastDiv& f) {
  return (__umulhi(n, f.mul) + n) >> f.shift;
}

constexpr int kMaxLoops = SPYRE_MAX_RANK;
constexpr int kThreads = 256;
constexpr int kItems = 4;       // vec kernel: items per lane, strided by the block size
constexpr int kTileSticks = 32; // stick tile: 32 x 32 sticks of 128 B per workgroup
constexpr int kAuxNT = 2;       // cache policy of a memory instruction: non-temporal
constexpr int kTransposeTiles = 4;  // 64x64 tiles per wavefront

struct Nest {
  int nouter;                 // loops decomposed from the item index (after the inner one)
  FastDiv inner;              // inner loop length in items
  FastDiv outer[kMaxLoops];   // outer loop lengths
  int64_t inner_ss, inner_sd; // inner strides (bytes per item)
  int64_t ss[kMaxLoops], sd[kMaxLoops];  // outer strides (bytes)
  int64_t off_s, off_d;       // bytes
  uint32_t total;             // items
};

template <int VB>
struct VecT;
template <> struct VecT<16> { using T = u32x4; };
template <> struct VecT<8> { using T = u32x2; };
template <> struct VecT<4> { using T = uint32_t; };
template <> struct VecT<2> { using T = uint16_t; };
template <> struct VecT<1> { using T = uint8_t; };

__device__ __forceinline__ void item_offsets(const Nest& n, uint32_t i, int64_t& so, int64_t& sd) {
  uint32_t q = fdiv(i, n.inner);
  const uint32_t r = i - q * n.inner.d;
  so = n.off_s + static_cast<int64_t>(r) * n.inner_ss;
  sd = n.off_d + static_cast<int64_t>(r) * n.inner_sd;
  for (int k = 0; k < n.nouter; ++k) {
    const uint32_t q2 = fdiv(q, n.outer[k]);
    const int64_t c = q - q2 * n.outer[k].d;
    so += c * n.ss[k];
    sd += c * n.sd[k];
    q = q2;
  }
}

// Each lane moves ITEMS items of VB bytes; all loads are issued before the
// stores so several cache lines per lane are in flight.
template <int VB, int ITEMS, bool GUARDED>
__device__ __forceinline__ void vec_items(const char* __restrict__ src, char* __restrict__ dst,
                                          const Nest& n, uint32_t base) {
  using T = typename VecT<VB>::T;
  T v[ITEMS];
  int64_t doff[ITEMS];
#pragma unroll
  for (int it = 0; it < ITEMS; ++it) {
    const uint32_t i = base + it * kThreads;
    if (!GUARDED || i < n.total) {
      int64_t so;
      item_offsets(n, i, so, doff[it]);
      v[it] = __builtin_nontemporal_load(reinterpret_cast<const T*>(src + so));
    }
  }
  __builtin_amdgcn_sched_barrier(0);  // keep every load ahead of the stores
#pragma unroll
  for (int it = 0; it < ITEMS; ++it)
    if (!GUARDED || base + it * kThreads < n.total)
      __builtin_nontemporal_store(v[it], reinterpret_cast<T*>(dst + doff[it]));
}

// Each lane moves ITEMS items of VB bytes; all loads are issued before the
// stores so several cache lines per lane are in flight.  Only the last
// block predicates its items.
template <int VB, int ITEMS>
__global__ __launch_bounds__(kThreads) void dma_vec_kernel(const char* __restrict__ src,
                                                           char* __restrict__ dst, Nest n) {
  const uint32_t first = blockIdx.x * (kThreads * ITEMS);
  const uint32_t base = first + threadIdx.x;
  if (first + kThreads * ITEMS <= n.total)
    vec_items<VB, ITEMS, false>(src, dst, n, base);
  else
    vec_items<VB, ITEMS, true>(src, dst, n, base);
}

// Stick-tile nest: a 128-byte stick (8 x 16 B) moved whole; loop A (nA
// sticks) continues it in dst (dst stride 128 B), loop B (nB sticks) in src
// (src stride 128 B).  Workgroups enumerate (tile of A, tile of B, outer
// loops).
struct SNest {
  uint32_t na, nb;
  FastDiv tiles_x, tiles_y;  // tile counts in enumeration order (x fastest)
  int b_first;               // x is B (else A)
  int nouter;
  FastDiv outer[kMaxLoops];
  int64_t ss[kMaxLoops], sd[kMaxLoops];
  int64_t a_ss;  // src stride of A (bytes)
  int64_t b_sd;  // dst stride of B (bytes)
  int64_t off_s, off_d;
};

// 16 bytes per lane from global memory straight into LDS: lane l of the
// wavefront writes lds + 16 l (lds wave-uniform).  Non-temporal: every
// byte is read once.
__device__ __forceinline__ void load_lds16(const char* g, char* lds) {
  __builtin_amdgcn_global_load_lds(static_cast<const void*>(g), (__attribute__((address_space(3))) void*)lds,
                                   16, 0, kAuxNT);
}

// The same through a buffer descriptor: base and extent in scalar
// registers, a 32-bit per-lane byte offset (one VGPR) -- fewer address
// instructions per load than 64-bit addresses.  kBufRange bounds the
// offsets (the host checks that a tile's span fits).
typedef __amdgpu_buffer_rsrc_t Rsrc;
constexpr uint32_t kBufRange = 0x7ffffff0u;
constexpr uint32_t kBufOob = 0x80000000u;  // an offset past kBufRange: the access is skipped
constexpr int kRsrcWord3 = 0x00020000;  // raw (untyped) buffer, 32-bit format

__device__ __forceinline__ Rsrc make_rsrc(const char* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(base), 0, kBufRange, kRsrcWord3);
}

__device__ __forceinline__ void load_lds16(Rsrc r, uint32_t off, char* lds) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, off, 0, 0, kAuxNT);
}

__device__ __forceinline__ void store16(Rsrc r, uint32_t off, u32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, kAuxNT);
}

// Descriptor of `range` bytes at base, and accesses whose offset is split
// into a per-lane part (voff, a VGPR) and a wave-uniform part (soff, an
// SGPR: one scalar add per access instead of a vector one).
__device__ __forceinline__ Rsrc make_rsrc(const char* base, uint32_t range) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(base), 0, range, kRsrcWord3);
}

__device__ __forceinline__ void load_lds16(Rsrc r, uint32_t voff, uint32_t soff, char* lds) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, soff, 0, kAuxNT);
}

__device__ __forceinline__ void store16(Rsrc r, uint32_t voff, uint32_t soff, u32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, voff, soff, kAuxNT);
}

__device__ __forceinline__ void wait_loads() {
  // s_waitcnt vmcnt(0); expcnt and lgkmcnt at their maxima (gfx9 encoding)
  __builtin_amdgcn_s_waitcnt(0 | (0x7 << 4) | (0xF << 8));
}

constexpr int kStepLoops = 4;

// The arguments of a stepped kernel: NL tile loops (the lengths and byte
// strides of the loops a tile index decomposes into, fastest first), and
// 32-bit offsets and descriptor ranges, the host having checked that each
// side's span fits a buffer descriptor.
template <int NL>
struct StepNest {
  uint32_t count;            // tiles (transpose: a multiple of kTransposeTiles)
  uint32_t off_s, off_d;     // byte offsets of the nest in src / dst
  uint32_t span_s, span_d;   // descriptor ranges (bytes)
  uint32_t s1, s2;           // transpose: src stride of B, dst stride of A;
                             // stick tile: src stride of A, dst stride of B
  FastDiv loop[NL];
  uint32_t ss[NL], sd[NL];
};

#define SPYRE_PIN_LOOP(k) "+s"(x.loop[k].d), "+s"(x.loop[k].mul), "+s"(x.loop[k].shift), "+s"(x.ss[k]), "+s"(x.sd[k])
#define SPYRE_PIN_HEAD "+s"(src), "+s"(dst), "+s"(x.count), "+s"(x.off_s), "+s"(x.off_d), "+s"(x.span_s), \
                       "+s"(x.span_d), "+s"(x.s1), "+s"(x.s2)
// Every field and both base pointers in scalar registers, read in one
// batch at entry (an argument read after another's wait costs a memory
// round trip before the first load).
template <int NL>
__device__ __forceinline__ StepNest<NL> read_step(const StepNest<NL>& n, const char*& src, char*& dst) {
  StepNest<NL> x = n;
  if constexpr (NL == 1) {
    asm volatile("" : SPYRE_PIN_HEAD, SPYRE_PIN_LOOP(0));
  } else if constexpr (NL == 2) {
    asm volatile("" : SPYRE_PIN_HEAD, SPYRE_PIN_LOOP(0), SPYRE_PIN_LOOP(1));
  } else if constexpr (NL == 3) {
    asm volatile("" : SPYRE_PIN_HEAD, SPYRE_PIN_LOOP(0), SPYRE_PIN_LOOP(1), SPYRE_PIN_LOOP(2));
  } else {
    static_assert(NL == 4, "1-4 tile loops");
    asm volatile("" : SPYRE_PIN_HEAD, SPYRE_PIN_LOOP(0), SPYRE_PIN_LOOP(1), SPYRE_PIN_LOOP(2), SPYRE_PIN_LOOP(3));
  }
  return x;
}
#undef SPYRE_PIN_HEAD
#undef SPYRE_PIN_LOOP

// Byte offsets of tile q of a stepped nest (shift and mask when every loop
// length is a power of two).
template <int NL, bool POW2>
__device__ __forceinline__ void step_offsets(const StepNest<NL>& x, uint32_t q, uint32_t& so, uint32_t& sd) {
  so = x.off_s;
  sd = x.off_d;
#pragma unroll
  for (int k = 0; k < NL; ++k) {
    uint32_t q2, c;
    if (POW2) {
      c = q & (x.loop[k].d - 1);
      q2 = q >> x.loop[k].shift;
    } else {
      q2 = fdiv(q, x.loop[k]);
      c = q - q2 * x.loop[k].d;
    }
    so += c * x.ss[k];
    sd += c * x.sd[k];
    q = q2;
  }
}

// Moves one tile of TA x TB sticks (128 KiB) through LDS.
// Loads: 1 KiB chunk c (the 8 B sticks 8 (c % (TB / 8)) .. + 7 of A row
// c / (TB / 8), contiguous in src) by wavefront c % 4, straight into LDS row
// a (TB sticks, padded by 128 B so the store-side reads of neighbouring A
// rows fall in different bank halves).
// Stores: 1 KiB chunk m (the 8 A sticks 8 (m % (TA / 8)) .. + 7 of B stick
// m / (TA / 8), contiguous in dst) by wavefront m % 4 (the four wavefronts
// write neighbouring chunks of one run together), or, WAVE_RUNS, chunks
// kPer w .. kPer (w + 1) - 1 by wavefront w (each writes whole runs).
// GUARDED: only A sticks < a_left and B sticks < b_left exist.
template <int TA, int TB, bool WAVE_RUNS, bool BUF, bool GUARDED>
__device__ __forceinline__ void stick_tile(const char* sp, char* dp, int64_t a_ss, int64_t b_sd,
                                           uint32_t a_left, uint32_t b_left, char* lds) {
  constexpr int kRowB = TB * 128 + 128;
  constexpr int kPer = TA * TB / 8 / 4;  // 1 KiB chunks per wavefront
  static_assert(TA * TB == 1024 && TA % 8 == 0 && TB % 8 == 0, "128 KiB tiles of whole 1 KiB chunks");
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x / 64));
  const int lane = static_cast<int>(threadIdx.x % 64);
  const Rsrc rs = make_rsrc(sp);
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int c = 4 * k + wave;
    const int a = c / (TB / 8), b = (c % (TB / 8)) * 8 + lane / 8;
    char* l = lds + a * kRowB + (c % (TB / 8)) * 1024;
    if (!GUARDED || (static_cast<uint32_t>(a) < a_left && static_cast<uint32_t>(b) < b_left)) {
      if (BUF)
        load_lds16(rs, static_cast<uint32_t>(a) * static_cast<uint32_t>(a_ss) + b * 128 + (lane % 8) * 16, l);
      else
        load_lds16(sp + a * a_ss + b * 128 + (lane % 8) * 16, l);
    }
  }
  wait_loads();
  __syncthreads();
  u32x4 x[kPer];
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int m = WAVE_RUNS ? kPer * wave + k : 4 * k + wave;
    const int b = m / (TA / 8), a = (m % (TA / 8)) * 8 + lane / 8;
    x[k] = *reinterpret_cast<const u32x4*>(lds + a * kRowB + b * 128 + (lane % 8) * 16);
  }
  const Rsrc rd = make_rsrc(dp);
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int m = WAVE_RUNS ? kPer * wave + k : 4 * k + wave;
    const int b = m / (TA / 8), a = (m % (TA / 8)) * 8 + lane / 8;
    if (!GUARDED || (static_cast<uint32_t>(a) < a_left && static_cast<uint32_t>(b) < b_left)) {
      if (BUF)
        store16(rd, static_cast<uint32_t>(b) * static_cast<uint32_t>(b_sd) + a * 128 + (lane % 8) * 16, x[k]);
      else
        __builtin_nontemporal_store(x[k], reinterpret_cast<u32x4*>(dp + b * b_sd + a * 128 + (lane % 8) * 16));
    }
  }
}

// BUF: the tile's spans fit 32-bit buffer offsets (checked on the host).
template <int TA, int TB, bool WAVE_RUNS, bool BUF>
__global__ __launch_bounds__(kThreads) void dma_stick_tile_kernel(const char* __restrict__ src,
                                                                   char* __restrict__ dst, SNest n) {
  __shared__ __align__(16) char lds[TA * (TB * 128 + 128)];
  // Every argument of the tile decomposition read by one statement: all the
  // reads are issued at entry and waited for once (an argument read after
  // another's wait costs a memory round trip before the first load).
  uint32_t na = n.na, nb = n.nb, nouter = n.nouter, b_first = n.b_first;
  int64_t a_ss = n.a_ss, b_sd = n.b_sd, so = n.off_s, sd = n.off_d;
  FastDiv dx = n.tiles_x, dy = n.tiles_y;
  asm volatile("" : "+s"(na), "+s"(nb), "+s"(nouter), "+s"(b_first), "+s"(a_ss), "+s"(b_sd), "+s"(so), "+s"(sd),
               "+s"(dx.d), "+s"(dx.mul), "+s"(dx.shift), "+s"(dy.d), "+s"(dy.mul), "+s"(dy.shift));
  uint32_t q = blockIdx.x;
  uint32_t q2 = fdiv(q, dx);
  const uint32_t tx = q - q2 * dx.d;
  q = q2;
  q2 = fdiv(q, dy);
  const uint32_t ty = q - q2 * dy.d;
  q = q2;
  const uint32_t ta = b_first ? ty : tx, tb = b_first ? tx : ty;
  for (uint32_t k = 0; k < nouter; ++k) {
    q2 = fdiv(q, n.outer[k]);
    const int64_t c = q - q2 * n.outer[k].d;
    so += c * n.ss[k];
    sd += c * n.sd[k];
    q = q2;
  }
  const uint32_t a0 = ta * TA, b0 = tb * TB;
  const char* sp = src + so + static_cast<int64_t>(a0) * a_ss + static_cast<int64_t>(b0) * 128;
  char* dp = dst + sd + static_cast<int64_t>(b0) * b_sd + static_cast<int64_t>(a0) * 128;
  // Edge tiles predicate every access; full tiles (all but the last along A
  // and B) run unpredicated.
  if (a0 + TA <= na && b0 + TB <= nb)
    stick_tile<TA, TB, WAVE_RUNS, BUF, false>(sp, dp, a_ss, b_sd, 0, 0, lds);
  else
    stick_tile<TA, TB, WAVE_RUNS, BUF, true>(sp, dp, a_ss, b_sd, na - a0, nb - b0, lds);
}

// The stepped form of dma_stick_tile_kernel: every tile whole, both spans
// within one buffer descriptor, the tile index decomposed over the tile
// loops (B tiles, A tiles, the outer loops; those longer than one) in
// 32-bit arithmetic.  Every access's per-lane offset is lane * 16 -- the
// eight lanes of a stick and the eight sticks of a 1 KiB chunk are
// contiguous on both sides -- and the rest is a scalar offset.
// (Storing the first half of a tile while its second half loads was
// measured no faster on fp16 [4096, 4096] in either direction -- the two
// streams share the same HBM -- and slower where the halves split 4 KiB
// src runs.)
template <int TA, int TB, bool WAVE_RUNS, int NL, bool POW2>
__global__ __launch_bounds__(kThreads) void dma_stick_step_kernel(const char* __restrict__ src_arg,
                                                                  char* __restrict__ dst_arg, StepNest<NL> n) {
  constexpr int kRowB = TB * 128 + 128;
  constexpr int kPer = TA * TB / 8 / 4;  // 1 KiB chunks per wavefront
  static_assert(TA * TB == 1024 && TA % 8 == 0 && TB % 8 == 0, "128 KiB tiles of whole 1 KiB chunks");
  __shared__ __align__(16) char lds[TA * kRowB];
  const char* src = src_arg;
  char* dst = dst_arg;
  const StepNest<NL> x = read_step(n, src, dst);
  const uint32_t a_ss = x.s1, b_sd = x.s2;
  uint32_t so, sd;
  step_offsets<NL, POW2>(x, blockIdx.x, so, sd);
  const Rsrc rs = make_rsrc(src, x.span_s), rd = make_rsrc(dst, x.span_d);
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
  const uint32_t lane = threadIdx.x % 64, v = lane * 16;
  // load chunk c: A row c / (TB / 8), sticks 8 (c % (TB / 8)) .. + 7
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const uint32_t c = 4 * k + wave, a = c / (TB / 8), cb = c % (TB / 8);
    load_lds16(rs, v, so + a * a_ss + cb * 1024, lds + a * kRowB + cb * 1024);
  }
  wait_loads();
  __syncthreads();
  // store chunk m: B stick m / (TA / 8), A sticks 8 (m % (TA / 8)) .. + 7
  u32x4 r[kPer];
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const uint32_t m = WAVE_RUNS ? kPer * wave + k : 4 * k + wave, b = m / (TA / 8), ca = m % (TA / 8);
    r[k] = *reinterpret_cast<const u32x4*>(lds + (ca * 8 + lane / 8) * kRowB + b * 128 + (lane % 8) * 16);
  }
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const uint32_t m = WAVE_RUNS ? kPer * wave + k : 4 * k + wave, b = m / (TA / 8), ca = m % (TA / 8);
    store16(rd, v, sd + b * b_sd + ca * 1024, r[k]);
  }
}

// A contiguous copy in 128 KiB blocks through LDS, the stick tiles' pattern
// with the identity mapping: a workgroup's block is kBlockRuns runs of
// kRunB bytes kPitchB apart, the kPitchB / kRunB workgroups of a region of
// kPitchB x kBlockRuns bytes interleaving their runs (as the stick tiles'
// 4 KiB src rows lie 8 KiB apart in a [4096, 4096] fp16 tensor).  1 KiB
// chunks, chunk c loaded (straight into LDS) and stored by wavefront c % 4,
// every load of the workgroup landed (barrier) before its first store: at
// one workgroup per CU the device reads a round's blocks in one phase and
// writes them in the next.  Measured on 32 MiB: 10.9 us, against 11.4 us
// for one contiguous 128 KiB per workgroup and 13.2 us for the vector
// kernel's interleaved loads and stores.
#ifndef SPYRE_BLOCK_RUN
#define SPYRE_BLOCK_RUN 4096
#endif
#ifndef SPYRE_BLOCK_PITCH
#define SPYRE_BLOCK_PITCH 8192
#endif
constexpr int kBlockB = 128 * 1024;
constexpr int kRunB = SPYRE_BLOCK_RUN, kPitchB = SPYRE_BLOCK_PITCH;
constexpr int kBlockRuns = kBlockB / kRunB, kRegionB = kPitchB * kBlockRuns, kRegionBlocks = kPitchB / kRunB;
static_assert(kRunB % 1024 == 0 && kPitchB % kRunB == 0, "whole 1 KiB chunks; runs tile the pitch");

__global__ __launch_bounds__(kThreads) void dma_block_copy_kernel(const char* __restrict__ src_arg,
                                                                  char* __restrict__ dst_arg) {
  constexpr int kPer = kBlockB / 1024 / 4;  // 1 KiB chunks per wavefront
  constexpr int kRunChunks = kRunB / 1024;
  __shared__ __align__(16) char lds[kBlockB];
  const int64_t base = static_cast<int64_t>(blockIdx.x / kRegionBlocks) * kRegionB +
                       static_cast<int64_t>(blockIdx.x % kRegionBlocks) * kRunB;
  const Rsrc rs = make_rsrc(src_arg + base, kRegionB), rd = make_rsrc(dst_arg + base, kRegionB);
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
  const uint32_t v = (threadIdx.x % 64) * 16;
  // chunk c of the block: run c / kRunChunks, 1 KiB piece c % kRunChunks
  auto off = [](uint32_t c) { return (c / kRunChunks) * kPitchB + (c % kRunChunks) * 1024; };
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const uint32_t c = 4 * k + wave;
    load_lds16(rs, v, off(c), lds + c * 1024);
  }
  wait_loads();
  __syncthreads();
  u32x4 r[kPer];
#pragma unroll
  for (int k = 0; k < kPer; ++k) r[k] = *reinterpret_cast<const u32x4*>(lds + (4 * k + wave) * 1024 + v);
#pragma unroll
  for (int k = 0; k < kPer; ++k) store16(rd, v, off(4 * k + wave), r[k]);
}

// A stick tile with a small side: n < 32 rows of T contiguous sticks on one
// side (rows r_stride bytes apart), and the same n x T sticks dense on the
// other, stick (y, x) at (y n + x) x 128 bytes.  Row-major -> sticks when a
// host dim of n sits beside the stick (a batch of 3: the n rows are src,
// the dense block dst), and the way back (D2R).  Per tile, the row side
// moves n runs of T x 128 bytes and the dense side one run of n T x 128.
struct SmallTile {
  uint32_t n, T;      // rows; sticks per row in a tile (a power of two >= 8, n T <= 1024)
  uint32_t r_stride;  // bytes between rows on the row side
  FastDiv div_n;      // stick index -> (y, x)
  uint32_t tc_shift;  // log2(T / 8): 1 KiB chunks per row
};
constexpr int kSmallLdsB = 1024 * 128 + 32 * 128;  // n rows of T sticks + 128 B each, or n T dense sticks

template <bool R2D, int NL, bool POW2>
__global__ __launch_bounds__(kThreads) void dma_stick_small_kernel(const char* __restrict__ src_arg,
                                                                   char* __restrict__ dst_arg, StepNest<NL> nst,
                                                                   SmallTile st) {
  __shared__ __align__(16) char lds[kSmallLdsB];
  const char* src = src_arg;
  char* dst = dst_arg;
  const StepNest<NL> x = read_step(nst, src, dst);
  const uint32_t n = pinned(st.n), T = pinned(st.T), r_stride = pinned(st.r_stride), tcs = pinned(st.tc_shift);
  const FastDiv dn{pinned(st.div_n.d), pinned(st.div_n.mul), pinned(st.div_n.shift)};
  uint32_t so, sd;
  step_offsets<NL, POW2>(x, blockIdx.x, so, sd);
  const Rsrc rs = make_rsrc(src, x.span_s), rd = make_rsrc(dst, x.span_d);
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
  const uint32_t lane = threadIdx.x % 64, v = lane * 16;
  const uint32_t chunks = n * T / 8;  // 1 KiB chunks per tile
  const uint32_t row_b = T * 128 + 128;  // R2D: a padded LDS row
  const uint32_t tc = T / 8;            // chunks per row (1 << tcs)
  constexpr int kMaxPer = 1024 / 8 / 4;  // chunks per wavefront at most
  // Loads: R2D, chunk c = sticks 8 (c % tc) .. + 7 of row c / tc into its
  // LDS row; D2R, dense chunk c into LDS as it lies.
#pragma unroll
  for (int k = 0; k < kMaxPer; ++k) {
    const uint32_t c = 4 * k + wave;
    if (c >= chunks) break;
    if constexpr (R2D) {
      const uint32_t r = c >> tcs, cy = c & (tc - 1);
      load_lds16(rs, v, so + r * r_stride + cy * 1024, lds + r * row_b + cy * 1024);
    } else {
      load_lds16(rs, v, so + c * 1024, lds + c * 1024);
    }
  }
  wait_loads();
  __syncthreads();
  // Stores: R2D, dense chunk m (sticks 8m .. 8m + 7, stick s = (y, x) =
  // (s / n, s % n)) from the LDS rows; D2R, chunk m = sticks 8 (m % tc) ..
  // + 7 of row m / tc from the dense LDS block.
  u32x4 r[kMaxPer];
#pragma unroll
  for (int k = 0; k < kMaxPer; ++k) {
    const uint32_t m = 4 * k + wave;
    if (m >= chunks) break;
    if constexpr (R2D) {
      const uint32_t s = 8 * m + lane / 8, y = fdiv(s, dn), xr = s - y * n;
      r[k] = *reinterpret_cast<const u32x4*>(lds + xr * row_b + y * 128 + (lane % 8) * 16);
    } else {
      const uint32_t row = m >> tcs, y = (m & (tc - 1)) * 8 + lane / 8;
      r[k] = *reinterpret_cast<const u32x4*>(lds + (y * n + row) * 128 + (lane % 8) * 16);
    }
  }
#pragma unroll
  for (int k = 0; k < kMaxPer; ++k) {
    const uint32_t m = 4 * k + wave;
    if (m >= chunks) break;
    if constexpr (R2D)
      store16(rd, v, sd + m * 1024, r[k]);
    else
      store16(rd, v, sd + (m >> tcs) * r_stride + (m & (tc - 1)) * 1024, r[k]);
  }
}

// Compute units of the current device, cached per device; 0 if the runtime
// cannot say.
int dma_device_cus() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  int v = cache[dev].load(std::memory_order_relaxed);
  if (v > 0) return v;
  if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) return 0;
  cache[dev].store(v, std::memory_order_relaxed);
  return v;
}

// Transpose nest: loop A is unit-stride in src, loop B unit-stride in dst.
// Blocks of N x N elements (N = 16 / ESZ); a wavefront covers 8 x 8 blocks.
struct TNest {
  uint32_t na, nb;            // blocks along A and B
  FastDiv tiles_a, tiles_b;   // wave tiles along A and B
  int nouter;
  FastDiv outer[kMaxLoops];
  int64_t ss[kMaxLoops], sd[kMaxLoops];
  int64_t a_sd;               // dst stride of A (bytes)
  int64_t b_ss;               // src stride of B (bytes)
  int64_t off_s, off_d;
  uint32_t tiles;             // total 64x64 (8x8-block) tiles
};

template <int ESZ>
__device__ __forceinline__ void transpose_block(u32x4 (&r)[16 / ESZ], u32x4 (&o)[16 / ESZ]);

template <>
__device__ __forceinline__ void transpose_block<2>(u32x4 (&r)[8], u32x4 (&o)[8]) {
  spyre_hip::transpose8x8_b16(r, o);
}

template <>
__device__ __forceinline__ void transpose_block<4>(u32x4 (&r)[4], u32x4 (&o)[4]) {
  const uint32_t* w = reinterpret_cast<const uint32_t*>(r);
  uint32_t* x = reinterpret_cast<uint32_t*>(o);
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b) x[a * 4 + b] = w[b * 4 + a];
}

// Moves a wavefront's kTransposeTiles tiles: every load first, then the
// register transposes and the stores.  GUARDED predicates each tile on ok[t]
// (edge waves); whole waves run unpredicated, so no wait separates one
// tile's stores from the next.
template <int ESZ, bool GUARDED>
__device__ __forceinline__ void transpose_tiles(const char* __restrict__ src, char* __restrict__ dst,
                                                const TNest& n, const int64_t (&so)[kTransposeTiles],
                                                const int64_t (&sd)[kTransposeTiles],
                                                const bool (&ok)[kTransposeTiles]) {
  constexpr int N = 16 / ESZ;
  u32x4 r[kTransposeTiles][N];
#pragma unroll
  for (int t = 0; t < kTransposeTiles; ++t)
    if (!GUARDED || ok[t]) {
#pragma unroll
      for (int b = 0; b < N; ++b)
        r[t][b] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + so[t] + b * n.b_ss));
    }
  __builtin_amdgcn_sched_barrier(0);  // keep every load ahead of the stores
#pragma unroll
  for (int t = 0; t < kTransposeTiles; ++t)
    if (!GUARDED || ok[t]) {
      u32x4 o[N];
      transpose_block<ESZ>(r[t], o);
#pragma unroll
      for (int a = 0; a < N; ++a)
        __builtin_nontemporal_store(o[a], reinterpret_cast<u32x4*>(dst + sd[t] + a * n.a_sd));
    }
}

// Wavefront w transposes tiles kTransposeTiles * w + t.  NOUT is the number
// of outer loops when it is small (straight-line index decomposition), -1
// for any count.
template <int ESZ, int NOUT>
__global__ __launch_bounds__(kThreads) void dma_transpose_kernel(const char* __restrict__ src,
                                                                 char* __restrict__ dst, TNest n) {
  constexpr int N = 16 / ESZ;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(blockIdx.x * (kThreads / 64) + threadIdx.x / 64);
  const uint32_t lane = threadIdx.x % 64;
  int64_t so[kTransposeTiles], sd[kTransposeTiles];
  bool ok[kTransposeTiles];
  bool whole = true;  // wave-uniform: every tile in range and whole
#pragma unroll
  for (int t = 0; t < kTransposeTiles; ++t) {
    const uint32_t tile = wave * kTransposeTiles + t;
    uint32_t q = fdiv(tile, n.tiles_a);
    const uint32_t ta = tile - q * n.tiles_a.d;
    uint32_t q2 = fdiv(q, n.tiles_b);
    const uint32_t tb = q - q2 * n.tiles_b.d;
    q = q2;
    int64_t s = n.off_s, d = n.off_d;
    const int nout = NOUT >= 0 ? NOUT : n.nouter;
#pragma unroll
    for (int k = 0; k < (NOUT >= 0 ? NOUT : kMaxLoops); ++k) {
      if (NOUT < 0 && k >= nout) break;
      q2 = fdiv(q, n.outer[k]);
      const int64_t c = q - q2 * n.outer[k].d;
      s += c * n.ss[k];
      d += c * n.sd[k];
      q = q2;
    }
    whole = whole && tile < n.tiles && ta * 8 + 8 <= n.na && tb * 8 + 8 <= n.nb;
    const uint32_t ablk = ta * 8 + lane % 8;
    const uint32_t bblk = tb * 8 + lane / 8;
    ok[t] = tile < n.tiles && ablk < n.na && bblk < n.nb;
    so[t] = s + static_cast<int64_t>(ablk) * 16 + static_cast<int64_t>(bblk) * N * n.b_ss;
    sd[t] = d + static_cast<int64_t>(bblk) * 16 + static_cast<int64_t>(ablk) * N * n.a_sd;
  }
  if (whole)
    transpose_tiles<ESZ, false>(src, dst, n, so, sd, ok);
  else
    transpose_tiles<ESZ, true>(src, dst, n, so, sd, ok);
}

// 2-byte transposes through LDS: a wavefront's kTransposeTiles 64 x 64 tiles
// travel from memory straight into LDS (each load instruction: 8 B rows of
// one tile, 128 contiguous bytes each), then every lane reads its 8 x 8
// block of each tile (row r at (r / 8) * 1152 + (r % 8) * 128, 8-row groups
// padded so that the eight groups a read touches fall in different bank
// halves), transposes it in registers and stores as dma_transpose_kernel.
// Measured on fp16 [4096, 4096] transpose-restick (tiles 8 KiB contiguous
// on both sides): 11.2 -> 10.9 us against the register-only kernel.
constexpr int kTrGroupB = 8 * 128 + 128;
constexpr int kTrTileB = 8 * kTrGroupB;

// NOUT: the number of outer loops, or -1 for any count (generic path).
// The prologue is straight-line code ending in one register barrier over
// everything the loads and stores use, so every argument is read in one
// batch at entry and all four tiles' offsets exist before the first load.
// (Arguments read in rounds -- here the loop sizes after the tile counts --
// each cost a memory round trip before the first load: measured 12.1 ->
// 11.1 us on the [4096, 4096] transpose-restick.)
// The arguments of a transpose nest with NOUT (0-3) outer loops, read into
// scalar registers by one statement: every read is issued at entry and
// waited for once.
template <int NOUT>
struct TArgs {
  uint32_t na, nb, tiles;
  FastDiv da, db, od[NOUT > 0 ? NOUT : 1];
  int64_t ss[NOUT > 0 ? NOUT : 1], sd[NOUT > 0 ? NOUT : 1];
  int64_t a_sd, b_ss, off_s, off_d;
};

#define SPYRE_PIN_DIV(f) "+s"(f.d), "+s"(f.mul), "+s"(f.shift)
template <int NOUT>
__device__ __forceinline__ TArgs<NOUT> read_targs(const TNest& n) {
  TArgs<NOUT> x;
  x.na = n.na;
  x.nb = n.nb;
  x.tiles = n.tiles;
  x.da = n.tiles_a;
  x.db = n.tiles_b;
  for (int k = 0; k < (NOUT > 0 ? NOUT : 1); ++k) {
    x.od[k] = n.outer[k];
    x.ss[k] = n.ss[k];
    x.sd[k] = n.sd[k];
  }
  x.a_sd = n.a_sd;
  x.b_ss = n.b_ss;
  x.off_s = n.off_s;
  x.off_d = n.off_d;
  if constexpr (NOUT <= 1) {
    asm volatile("" : "+s"(x.na), "+s"(x.nb), "+s"(x.tiles), SPYRE_PIN_DIV(x.da), SPYRE_PIN_DIV(x.db),
                 SPYRE_PIN_DIV(x.od[0]), "+s"(x.ss[0]), "+s"(x.sd[0]), "+s"(x.a_sd), "+s"(x.b_ss), "+s"(x.off_s),
                 "+s"(x.off_d));
  } else if constexpr (NOUT == 2) {
    asm volatile("" : "+s"(x.na), "+s"(x.nb), "+s"(x.tiles), SPYRE_PIN_DIV(x.da), SPYRE_PIN_DIV(x.db),
                 SPYRE_PIN_DIV(x.od[0]), SPYRE_PIN_DIV(x.od[1]), "+s"(x.ss[0]), "+s"(x.sd[0]), "+s"(x.ss[1]),
                 "+s"(x.sd[1]), "+s"(x.a_sd), "+s"(x.b_ss), "+s"(x.off_s), "+s"(x.off_d));
  } else {
    static_assert(NOUT == 3, "read_targs serves 0-3 outer loops");
    asm volatile("" : "+s"(x.na), "+s"(x.nb), "+s"(x.tiles), SPYRE_PIN_DIV(x.da), SPYRE_PIN_DIV(x.db),
                 SPYRE_PIN_DIV(x.od[0]), SPYRE_PIN_DIV(x.od[1]), SPYRE_PIN_DIV(x.od[2]), "+s"(x.ss[0]),
                 "+s"(x.sd[0]), "+s"(x.ss[1]), "+s"(x.sd[1]), "+s"(x.ss[2]), "+s"(x.sd[2]), "+s"(x.a_sd),
                 "+s"(x.b_ss), "+s"(x.off_s), "+s"(x.off_d));
  }
  return x;
}
#undef SPYRE_PIN_DIV

// NOUT: the number of outer loops (0-3).  Every argument is read in one
// batch at entry (read_targs); each tile's loads are issued as soon as its
// offsets are known.  (Arguments read in rounds -- the loop sizes after the
// tile counts -- each cost a memory round trip before the first load, and a
// prologue that computed all four tiles before loading delayed the chip's
// first reads: 12.1 -> 11.2 us on the [4096, 4096] transpose-restick.)
// BUF: the loads use a per-tile buffer descriptor (64 rows of b_ss fit
// 32-bit offsets, checked on the host).
template <int NOUT, bool BUF>
__global__ __launch_bounds__(kThreads) void dma_transpose_lds_kernel(const char* __restrict__ src,
                                                                     char* __restrict__ dst, TNest n) {
  __shared__ __align__(16) char lds[kThreads / 64 * kTransposeTiles * kTrTileB];
  const TArgs<NOUT> x = read_targs<NOUT>(n);
  const uint32_t wv = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
  const uint32_t wave = blockIdx.x * (kThreads / 64) + wv;
  const uint32_t lane = threadIdx.x % 64;
  const uint32_t na = x.na, nb = x.nb;
  const int64_t b_ss = x.b_ss, a_sd = x.a_sd;
  char* wl = lds + wv * kTransposeTiles * kTrTileB;
  int64_t sd[kTransposeTiles];
  uint32_t ta[kTransposeTiles], tb[kTransposeTiles];
  bool in[kTransposeTiles], whole[kTransposeTiles];
#pragma unroll
  for (int t = 0; t < kTransposeTiles; ++t) {
    const uint32_t tile = wave * kTransposeTiles + t;
    uint32_t q = fdiv(tile, x.da);
    ta[t] = tile - q * x.da.d;
    uint32_t q2 = fdiv(q, x.db);
    tb[t] = q - q2 * x.db.d;
    q = q2;
    int64_t so = x.off_s, d = x.off_d;
#pragma unroll
    for (int k = 0; k < NOUT; ++k) {
      q2 = fdiv(q, x.od[k]);
      const int64_t c = q - q2 * x.od[k].d;
      so += c * x.ss[k];
      d += c * x.sd[k];
      q = q2;
    }
    sd[t] = d;
    in[t] = tile < x.tiles;
    whole[t] = in[t] && ta[t] * 8 + 8 <= na && tb[t] * 8 + 8 <= nb;  // wave-uniform
    // Loads: group g is src rows 8 (8 tb + g) .. + 7 (this lane: row + lane
    // / 8) of A block 8 ta + lane % 8, into LDS group g.
    const uint32_t ablk = ta[t] * 8 + lane % 8;
    const char* tbase = src + so + static_cast<int64_t>(ta[t]) * 128 + static_cast<int64_t>(64 * tb[t]) * b_ss;
    const Rsrc rs = make_rsrc(tbase);
#pragma unroll
    for (int g = 0; g < 8; ++g) {
      char* l = wl + t * kTrTileB + g * kTrGroupB;
      const bool ok = whole[t] | (in[t] & (ablk < na) & (tb[t] * 8 + g < nb));
      if (BUF) {
        // a lane outside the nest gets an offset past the descriptor's
        // range: the load is skipped (its LDS slot feeds no store), no branch
        const uint32_t off = (lane % 8) * 16 + static_cast<uint32_t>(8 * g + lane / 8) * static_cast<uint32_t>(b_ss);
        load_lds16(rs, ok ? off : kBufOob, l);
      } else if (ok) {
        load_lds16(tbase + (lane % 8) * 16 + static_cast<int64_t>(8 * g + lane / 8) * b_ss, l);
      }
    }
  }
  wait_loads();
  // This lane's block: A block 8 ta + lane % 8, B block 8 tb + lane / 8.
  const uint32_t la = lane % 8, lb = lane / 8;
#pragma unroll
  for (int t = 0; t < kTransposeTiles; ++t) {
    u32x4 r[8], o[8];
#pragma unroll
    for (int b = 0; b < 8; ++b)
      r[b] = *reinterpret_cast<const u32x4*>(wl + t * kTrTileB + lb * kTrGroupB + b * 128 + la * 16);
    spyre_hip::transpose8x8_b16(r, o);
    const uint32_t ablk = ta[t] * 8 + la, sb = tb[t] * 8 + lb;
    if (whole[t] || (in[t] && ablk < na && sb < nb)) {
      char* dp = dst + sd[t] + static_cast<int64_t>(sb) * 16 + static_cast<int64_t>(ablk) * 8 * a_sd;
#pragma unroll
      for (int a = 0; a < 8; ++a) __builtin_nontemporal_store(o[a], reinterpret_cast<u32x4*>(dp + a * a_sd));
    }
  }
}

// The stepped form of dma_transpose_lds_kernel, for nests whose tiles are
// all whole, whose tile count is a multiple of kTransposeTiles, whose src
// and dst spans fit one buffer descriptor each, and whose tiles of one
// wavefront lie along one loop (all checked on the host).  The tile loops
// -- A tiles, B tiles and the outer loops, those longer than one, the first
// of them the one a wavefront's tiles step along -- are decomposed once per
// wavefront in 32-bit arithmetic (shift and mask when every loop length is
// a power of two), each load and store adds a scalar offset to a per-lane
// one, and nothing is predicated.  The prologue before the first load is
// what this saves: the general kernel decomposes every tile with 64-bit
// multiply-adds, ~80 scalar instructions between one tile's loads and the
// next.
template <int NL, bool POW2>
__global__ __launch_bounds__(kThreads) void dma_transpose_step_kernel(const char* __restrict__ src_arg,
                                                                      char* __restrict__ dst_arg, StepNest<NL> n) {
  __shared__ __align__(16) char lds[kThreads / 64 * kTransposeTiles * kTrTileB];
  const char* src = src_arg;
  char* dst = dst_arg;
  const StepNest<NL> x = read_step(n, src, dst);
  const uint32_t b_ss = x.s1, a_sd = x.s2;
  const uint32_t wv = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
  const uint32_t tile = (blockIdx.x * (kThreads / 64) + wv) * kTransposeTiles;
  if (tile >= x.count) return;  // wave-uniform; no barrier follows
  uint32_t so, sd;
  step_offsets<NL, POW2>(x, tile, so, sd);
  const Rsrc rs = make_rsrc(src, x.span_s), rd = make_rsrc(dst, x.span_d);
  const uint32_t lane = threadIdx.x % 64, la = lane % 8, lb = lane / 8;
  char* wl = lds + wv * kTransposeTiles * kTrTileB;
  // load group g of a tile: its src rows 8 g + lb, bytes la * 16 of each
  const uint32_t vs = la * 16 + lb * b_ss;
#pragma unroll
  for (int t = 0; t < kTransposeTiles; ++t)
#pragma unroll
    for (int g = 0; g < 8; ++g)
      load_lds16(rs, vs, so + t * x.ss[0] + 8 * g * b_ss, wl + t * kTrTileB + g * kTrGroupB);
  wait_loads();
  // store a of this lane's block: dst row 8 la + a of the tile, bytes lb * 16
  const uint32_t vd = lb * 16 + la * 8 * a_sd;
#pragma unroll
  for (int t = 0; t < kTransposeTiles; ++t) {
    u32x4 r[8], o[8];
#pragma unroll
    for (int b = 0; b < 8; ++b)
      r[b] = *reinterpret_cast<const u32x4*>(wl + t * kTrTileB + lb * kTrGroupB + b * 128 + la * 16);
    spyre_hip::transpose8x8_b16(r, o);
#pragma unroll
    for (int a = 0; a < 8; ++a) store16(rd, vd, sd + t * x.sd[0] + a * a_sd, o[a]);
  }
}

template <int ESZ>
__global__ __launch_bounds__(kThreads) void dma_scalar_kernel(const char* __restrict__ src,
                                                              char* __restrict__ dst, Nest n) {
  using T = typename VecT<ESZ>::T;
  const uint32_t i = blockIdx.x * kThreads + threadIdx.x;
  if (i >= n.total) return;
  int64_t so, sd;
  item_offsets(n, i, so, sd);
  *reinterpret_cast<T*>(dst + sd) = *reinterpret_cast<const T*>(src + so);
}

struct Loop {
  int64_t size, ss, sd;  // strides in bytes
};

// Drops unit loops and merges loops that are contiguous on both sides.
std::vector<Loop> normalise(const spyre_stride_info& info, int esz) {
  std::vector<Loop> l;
  for (int q = 0; q < info.rank; ++q)
    if (info.size[q] != 1) l.push_back({info.size[q], info.stride_src[q] * esz, info.stride_dst[q] * esz});
  std::stable_sort(l.begin(), l.end(), [](const Loop& a, const Loop& b) {
    return a.sd != b.sd ? a.sd < b.sd : a.ss < b.ss;
  });
  std::vector<Loop> m;
  for (const Loop& x : l) {
    if (!m.empty() && x.ss == m.back().ss * m.back().size && x.sd == m.back().sd * m.back().size)
      m.back().size *= x.size;
    else
      m.push_back(x);
  }
  return m;
}

bool aligned(const void* p, int64_t v) { return reinterpret_cast<uintptr_t>(p) % v == 0; }

template <int NL>
StepNest<NL> make_step(const std::vector<Loop>& tl, int64_t count, int64_t off_s, int64_t off_d, int64_t span_s,
                       int64_t span_d, int64_t s1, int64_t s2) {
  StepNest<NL> x{};
  x.count = static_cast<uint32_t>(count);
  x.off_s = static_cast<uint32_t>(off_s);
  x.off_d = static_cast<uint32_t>(off_d);
  x.span_s = static_cast<uint32_t>(span_s);
  x.span_d = static_cast<uint32_t>(span_d);
  x.s1 = static_cast<uint32_t>(s1);
  x.s2 = static_cast<uint32_t>(s2);
  for (int k = 0; k < NL; ++k) {
    x.loop[k] = make_fastdiv(static_cast<uint32_t>(tl[k].size));
    x.ss[k] = static_cast<uint32_t>(tl[k].ss);
    x.sd[k] = static_cast<uint32_t>(tl[k].sd);
  }
  return x;
}

// The span checks of a stepped nest: strides non-negative, every loop
// length a power of two or not, and the byte extent of each side, given the
// extent of one tile.
struct StepSpan {
  bool ok = true, pow2 = true;
  int64_t span_s = 0, span_d = 0;
};
StepSpan step_span(const std::vector<Loop>& tl, int64_t off_s, int64_t off_d, int64_t tile_s, int64_t tile_d) {
  StepSpan r;
  r.ok = !tl.empty() && static_cast<int>(tl.size()) <= kStepLoops && off_s >= 0 && off_d >= 0;
  r.span_s = off_s + tile_s;
  r.span_d = off_d + tile_d;
  for (const Loop& l : tl) {
    r.ok = r.ok && l.ss >= 0 && l.sd >= 0;
    r.span_s += (l.size - 1) * l.ss;
    r.span_d += (l.size - 1) * l.sd;
    r.pow2 = r.pow2 && (l.size & (l.size - 1)) == 0;
  }
  r.ok = r.ok && r.span_s <= int64_t{kBufRange} && r.span_d <= int64_t{kBufRange};
  return r;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  SPYRE_REQUIRE(e == hipSuccess, SPYRE_EHIP, "%s launch failed: %s", what, hipGetErrorString(e));
  return SPYRE_OK;
}

// Fills a Nest whose inner loop is `inner` (already scaled to `vb`-byte items)
// and whose outer loops are `outer`; splits the launch along the outermost
// loop when the item count exceeds 2^31.
template <typename Launch>
int launch_nest(const Loop& inner, std::vector<Loop> outer, int64_t off_s, int64_t off_d,
                int64_t item_bytes, Launch&& launch) {
  int64_t per = inner.size;
  for (const Loop& o : outer) per *= o.size;
  if (per == 0) return SPYRE_OK;
  const int64_t kMaxItems = int64_t{1} << 30;
  if (per > kMaxItems) {
    SPYRE_REQUIRE(!outer.empty(), SPYRE_EUNSUPPORTED, "inner loop too long");
    Loop top = outer.back();
    outer.pop_back();
    const int64_t slice = per / top.size;
    SPYRE_REQUIRE(slice <= kMaxItems, SPYRE_EUNSUPPORTED, "loop nest too large");
    const int64_t step = std::max<int64_t>(1, kMaxItems / slice);
    for (int64_t c = 0; c < top.size; c += step) {
      std::vector<Loop> o2 = outer;
      o2.push_back({std::min(step, top.size - c), top.ss, top.sd});
      const int rc = launch_nest(inner, o2, off_s + c * top.ss, off_d + c * top.sd, item_bytes, launch);
      if (rc != SPYRE_OK) return rc;
    }
    return SPYRE_OK;
  }
  Nest n{};
  n.nouter = static_cast<int>(outer.size());
  n.inner = make_fastdiv(static_cast<uint32_t>(inner.size));
  n.inner_ss = inner.ss;
  n.inner_sd = inner.sd;
  for (size_t k = 0; k < outer.size(); ++k) {
    n.outer[k] = make_fastdiv(static_cast<uint32_t>(outer[k].size));
    n.ss[k] = outer[k].ss;
    n.sd[k] = outer[k].sd;
  }
  n.off_s = off_s;
  n.off_d = off_d;
  n.total = static_cast<uint32_t>(per);
  (void)item_bytes;
  return launch(n);
}

int run_info(const char* src, char* dst, int esz, const spyre_stride_info& info, hipStream_t st) {
  for (int q = 0; q < info.rank; ++q)
    if (info.size[q] == 0) return SPYRE_OK;
  std::vector<Loop> loops = normalise(info, esz);
  const int64_t off_s = info.offset_src * esz, off_d = info.offset_dst * esz;
  if (loops.empty()) loops.push_back({1, esz, esz});
  SPYRE_REQUIRE(loops.size() <= static_cast<size_t>(kMaxLoops), SPYRE_EUNSUPPORTED,
                "too many loops");

  // vec: a loop contiguous on both sides.
  int vi = -1;
  for (size_t k = 0; k < loops.size(); ++k)
    if (loops[k].ss == esz && loops[k].sd == esz) vi = static_cast<int>(k);
  if (vi >= 0) {
    std::vector<Loop> outer;
    for (size_t k = 0; k < loops.size(); ++k)
      if (static_cast<int>(k) != vi) outer.push_back(loops[k]);
    const int64_t row = loops[vi].size * esz;
    int vb = 16;
    auto fits = [&](int b) {
      if (b < esz || row % b || off_s % b || off_d % b || !aligned(src, b) || !aligned(dst, b))
        return false;
      for (const Loop& o : outer)
        if (o.ss % b || o.sd % b) return false;
      return true;
    };
    while (vb > esz && !fits(vb)) vb /= 2;
    if (!fits(vb)) vb = esz;
    if (vb == 16 && outer.empty() && row >= kRegionB) {
      // one contiguous run: whole regions of 128 KiB blocks through LDS,
      // the tail (a multiple of 16 B) by the vector kernel
      const int64_t regions = row / kRegionB;
      const int64_t per_launch = (int64_t{1} << 30) / kRegionBlocks;
      for (int64_t r0 = 0; r0 < regions; r0 += per_launch) {
        const int64_t nr = std::min<int64_t>(regions - r0, per_launch);
        dma_block_copy_kernel<<<dim3(static_cast<uint32_t>(nr * kRegionBlocks)), kThreads, 0, st>>>(
            src + off_s + r0 * kRegionB, dst + off_d + r0 * kRegionB);
        const int rc = check_launch("dma_block_copy_kernel");
        if (rc != SPYRE_OK) return rc;
      }
      const int64_t done = regions * kRegionB;
      if (done == row) return SPYRE_OK;
      spyre_stride_info tail = info;
      tail.rank = 1;
      tail.size[0] = (row - done) / esz;
      tail.stride_src[0] = tail.stride_dst[0] = 1;
      tail.offset_src = info.offset_src + done / esz;
      tail.offset_dst = info.offset_dst + done / esz;
      return run_info(src, dst, esz, tail, st);
    }
    if (vb == 16 && row == 128) {
      // stick tile: loop A continues the stick in dst, loop B in src.
      int ai = -1, bi = -1;
      for (size_t k = 0; k < outer.size(); ++k) {
        if (outer[k].sd == row && ai < 0) ai = static_cast<int>(k);
        else if (outer[k].ss == row && bi < 0) bi = static_cast<int>(k);
      }
      // A narrow A or B loop (8, 16 or 24 sticks: a batch dim of 8 above the
      // stick, a KV cache of 8 sequences) takes 8 x 128 or 16 x 64 stick
      // tiles (128 x 8 or 64 x 16 for B), whole tiles only.
      auto narrow = [](int64_t size) { return size < kTileSticks && size % 8 == 0; };
      const bool wide_a = ai >= 0 && outer[ai].size >= kTileSticks, wide_b = bi >= 0 && outer[bi].size >= kTileSticks;
      const bool narrow_a = wide_b && ai >= 0 && narrow(outer[ai].size);
      const bool narrow_b = wide_a && bi >= 0 && narrow(outer[bi].size);
      if ((wide_a && wide_b) || narrow_a || narrow_b) {
        SNest n{};
        n.na = static_cast<uint32_t>(outer[ai].size);
        n.nb = static_cast<uint32_t>(outer[bi].size);
        // Tile shape: 32 x 32 sticks; 64 x 16 when the 64 A sticks are a
        // whole dst row that B continues (sticks -> row-major of 8 KiB
        // rows): a workgroup then writes 128 KiB of contiguous dst and each
        // wavefront a quarter of it (measured: 11.4 -> 11.0 us on fp16
        // [4096, 4096]; the 32 x 32 tile with interleaved stores is best for
        // row-major -> sticks).
        const bool tall = n.na == 64 && outer[bi].sd == 64 * row;
        const uint32_t TA = narrow_a   ? (n.na == 16 ? 16 : 8)
                            : narrow_b ? (n.nb == 16 ? 64 : 128)
                            : tall     ? 64
                                       : kTileSticks;
        const uint32_t TB = 1024 / TA;
        const uint32_t ta = (n.na + TA - 1) / TA;
        const uint32_t tb = (n.nb + TB - 1) / TB;
        int64_t tiles = int64_t{ta} * tb;
        // Consecutive workgroups step along B, the loop contiguous in src:
        // neighbouring tiles read neighbouring memory (measured: ~1 %
        // faster than stepping along A on row-major -> sticks).
        n.b_first = 1;
        n.tiles_x = make_fastdiv(n.b_first ? tb : ta);
        n.tiles_y = make_fastdiv(n.b_first ? ta : tb);
        n.a_ss = outer[ai].ss;
        n.b_sd = outer[bi].sd;
        n.off_s = off_s;
        n.off_d = off_d;
        for (size_t k = 0; k < outer.size(); ++k) {
          if (static_cast<int>(k) == ai || static_cast<int>(k) == bi) continue;
          n.outer[n.nouter] = make_fastdiv(static_cast<uint32_t>(outer[k].size));
          n.ss[n.nouter] = outer[k].ss;
          n.sd[n.nouter] = outer[k].sd;
          ++n.nouter;
          tiles *= outer[k].size;
        }
        // Stepped kernel: whole tiles, spans within a descriptor.
        std::vector<Loop> tl;
        if (tb > 1) tl.push_back({tb, int64_t{TB} * row, int64_t{TB} * n.b_sd});
        if (ta > 1) tl.push_back({ta, int64_t{TA} * n.a_ss, int64_t{TA} * row});
        for (int k = 0; k < n.nouter; ++k) tl.push_back({n.outer[k].d, n.ss[k], n.sd[k]});
        const StepSpan sp = step_span(tl, off_s, off_d, (int64_t{TA} - 1) * n.a_ss + int64_t{TB} * row,
                                      (int64_t{TB} - 1) * n.b_sd + int64_t{TA} * row);
        if (sp.ok && n.na % TA == 0 && n.nb % TB == 0 && n.a_ss > 0 && n.b_sd > 0 && tiles < (int64_t{1} << 31)) {
          const dim3 grid(static_cast<uint32_t>(tiles));
          auto step_go = [&](auto nl_c) {
            constexpr int NL = decltype(nl_c)::value;
            const StepNest<NL> x = make_step<NL>(tl, tiles, off_s, off_d, sp.span_s, sp.span_d, n.a_ss, n.b_sd);
            if (narrow_a && TA == 8 && sp.pow2)
              dma_stick_step_kernel<8, 128, true, NL, true><<<grid, kThreads, 0, st>>>(src, dst, x);
            else if (narrow_a && TA == 8)
              dma_stick_step_kernel<8, 128, true, NL, false><<<grid, kThreads, 0, st>>>(src, dst, x);
            else if (narrow_a && sp.pow2)
              dma_stick_step_kernel<16, 64, true, NL, true><<<grid, kThreads, 0, st>>>(src, dst, x);
            else if (narrow_a)
              dma_stick_step_kernel<16, 64, true, NL, false><<<grid, kThreads, 0, st>>>(src, dst, x);
            else if (TA == 128 && sp.pow2)
              dma_stick_step_kernel<128, 8, true, NL, true><<<grid, kThreads, 0, st>>>(src, dst, x);
            else if (TA == 128)
              dma_stick_step_kernel<128, 8, true, NL, false><<<grid, kThreads, 0, st>>>(src, dst, x);
            else if (TA == 64 && sp.pow2)
              dma_stick_step_kernel<64, 16, true, NL, true><<<grid, kThreads, 0, st>>>(src, dst, x);
            else if (TA == 64)
              dma_stick_step_kernel<64, 16, true, NL, false><<<grid, kThreads, 0, st>>>(src, dst, x);
            else if (sp.pow2)
              dma_stick_step_kernel<32, 32, false, NL, true><<<grid, kThreads, 0, st>>>(src, dst, x);
            else
              dma_stick_step_kernel<32, 32, false, NL, false><<<grid, kThreads, 0, st>>>(src, dst, x);
          };
          switch (tl.size()) {
            case 1: step_go(std::integral_constant<int, 1>{}); break;
            case 2: step_go(std::integral_constant<int, 2>{}); break;
            case 3: step_go(std::integral_constant<int, 3>{}); break;
            default: step_go(std::integral_constant<int, 4>{}); break;
          }
          return check_launch("dma_stick_step_kernel");
        }
        if (!narrow_a && !narrow_b && tiles < (int64_t{1} << 31)) {  // narrow nests with edges: the vec kernel
          const dim3 grid(static_cast<uint32_t>(tiles));
          // 32-bit buffer offsets when a tile's spans fit them
          const bool buf = (int64_t{TA} - 1) * n.a_ss + int64_t{TB} * row < int64_t{kBufRange} &&
                           (int64_t{TB} - 1) * n.b_sd + int64_t{TA} * row < int64_t{kBufRange};
          if (tall && buf)
            dma_stick_tile_kernel<64, 16, true, true><<<grid, kThreads, 0, st>>>(src, dst, n);
          else if (tall)
            dma_stick_tile_kernel<64, 16, true, false><<<grid, kThreads, 0, st>>>(src, dst, n);
          else if (buf)
            dma_stick_tile_kernel<32, 32, false, true><<<grid, kThreads, 0, st>>>(src, dst, n);
          else
            dma_stick_tile_kernel<32, 32, false, false><<<grid, kThreads, 0, st>>>(src, dst, n);
          return check_launch("dma_stick_tile_kernel");
        }
      }
      // A small side (n < 32 sticks, no multiple of 8: a batch of 3 beside
      // the stick) whose other side is dense over both loops: n runs of T
      // sticks against one dense run per tile (dma_stick_small_kernel).
      const bool small_a = ai >= 0 && bi >= 0 && outer[ai].size < kTileSticks && outer[ai].size % 8 != 0 &&
                           outer[bi].sd == outer[ai].size * row;
      const bool small_b = !small_a && ai >= 0 && bi >= 0 && outer[bi].size < kTileSticks &&
                           outer[bi].size % 8 != 0 && outer[ai].ss == outer[bi].size * row;
      if (small_a || small_b) {
        const int64_t ns = small_a ? outer[ai].size : outer[bi].size;    // rows
        const int64_t nl = small_a ? outer[bi].size : outer[ai].size;    // sticks along a row
        const int64_t rs = small_a ? outer[ai].ss : outer[bi].sd;        // row stride, row side
        int64_t T = 8;
        while (ns * T * 2 <= 1024 && nl % (T * 2) == 0) T *= 2;
        // Smaller tiles while the grid would leave compute units idle (a
        // 16 MiB tensor in 128 KiB tiles fills half the device).
        int64_t others = 1;
        for (size_t k = 0; k < outer.size(); ++k)
          if (static_cast<int>(k) != ai && static_cast<int>(k) != bi) others *= outer[k].size;
        const int64_t cus = dma_device_cus() > 0 ? dma_device_cus() : 256;
        while (T > 8 && nl / T * others < cus) T /= 2;
        std::vector<Loop> tl;
        if (nl / T > 1) tl.push_back({nl / T, small_a ? T * row : ns * T * row, small_a ? ns * T * row : T * row});
        int64_t tiles = nl / T;
        for (size_t k = 0; k < outer.size(); ++k) {
          if (static_cast<int>(k) == ai || static_cast<int>(k) == bi) continue;
          tl.push_back(outer[k]);
          tiles *= outer[k].size;
        }
        const int64_t tile_s = small_a ? (ns - 1) * rs + T * row : ns * T * row;
        const int64_t tile_d = small_a ? ns * T * row : (ns - 1) * rs + T * row;
        const StepSpan sp = step_span(tl, off_s, off_d, tile_s, tile_d);
        if (nl % T == 0 && sp.ok && rs > 0 && tiles < (int64_t{1} << 31)) {
          uint32_t tcs = 0;
          while ((int64_t{8} << tcs) < T) ++tcs;
          const SmallTile smt{static_cast<uint32_t>(ns), static_cast<uint32_t>(T), static_cast<uint32_t>(rs),
                              make_fastdiv(static_cast<uint32_t>(ns)), tcs};
          const dim3 grid(static_cast<uint32_t>(tiles));
          auto small_go = [&](auto nl_c) {
            constexpr int NL = decltype(nl_c)::value;
            const StepNest<NL> x = make_step<NL>(tl, tiles, off_s, off_d, sp.span_s, sp.span_d, 0, 0);
            if (small_a && sp.pow2)
              dma_stick_small_kernel<true, NL, true><<<grid, kThreads, 0, st>>>(src, dst, x, smt);
            else if (small_a)
              dma_stick_small_kernel<true, NL, false><<<grid, kThreads, 0, st>>>(src, dst, x, smt);
            else if (sp.pow2)
              dma_stick_small_kernel<false, NL, true><<<grid, kThreads, 0, st>>>(src, dst, x, smt);
            else
              dma_stick_small_kernel<false, NL, false><<<grid, kThreads, 0, st>>>(src, dst, x, smt);
          };
          switch (tl.size()) {
            case 1: small_go(std::integral_constant<int, 1>{}); break;
            case 2: small_go(std::integral_constant<int, 2>{}); break;
            case 3: small_go(std::integral_constant<int, 3>{}); break;
            default: small_go(std::integral_constant<int, 4>{}); break;
          }
          return check_launch("dma_stick_small_kernel");
        }
      }
    }
    const Loop inner{row / vb, vb, vb};
    return launch_nest(inner, outer, off_s, off_d, vb, [&](const Nest& n) {
      const dim3 grid((n.total + kThreads * kItems - 1) / (kThreads * kItems));
      switch (vb) {
        case 16: dma_vec_kernel<16, kItems><<<grid, kThreads, 0, st>>>(src, dst, n); break;
        case 8: dma_vec_kernel<8, kItems><<<grid, kThreads, 0, st>>>(src, dst, n); break;
        case 4: dma_vec_kernel<4, kItems><<<grid, kThreads, 0, st>>>(src, dst, n); break;
        case 2: dma_vec_kernel<2, kItems><<<grid, kThreads, 0, st>>>(src, dst, n); break;
        default: dma_vec_kernel<1, kItems><<<grid, kThreads, 0, st>>>(src, dst, n); break;
      }
      return check_launch("dma_vec_kernel");
    });
  }

  // transpose: loop A unit-stride in src, loop B unit-stride in dst.
  int ai = -1, bi = -1;
  for (size_t k = 0; k < loops.size(); ++k) {
    if (loops[k].ss == esz) ai = static_cast<int>(k);
    if (loops[k].sd == esz) bi = static_cast<int>(k);
  }
  if ((esz == 2 || esz == 4) && ai >= 0 && bi >= 0) {
    const int N = 16 / esz;
    const Loop& A = loops[ai];
    const Loop& B = loops[bi];
    bool ok = A.size % N == 0 && B.size % N == 0 && A.sd % 16 == 0 && B.ss % 16 == 0 &&
              off_s % 16 == 0 && off_d % 16 == 0 && aligned(src, 16) && aligned(dst, 16);
    std::vector<Loop> outer;
    for (size_t k = 0; k < loops.size(); ++k) {
      if (static_cast<int>(k) == ai || static_cast<int>(k) == bi) continue;
      outer.push_back(loops[k]);
      ok = ok && loops[k].ss % 16 == 0 && loops[k].sd % 16 == 0;
    }
    if (ok) {
      // Consecutive tiles (a wavefront's four, then neighbouring waves) step
      // along the outer loop with the smallest src stride: each wavefront
      // reads one contiguous run.
      std::stable_sort(outer.begin(), outer.end(),
                       [](const Loop& x, const Loop& y) { return x.ss < y.ss; });
      TNest n{};
      n.na = static_cast<uint32_t>(A.size / N);
      n.nb = static_cast<uint32_t>(B.size / N);
      const uint32_t ta = (n.na + 7) / 8, tb = (n.nb + 7) / 8;
      int64_t tiles = int64_t{ta} * tb;
      n.tiles_a = make_fastdiv(ta);
      n.tiles_b = make_fastdiv(tb);
      n.nouter = static_cast<int>(outer.size());
      for (size_t k = 0; k < outer.size(); ++k) {
        n.outer[k] = make_fastdiv(static_cast<uint32_t>(outer[k].size));
        n.ss[k] = outer[k].ss;
        n.sd[k] = outer[k].sd;
        tiles *= outer[k].size;
      }
      SPYRE_REQUIRE(tiles < (int64_t{1} << 30), SPYRE_EUNSUPPORTED, "transpose nest too large");
      n.a_sd = A.sd;
      n.b_ss = B.ss;
      n.off_s = off_s;
      n.off_d = off_d;
      n.tiles = static_cast<uint32_t>(tiles);
      constexpr uint32_t per_block = kThreads / 64 * kTransposeTiles;
      const dim3 grid((n.tiles + per_block - 1) / per_block);
      if (esz == 2) {
        // the stepped kernel's tile loops: A tiles, B tiles, the outer loops
        std::vector<Loop> tl;
        if (ta > 1) tl.push_back({ta, 128, 64 * A.sd});
        if (tb > 1) tl.push_back({tb, 64 * B.ss, 128});
        for (const Loop& o : outer) tl.push_back(o);
        // A wavefront's four tiles run along tl[0].  When they are B tiles
        // (contiguous in dst) and another loop steps by one 128-byte row in
        // src (a 3-D transpose back to host order: the host dim beside the
        // stick), that loop goes right after the four, so the four
        // wavefronts of a workgroup read adjacent src rows: 512-byte runs on
        // both sides instead of 128-byte src pieces 16 KiB apart (measured
        // [8, 1024, 4096], dim order [0, 2, 1], back to host order: 35.2 ->
        // 34.0 us).  With A tiles first the same move cost more than it gave
        // (27.0 -> 32.3 us the other way): src runs of 2 KiB per workgroup
        // row matter more there than dst runs of 512 B.
        if (!tl.empty() && ta <= 1 && tl.size() <= 3 && tl[0].size > kTransposeTiles &&
            tl[0].size % kTransposeTiles == 0) {
          for (size_t k = 1; k < tl.size(); ++k) {
            if (tl[k].ss != 128) continue;
            const Loop partner = tl[k];
            tl.erase(tl.begin() + static_cast<std::ptrdiff_t>(k));
            const Loop first = tl[0];
            tl[0] = {kTransposeTiles, first.ss, first.sd};
            tl.insert(tl.begin() + 1, partner);
            tl.insert(tl.begin() + 2, {first.size / kTransposeTiles, first.ss * kTransposeTiles,
                                       first.sd * kTransposeTiles});
            break;
          }
        }
        const StepSpan sp = step_span(tl, off_s, off_d, 63 * B.ss + 128, 63 * A.sd + 128);
        if (sp.ok && !tl.empty() && n.na % 8 == 0 && n.nb % 8 == 0 && tl[0].size % kTransposeTiles == 0 &&
            A.sd > 0 && B.ss > 0) {
          auto step_go = [&](auto nl_c) {
            constexpr int NL = decltype(nl_c)::value;
            const StepNest<NL> x = make_step<NL>(tl, n.tiles, off_s, off_d, sp.span_s, sp.span_d, B.ss, A.sd);
            if (sp.pow2)
              dma_transpose_step_kernel<NL, true><<<grid, kThreads, 0, st>>>(src, dst, x);
            else
              dma_transpose_step_kernel<NL, false><<<grid, kThreads, 0, st>>>(src, dst, x);
          };
          switch (tl.size()) {
            case 1: step_go(std::integral_constant<int, 1>{}); break;
            case 2: step_go(std::integral_constant<int, 2>{}); break;
            case 3: step_go(std::integral_constant<int, 3>{}); break;
            default: step_go(std::integral_constant<int, 4>{}); break;
          }
          return check_launch("dma_transpose_step_kernel");
        }
      }
      auto go = [&](auto esz_c, auto nout_c) {
        dma_transpose_kernel<decltype(esz_c)::value, decltype(nout_c)::value>
            <<<grid, kThreads, 0, st>>>(src, dst, n);
      };
      using I2 = std::integral_constant<int, 2>;
      using I4 = std::integral_constant<int, 4>;
      auto by_nout = [&](auto esz_c) {
        switch (n.nouter) {
          case 0: go(esz_c, std::integral_constant<int, 0>{}); break;
          case 1: go(esz_c, std::integral_constant<int, 1>{}); break;
          case 2: go(esz_c, std::integral_constant<int, 2>{}); break;
          case 3: go(esz_c, std::integral_constant<int, 3>{}); break;
          default: go(esz_c, std::integral_constant<int, -1>{}); break;
        }
      };
      if (esz == 2 && n.nouter <= 3) {
        // LDS-staged loads for 2-byte tiles (one 147 KiB workgroup per CU);
        // a tile's 64 rows in 32-bit buffer offsets when they fit
        const bool buf = 64 * n.b_ss + 128 < int64_t{kBufRange};
        auto lds_go = [&](auto nout_c, auto buf_c) {
          dma_transpose_lds_kernel<decltype(nout_c)::value, decltype(buf_c)::value>
              <<<grid, kThreads, 0, st>>>(src, dst, n);
        };
        auto by_buf = [&](auto nout_c) {
          if (buf)
            lds_go(nout_c, std::true_type{});
          else
            lds_go(nout_c, std::false_type{});
        };
        switch (n.nouter) {
          case 0: by_buf(std::integral_constant<int, 0>{}); break;
          case 1: by_buf(std::integral_constant<int, 1>{}); break;
          case 2: by_buf(std::integral_constant<int, 2>{}); break;
          default: by_buf(std::integral_constant<int, 3>{}); break;
        }
      } else if (esz == 2) {
        by_nout(I2{});
      } else {
        by_nout(I4{});
      }
      return check_launch("dma_transpose_kernel");
    }
  }

  // scalar fallback: innermost-by-dst loop first.
  const Loop inner{loops[0].size, loops[0].ss, loops[0].sd};
  std::vector<Loop> outer(loops.begin() + 1, loops.end());
  return launch_nest(inner, outer, off_s, off_d, esz, [&](const Nest& n) {
    const dim3 grid((n.total + kThreads - 1) / kThreads);
    switch (esz) {
      case 1: dma_scalar_kernel<1><<<grid, kThreads, 0, st>>>(src, dst, n); break;
      case 2: dma_scalar_kernel<2><<<grid, kThreads, 0, st>>>(src, dst, n); break;
      case 4: dma_scalar_kernel<4><<<grid, kThreads, 0, st>>>(src, dst, n); break;
      default: dma_scalar_kernel<8><<<grid, kThreads, 0, st>>>(src, dst, n); break;
    }
    return check_launch("dma_scalar_kernel");
  });
}

}  // namespace

// Largest element index a loop nest touches on one side (strides >= 0).
static bool nest_extent(const spyre_stride_info& s, bool src_side, int64_t& hi) {
  int64_t off = src_side ? s.offset_src : s.offset_dst;
  if (off < 0) return false;
  for (int q = 0; q < s.rank; ++q) {
    const int64_t st = src_side ? s.stride_src[q] : s.stride_dst[q];
    if (st < 0) return false;
    if (s.size[q] == 0) {
      hi = -1;
      return true;
    }
    off += (s.size[q] - 1) * st;
  }
  hi = off;
  return true;
}

extern "C" int spyre_dma_copy(const void* src, size_t src_bytes, void* dst, size_t dst_bytes,
                              int elem_bytes, const spyre_stride_info* infos, int n_infos,
                              void* stream) {
  spyre_hip::clear_error();
  SPYRE_REQUIRE(src && dst && infos, SPYRE_EINVAL, "null pointer argument");
  SPYRE_REQUIRE(elem_bytes == 1 || elem_bytes == 2 || elem_bytes == 4 || elem_bytes == 8,
                SPYRE_EINVAL, "elem_bytes must be 1, 2, 4 or 8 (got %d)", elem_bytes);
  SPYRE_REQUIRE(n_infos >= 0 && n_infos <= SPYRE_MAX_INFOS, SPYRE_EINVAL, "bad n_infos %d",
                n_infos);
  for (int i = 0; i < n_infos; ++i) {
    const spyre_stride_info& s = infos[i];
    SPYRE_REQUIRE(s.rank >= 1 && s.rank <= SPYRE_MAX_RANK, SPYRE_EINVAL, "bad rank %d", s.rank);
    for (int q = 0; q < s.rank; ++q)
      SPYRE_REQUIRE(s.size[q] >= 0 && s.size[q] < (int64_t{1} << 31), SPYRE_EINVAL,
                    "bad loop size %lld", static_cast<long long>(s.size[q]));
    int64_t hs = 0, hd = 0;
    SPYRE_REQUIRE(nest_extent(s, true, hs) && nest_extent(s, false, hd), SPYRE_EINVAL,
                  "negative stride or offset in loop nest %d", i);
    SPYRE_REQUIRE((hs + 1) * elem_bytes <= static_cast<int64_t>(src_bytes), SPYRE_EINVAL,
                  "loop nest %d reads past the source buffer (%lld > %zu bytes)", i,
                  static_cast<long long>((hs + 1) * elem_bytes), src_bytes);
    SPYRE_REQUIRE((hd + 1) * elem_bytes <= static_cast<int64_t>(dst_bytes), SPYRE_EINVAL,
                  "loop nest %d writes past the destination buffer (%lld > %zu bytes)", i,
                  static_cast<long long>((hd + 1) * elem_bytes), dst_bytes);
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  for (int i = 0; i < n_infos; ++i) {
    const int rc = run_info(static_cast<const char*>(src), static_cast<char*>(dst), elem_bytes,
                            infos[i], st);
    if (rc != SPYRE_OK) return rc;
  }
  return SPYRE_OK;
}
