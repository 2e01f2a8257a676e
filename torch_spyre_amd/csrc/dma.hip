// GPU executor of DMA loop nests (spyre_dma_copy).
//
// A loop nest says: for every index tuple i, dst[off_d + i.sd] = src[off_s + i.ss].
// The host normalises it (drops unit loops, merges loops that are contiguous
// on both sides) and picks one of three kernels:
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
//               owns four 64x64 tiles of 2-byte elements; each lane loads an
//               8x8 block per tile as eight 16-byte row segments (all 32
//               loads first), transposes them in registers and stores eight
//               16-byte column segments per tile.  Loads and stores are both
//               128-byte-line coalesced and LDS is not used.
//  * scalar:    anything else, element by element.
//
// Index decomposition uses multiply-high division by loop-invariant divisors
// (Granlund & Montgomery, "Division by Invariant Integers using
// Multiplication", PLDI 1994, round-up variant), valid for 0 <= n, d < 2^31.

#include <hip/hip_runtime.h>

#include <algorithm>
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
constexpr int kTilePad = 8;     // 16-B units of LDS padding per tile row (bank spread)
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

// Moves one tile of kTileSticks x kTileSticks sticks: load k reads the B
// run of A stick k (this lane: B stick `stick`, 16-byte unit `unit`) at
// sp + k * a_ss; store k writes the A run of B stick k at dp + k * b_sd.
// GUARDED: only A sticks < a_left and B sticks < b_left exist (b_lane /
// a_lane: this lane's B / A stick exists).
template <bool GUARDED>
__device__ __forceinline__ void stick_tile(const char* sp, char* dp, int64_t a_ss, int64_t b_sd,
                                           bool b_lane, bool a_lane, uint32_t a_left,
                                           uint32_t b_left, u32x4* lds) {
  constexpr int kRow = kTileSticks * 8 + kTilePad;  // LDS row: one B stick's A run, in 16-B units
  const uint32_t stick = threadIdx.x >> 3, unit = threadIdx.x & 7;
  u32x4 x[kTileSticks];
#pragma unroll
  for (int k = 0; k < kTileSticks; ++k, sp += a_ss)
    if (!GUARDED || (b_lane && static_cast<uint32_t>(k) < a_left)) x[k] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(sp));
#pragma unroll
  for (int k = 0; k < kTileSticks; ++k) lds[stick * kRow + k * 8 + unit] = x[k];
  __syncthreads();
#pragma unroll
  for (int k = 0; k < kTileSticks; ++k) x[k] = lds[k * kRow + threadIdx.x];
#pragma unroll
  for (int k = 0; k < kTileSticks; ++k, dp += b_sd)
    if (!GUARDED || (a_lane && static_cast<uint32_t>(k) < b_left)) __builtin_nontemporal_store(x[k], reinterpret_cast<u32x4*>(dp));
}

__global__ __launch_bounds__(kThreads) void dma_stick_tile_kernel(const char* __restrict__ src,
                                                                   char* __restrict__ dst, SNest n) {
  __shared__ u32x4 lds[kTileSticks * (kTileSticks * 8 + kTilePad)];
  const uint32_t na = pinned(n.na), nb = pinned(n.nb);
  const int64_t a_ss = pinned(n.a_ss), b_sd = pinned(n.b_sd);
  uint32_t q = blockIdx.x;
  uint32_t q2 = fdiv(q, n.tiles_x);
  const uint32_t tx = q - q2 * n.tiles_x.d;
  q = q2;
  q2 = fdiv(q, n.tiles_y);
  const uint32_t ty = q - q2 * n.tiles_y.d;
  q = q2;
  const uint32_t ta = n.b_first ? ty : tx, tb = n.b_first ? tx : ty;
  int64_t so = n.off_s, sd = n.off_d;
  for (int k = 0; k < n.nouter; ++k) {
    q2 = fdiv(q, n.outer[k]);
    const int64_t c = q - q2 * n.outer[k].d;
    so += c * n.ss[k];
    sd += c * n.sd[k];
    q = q2;
  }
  const uint32_t a0 = ta * kTileSticks, b0 = tb * kTileSticks;
  const uint32_t stick = threadIdx.x >> 3, unit = threadIdx.x & 7;
  const char* sp = src + so + static_cast<int64_t>(a0) * a_ss + static_cast<int64_t>(b0 + stick) * 128 + unit * 16;
  char* dp = dst + sd + static_cast<int64_t>(b0) * b_sd + static_cast<int64_t>(a0 + stick) * 128 + unit * 16;
  // Edge tiles predicate every access; full tiles (all but the last along A
  // and B) run unpredicated, so their LDS writes follow the loads as the
  // data arrives.
  if (a0 + kTileSticks <= na && b0 + kTileSticks <= nb)
    stick_tile<false>(sp, dp, a_ss, b_sd, true, true, 0, 0, lds);
  else
    stick_tile<true>(sp, dp, a_ss, b_sd, b0 + stick < nb, a0 + stick < na, na - a0, nb - b0, lds);
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
    if (vb == 16 && row == 128) {
      // stick tile: loop A continues the stick in dst, loop B in src.
      int ai = -1, bi = -1;
      for (size_t k = 0; k < outer.size(); ++k) {
        if (outer[k].sd == row && ai < 0) ai = static_cast<int>(k);
        else if (outer[k].ss == row && bi < 0) bi = static_cast<int>(k);
      }
      if (ai >= 0 && bi >= 0 && outer[ai].size >= kTileSticks && outer[bi].size >= kTileSticks) {
        SNest n{};
        n.na = static_cast<uint32_t>(outer[ai].size);
        n.nb = static_cast<uint32_t>(outer[bi].size);
        const uint32_t ta = (n.na + kTileSticks - 1) / kTileSticks;
        const uint32_t tb = (n.nb + kTileSticks - 1) / kTileSticks;
        int64_t tiles = int64_t{ta} * tb;
        // Consecutive workgroups step along the loop whose other-side stride
        // is smaller (the row-major rows), so concurrently running tiles
        // cover neighbouring memory on both sides.
        n.b_first = outer[bi].sd < outer[ai].ss;
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
        if (tiles < (int64_t{1} << 31)) {
          dma_stick_tile_kernel<<<dim3(static_cast<uint32_t>(tiles)), kThreads, 0, st>>>(src, dst, n);
          return check_launch("dma_stick_tile_kernel");
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
      if (esz == 2)
        by_nout(I2{});
      else
        by_nout(I4{});
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
