// GPU executor of DMA loop nests (spyre_dma_copy).
//
// A loop nest says: for every index tuple i, dst[off_d + i.sd] = src[off_s + i.ss].
// The host normalises it (drops unit loops, merges loops that are contiguous
// on both sides) and picks one of three kernels:
//
//  * vec:       one loop is unit-stride on both sides (a stick moved as a
//               whole, e.g. row-major <-> sticks).  Each lane moves 16 bytes;
//               eight lanes cover one 128-byte stick, so every wavefront
//               touches whole cache lines on both sides.  No LDS: with whole
//               sticks as the unit there is nothing to transpose.
//  * transpose: one loop is unit-stride in src and another in dst (the stick
//               moves to another dim, e.g. transpose-restick).  A wavefront
//               owns a 64x64 tile of 2-byte elements; each lane loads an 8x8
//               block as eight 16-byte row segments, transposes it in
//               registers and stores eight 16-byte column segments.  Loads and
//               stores are both 128-byte-line coalesced and LDS is not used,
//               so there are no bank conflicts to avoid.
//  * scalar:    anything else, element by element.
//
// Index decomposition uses multiply-high division by loop-invariant divisors
// (Granlund & Montgomery, "Division by Invariant Integers using
// Multiplication", PLDI 1994, round-up variant), valid for 0 <= n, d < 2^31.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <vector>

#include "spyre_common.h"

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

__device__ __forceinline__ uint32_t fdiv(uint32_t n, const FastDiv& f) {
  return (__umulhi(n, f.mul) + n) >> f.shift;
}

constexpr int kMaxLoops = SPYRE_MAX_RANK;
constexpr int kThreads = 256;
constexpr int kItems = 4;  // vec kernel: items per lane, strided by the block size

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

// Each lane moves kItems items of VB bytes; all loads are issued before the
// stores so several cache lines per lane are in flight.
template <int VB>
__global__ __launch_bounds__(kThreads) void dma_vec_kernel(const char* __restrict__ src,
                                                           char* __restrict__ dst, Nest n) {
  using T = typename VecT<VB>::T;
  const uint32_t base = blockIdx.x * (kThreads * kItems) + threadIdx.x;
  T v[kItems];
  int64_t doff[kItems];
#pragma unroll
  for (int it = 0; it < kItems; ++it) {
    const uint32_t i = base + it * kThreads;
    doff[it] = -1;
    if (i < n.total) {
      int64_t so;
      item_offsets(n, i, so, doff[it]);
      v[it] = __builtin_nontemporal_load(reinterpret_cast<const T*>(src + so));
    }
  }
#pragma unroll
  for (int it = 0; it < kItems; ++it)
    if (doff[it] >= 0) __builtin_nontemporal_store(v[it], reinterpret_cast<T*>(dst + doff[it]));
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
  uint32_t waves;             // total wave tiles
};

template <int ESZ>
__device__ __forceinline__ void transpose_block(u32x4 (&r)[16 / ESZ], u32x4 (&o)[16 / ESZ]);

template <>
__device__ __forceinline__ void transpose_block<2>(u32x4 (&r)[8], u32x4 (&o)[8]) {
  // r[b] holds elements a = 0..7 of row b; o[a] gets elements b = 0..7 of column a.
  const uint32_t* w = reinterpret_cast<const uint32_t*>(r);
  uint32_t* x = reinterpret_cast<uint32_t*>(o);
#pragma unroll
  for (int a = 0; a < 8; ++a) {
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const uint32_t lo = w[(2 * p) * 4 + a / 2];
      const uint32_t hi = w[(2 * p + 1) * 4 + a / 2];
      x[a * 4 + p] = (a & 1) ? ((lo >> 16) | (hi & 0xffff0000u)) : ((lo & 0xffffu) | (hi << 16));
    }
  }
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

template <int ESZ>
__global__ __launch_bounds__(kThreads) void dma_transpose_kernel(const char* __restrict__ src,
                                                                 char* __restrict__ dst, TNest n) {
  constexpr int N = 16 / ESZ;
  const uint32_t wave = blockIdx.x * (kThreads / 64) + threadIdx.x / 64;
  if (wave >= n.waves) return;
  const uint32_t lane = threadIdx.x % 64;
  uint32_t q = fdiv(wave, n.tiles_a);
  const uint32_t ta = wave - q * n.tiles_a.d;
  uint32_t q2 = fdiv(q, n.tiles_b);
  const uint32_t tb = q - q2 * n.tiles_b.d;
  q = q2;
  int64_t so = n.off_s, sd = n.off_d;
  for (int k = 0; k < n.nouter; ++k) {
    q2 = fdiv(q, n.outer[k]);
    const int64_t c = q - q2 * n.outer[k].d;
    so += c * n.ss[k];
    sd += c * n.sd[k];
    q = q2;
  }
  const uint32_t ablk = ta * 8 + lane % 8;
  const uint32_t bblk = tb * 8 + lane / 8;
  if (ablk >= n.na || bblk >= n.nb) return;
  so += static_cast<int64_t>(ablk) * 16 + static_cast<int64_t>(bblk) * N * n.b_ss;
  sd += static_cast<int64_t>(bblk) * 16 + static_cast<int64_t>(ablk) * N * n.a_sd;
  u32x4 r[N], o[N];
#pragma unroll
  for (int b = 0; b < N; ++b)
    r[b] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + so + b * n.b_ss));
  transpose_block<ESZ>(r, o);
#pragma unroll
  for (int a = 0; a < N; ++a)
    __builtin_nontemporal_store(o[a], reinterpret_cast<u32x4*>(dst + sd + a * n.a_sd));
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
    const Loop inner{row / vb, vb, vb};
    return launch_nest(inner, outer, off_s, off_d, vb, [&](const Nest& n) {
      const dim3 grid((n.total + kThreads * kItems - 1) / (kThreads * kItems));
      switch (vb) {
        case 16: dma_vec_kernel<16><<<grid, kThreads, 0, st>>>(src, dst, n); break;
        case 8: dma_vec_kernel<8><<<grid, kThreads, 0, st>>>(src, dst, n); break;
        case 4: dma_vec_kernel<4><<<grid, kThreads, 0, st>>>(src, dst, n); break;
        case 2: dma_vec_kernel<2><<<grid, kThreads, 0, st>>>(src, dst, n); break;
        default: dma_vec_kernel<1><<<grid, kThreads, 0, st>>>(src, dst, n); break;
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
      TNest n{};
      n.na = static_cast<uint32_t>(A.size / N);
      n.nb = static_cast<uint32_t>(B.size / N);
      const uint32_t ta = (n.na + 7) / 8, tb = (n.nb + 7) / 8;
      int64_t waves = int64_t{ta} * tb;
      n.tiles_a = make_fastdiv(ta);
      n.tiles_b = make_fastdiv(tb);
      n.nouter = static_cast<int>(outer.size());
      for (size_t k = 0; k < outer.size(); ++k) {
        n.outer[k] = make_fastdiv(static_cast<uint32_t>(outer[k].size));
        n.ss[k] = outer[k].ss;
        n.sd[k] = outer[k].sd;
        waves *= outer[k].size;
      }
      SPYRE_REQUIRE(waves < (int64_t{1} << 30), SPYRE_EUNSUPPORTED, "transpose nest too large");
      n.a_sd = A.sd;
      n.b_ss = B.ss;
      n.off_s = off_s;
      n.off_d = off_d;
      n.waves = static_cast<uint32_t>(waves);
      const dim3 grid((n.waves + kThreads / 64 - 1) / (kThreads / 64));
      if (esz == 2)
        dma_transpose_kernel<2><<<grid, kThreads, 0, st>>>(src, dst, n);
      else
        dma_transpose_kernel<4><<<grid, kThreads, 0, st>>>(src, dst, n);
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
