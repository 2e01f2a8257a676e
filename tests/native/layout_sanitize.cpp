// Host-only driver for the layout planner (csrc/layout.cpp) built with
// AddressSanitizer and UndefinedBehaviorSanitizer: seeded random shapes,
// dtypes, strides and dim orders through every planner entry point, both
// DMA directions and layout-to-layout resticks, plus argument errors.  It
// checks that each call either succeeds with nests inside the layout's
// allocation or fails with an error code -- the sanitizers catch any
// out-of-bounds access or undefined behaviour on the way.
#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <random>
#include <vector>

#include "../../include/spyre_hip.h"

namespace {

int fails = 0;

void expect(bool ok, const char* what, int iter) {
  if (!ok) {
    std::fprintf(stderr, "iteration %d: %s (%s)\n", iter, what, spyre_last_error());
    ++fails;
  }
}

// Highest element offset a nest touches on one side, from its strides and
// sizes (non-negative strides only; the planner emits no others).
int64_t span_of(const spyre_stride_info& s, bool dst) {
  int64_t hi = dst ? s.offset_dst : s.offset_src;
  for (int k = 0; k < s.rank; ++k) {
    const int64_t st = dst ? s.stride_dst[k] : s.stride_src[k];
    if (s.size[k] > 0 && st > 0) hi += (s.size[k] - 1) * st;
  }
  return hi;
}

}  // namespace

int main() {
  std::mt19937_64 rng(0x5EED);
  const int64_t dims[] = {1, 2, 3, 7, 8, 63, 64, 65, 100, 128, 200};
  const int dtypes[] = {SPYRE_DT_FLOAT16, SPYRE_DT_BFLOAT16, SPYRE_DT_FLOAT32, SPYRE_DT_INT32, SPYRE_DT_BOOL};
  int ok_layouts = 0, ok_plans = 0, ok_resticks = 0;
  for (int it = 0; it < 4000; ++it) {
    const int rank = 1 + static_cast<int>(rng() % 6);
    std::vector<int64_t> size(rank), stride(rank);
    int64_t n = 1;
    for (int i = 0; i < rank; ++i) size[i] = dims[rng() % (sizeof(dims) / sizeof(dims[0]))];
    for (int i = rank - 1; i >= 0; --i) {
      stride[i] = n;
      n *= size[i];
    }
    if (n > (int64_t{1} << 26)) continue;
    const int dt = dtypes[rng() % (sizeof(dtypes) / sizeof(dtypes[0]))];
    // A dim order: none, a permutation, or a permutation with the sparse -1.
    std::vector<int32_t> order(rank);
    for (int i = 0; i < rank; ++i) order[i] = i;
    std::shuffle(order.begin(), order.end(), rng);
    const int mode = static_cast<int>(rng() % 3);
    if (mode == 2) order.push_back(-1);
    int64_t dsize[SPYRE_MAX_RANK], smap[SPYRE_MAX_RANK];
    int drank = 0, fmt = 0;
    const int rc = spyre_stl_init(size.data(), rank, mode ? stride.data() : nullptr, dt,
                                  mode ? order.data() : nullptr, mode ? static_cast<int>(order.size()) : 0, dsize,
                                  smap, &drank, &fmt);
    if (rc != SPYRE_OK) continue;
    ++ok_layouts;
    expect(drank >= 1 && drank <= SPYRE_MAX_RANK, "device rank out of range", it);
    const uint64_t bytes = spyre_device_size_in_bytes(dsize, drank);
    const int esz = dt == SPYRE_DT_FLOAT32 || dt == SPYRE_DT_INT32 ? 4 : 2;
    const int64_t dev_elems = static_cast<int64_t>(bytes / esz);
    for (int h2d = 0; h2d < 2; ++h2d) {
      spyre_stride_info infos[SPYRE_MAX_INFOS];
      int ninf = 0;
      const int prc = spyre_dma_plan(size.data(), stride.data(), stride.data(), rank, 0, dsize, smap, drank, h2d,
                                     infos, SPYRE_MAX_INFOS, &ninf);
      if (prc != SPYRE_OK) continue;
      ++ok_plans;
      for (int i = 0; i < ninf; ++i) {
        const int64_t dev_hi = span_of(infos[i], h2d != 0);
        const int64_t host_hi = span_of(infos[i], h2d == 0);
        expect(dev_hi < dev_elems || dev_elems == 0, "nest past the device allocation", it);
        expect(host_hi < n, "nest past the host tensor", it);
      }
    }
    // Restick to the default layout of the same shape and back.
    int64_t dsize2[SPYRE_MAX_RANK], smap2[SPYRE_MAX_RANK];
    int drank2 = 0, fmt2 = 0;
    if (spyre_stl_init(size.data(), rank, nullptr, dt, nullptr, 0, dsize2, smap2, &drank2, &fmt2) == SPYRE_OK) {
      spyre_stride_info r;
      if (spyre_restick_plan(size.data(), rank, dsize, smap, drank, dsize2, smap2, drank2, &r) == SPYRE_OK) {
        ++ok_resticks;
        expect(r.rank >= 1 && r.rank <= SPYRE_MAX_RANK, "restick rank out of range", it);
      }
    }
  }
  // Argument errors come back as codes.
  int64_t s1[1] = {64}, d[SPYRE_MAX_RANK], m[SPYRE_MAX_RANK];
  int dr = 0, f = 0, ni = 0;
  expect(spyre_stl_init(nullptr, 1, nullptr, SPYRE_DT_FLOAT16, nullptr, 0, d, m, &dr, &f) != SPYRE_OK, "null size", -1);
  expect(spyre_stl_init(s1, 7, nullptr, SPYRE_DT_FLOAT16, nullptr, 0, d, m, &dr, &f) != SPYRE_OK, "rank 7", -1);
  expect(spyre_stl_init(s1, 1, nullptr, 12345, nullptr, 0, d, m, &dr, &f) != SPYRE_OK, "bad dtype", -1);
  spyre_stride_info one[1];
  expect(spyre_dma_plan(s1, s1, s1, 1, 0, nullptr, nullptr, 0, 1, one, 1, &ni) != SPYRE_OK, "null layout", -1);
  std::printf("layouts %d, plans %d, resticks %d, failures %d\n", ok_layouts, ok_plans, ok_resticks, fails);
  return fails == 0 ? 0 : 1;
}
