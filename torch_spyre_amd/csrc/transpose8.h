// In-register transpose of an 8 x 8 block of 16-bit elements, shared by the
// relayout transposes and the attention V restick.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace spyre_hip {

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// r[b] holds elements a = 0..7 of row b (16 bytes); o[a] receives elements
// b = 0..7 of column a.
__device__ __forceinline__ void transpose8x8_b16(const u32x4_t (&r)[8], u32x4_t (&o)[8]) {
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

}  // namespace spyre_hip
