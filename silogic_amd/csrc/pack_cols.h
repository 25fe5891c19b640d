// Bit-packing of sample rows into 64-sample words, shared by the input
// encoders (encode.hip) and pack_bits (fc_hard.hip).
#pragma once
#include "slg_common.h"

namespace slg {

// The words of V features over the 64 samples of one word, built in
// registers (no LDS, no ballot): xr points at the word's first row (rows D
// elements apart), nr rows exist (1..64; rows past them read the last row,
// so no load is branched, and their bits are cleared), src[v] is feature
// v's offset in a row and bit(value, v) its test. VEC: the features are
// V = 4 contiguous, 4-aligned elements read as one vector per row. Byte
// inputs issue all 64 rows' loads before the first test (one register per
// load); 4-byte inputs go 16 rows at a time.
template <int V, bool VEC, typename TX, typename BitFn>
__device__ __forceinline__ void pack_cols(const TX* __restrict__ xr, int D, int nr,
                                          const int (&src)[V], BitFn bit, uint64_t (&word)[V]) {
  static_assert(!VEC || V == 4, "vector rows are 4 features");
#pragma unroll
  for (int v = 0; v < V; ++v) word[v] = 0;
  auto chunk = [&](int c) {
    uint32_t m[V];
#pragma unroll
    for (int v = 0; v < V; ++v) m[v] = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const TX* row = xr + (int64_t)min(c + i, nr - 1) * D;
      if constexpr (VEC) {
        if constexpr (sizeof(TX) == 1) {
          const uint32_t q = *reinterpret_cast<const uint32_t*>(row + src[0]);
#pragma unroll
          for (int v = 0; v < 4; ++v) m[v] |= (bit((TX)(q >> (8 * v)), v) ? 1u : 0u) << i;
        } else {
          const float4 q = *reinterpret_cast<const float4*>(row + src[0]);
          const float qv[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
          for (int v = 0; v < 4; ++v) m[v] |= (bit(qv[v], v) ? 1u : 0u) << i;
        }
      } else {
#pragma unroll
        for (int v = 0; v < V; ++v) m[v] |= (bit(row[src[v]], v) ? 1u : 0u) << i;
      }
    }
#pragma unroll
    for (int v = 0; v < V; ++v) word[v] |= (uint64_t)m[v] << c;
  };
  if constexpr (sizeof(TX) == 1) {
    chunk(0); chunk(16); chunk(32); chunk(48);
  } else {
#pragma unroll 1
    for (int c = 0; c < 64; c += 16) chunk(c);
  }
  const uint64_t valid = nr == 64 ? ~0ull : (1ull << nr) - 1;
#pragma unroll
  for (int v = 0; v < V; ++v) word[v] &= valid;
}

}  // namespace slg
