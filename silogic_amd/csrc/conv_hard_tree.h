// Tree evaluation of the hard conv blocks on packed words (32 samples per
// 32-bit half), shared by the conv block kernels (conv_hard.hip) and the
// kernel that evaluates a last conv block inside a conv network's head
// (fc_hard.hip). Node semantics: silogic/nodes.py:183-189,
// layers.py:515-527; gate16 trees and LUTs as multiplexer trees whose masks
// come from the table bits.
#pragma once
#include "slg_common.h"

namespace slg {

__device__ __forceinline__ uint32_t mux32(uint32_t s, uint32_t a, uint32_t b) {
  return __builtin_amdgcn_bitop3_b32(s, a, b, (unsigned char)0xCA);  // s ? a : b, bitwise
}

// The level-1 masks of a channel's tables, half in VGPRs and half in SGPRs
// (a VALU instruction reads at most one scalar operand): entry pair m of a
// LUT is (ev[m], es[m]) = (entry 2m+1, entry 2m); gate16 node k is
// (ev[2k+1], es[2k+1]) = (entry 3, entry 2) and (ev[2k], es[2k]) =
// (entry 1, entry 0) of its 4-bit table.
template <int NODE, int NLEAF>
constexpr int n_mux_masks() {
  return NODE == SLG_NODE_GATE16 ? 2 * (NLEAF - 1) : (1 << (NLEAF - 1));
}

// a copy of a uniform value in a vector register
__device__ __forceinline__ uint32_t to_vgpr(uint32_t s) {
  uint32_t v;
  asm("v_mov_b32 %0, %1" : "=v"(v) : "s"(s));
  return v;
}

template <int NODE, int NLEAF>
__device__ __forceinline__ void tree_masks(uint32_t tlo, uint32_t thi,
                                           uint32_t (&ev)[n_mux_masks<NODE, NLEAF>()],
                                           uint32_t (&es)[n_mux_masks<NODE, NLEAF>()]) {
  constexpr int NM = n_mux_masks<NODE, NLEAF>();
  const uint32_t vlo = to_vgpr(tlo), vhi = to_vgpr(thi);
#pragma unroll
  for (int m = 0; m < NM; ++m) {
    const int odd = 2 * m + 1, even = 2 * m;  // table bits (gate16: node m/2, entries 2(m&1)+{1,0})
    ev[m] = (uint32_t)__builtin_amdgcn_sbfe((int)(odd < 32 ? vlo : vhi), odd & 31, 1);
    es[m] = (uint32_t)__builtin_amdgcn_sbfe((int)(even < 32 ? tlo : thi), even & 31, 1);
  }
}

// one tree (NODE, NLEAF leaves) on 32 samples with the masks above
template <int NODE, int NLEAF>
__device__ __forceinline__ uint32_t tree_eval32(const uint32_t (&v)[NLEAF],
                                                const uint32_t (&ev)[n_mux_masks<NODE, NLEAF>()],
                                                const uint32_t (&es)[n_mux_masks<NODE, NLEAF>()]) {
  if constexpr (NODE == SLG_NODE_GATE16) {
    uint32_t t[NLEAF];
#pragma unroll
    for (int l = 0; l < NLEAF; ++l) t[l] = v[l];
    int nb = 0;
#pragma unroll
    for (int cnt = NLEAF; cnt > 1; cnt >>= 1) {
#pragma unroll
      for (int m = 0; m < cnt / 2; ++m) {
        const int k = nb + m;
        const uint32_t a = t[2 * m], b = t[2 * m + 1];
        t[m] = mux32(a, mux32(b, ev[2 * k + 1], es[2 * k + 1]), mux32(b, ev[2 * k], es[2 * k]));
      }
      nb += cnt / 2;
    }
    return t[0];
  } else {
    uint32_t t[1 << (NLEAF - 1)];
#pragma unroll
    for (int m = 0; m < (1 << (NLEAF - 1)); ++m) t[m] = mux32(v[0], ev[m], es[m]);
#pragma unroll
    for (int j = 1; j < NLEAF; ++j)
#pragma unroll
      for (int m = 0; m < (1 << (NLEAF - 1 - j)); ++m) t[m] = mux32(v[j], t[2 * m + 1], t[2 * m]);
    return t[0];
  }
}

// The masks of tree_masks for a table held per lane (each lane's own
// channel): both halves in vector registers.
template <int NODE, int NLEAF>
__device__ __forceinline__ void tree_masks_lane(uint32_t tlo, uint32_t thi,
                                                uint32_t (&ev)[n_mux_masks<NODE, NLEAF>()],
                                                uint32_t (&es)[n_mux_masks<NODE, NLEAF>()]) {
  constexpr int NM = n_mux_masks<NODE, NLEAF>();
#pragma unroll
  for (int m = 0; m < NM; ++m) {
    const int odd = 2 * m + 1, even = 2 * m;
    ev[m] = (uint32_t)__builtin_amdgcn_sbfe((int)(odd < 32 ? tlo : thi), odd & 31, 1);
    es[m] = (uint32_t)__builtin_amdgcn_sbfe((int)(even < 32 ? tlo : thi), even & 31, 1);
  }
}

}  // namespace slg
