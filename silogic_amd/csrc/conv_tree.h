// The tree of one ConvLogicTree output channel, shared by the soft forward
// and backward kernels so that both evaluate it with the same operations
// (the backward's max-pool routing compares the forward's exact values).
#pragma once

#include "slg_common.h"

namespace slg {

// NODE: SLG_NODE_GATE16 (NLEAF = 2^depth leaves, binary BasisProj tree),
// SLG_NODE_MULTILINEAR2 used as "LUT" (NLEAF = arity, depth 1), or
// SLG_NODE_HYBRID (the same LUT read at the address of the leaves
// thresholded at 0.5, nodes.py:198-206).
template <int NODE, int NLEAF>
struct ConvNode {
  static constexpr int NN = (NODE == SLG_NODE_GATE16) ? NLEAF - 1 : 1;  // tree nodes
  // parameters kept per channel: gate16 coefficients [NN][4]; for the
  // multilinear LUT, per group of 2^LG corners (LG = min(NLEAF, 3): the
  // corners that differ in leaves 0..LG-1) the group's polynomial
  // coefficients (lut_group_coeffs); for the hybrid LUT the values s[p] as
  // they are
  static constexpr int NPR = (NODE == SLG_NODE_GATE16) ? 4 * NN : (1 << NLEAF);
  static constexpr int LG = NLEAF < 3 ? NLEAF : 3;
  static constexpr int NP = (NODE == SLG_NODE_GATE16) ? 4 * NN : (1 << NLEAF);  // raw params
};

// The multilinear LUT's kept form: the corners of a group (index i over
// leaves 0..G-1) as the coefficients of the group's multilinear polynomial
// in those leaves, c[i] = sum over subsets j of i of (-1)^|i-j| s[j] (the
// subset-difference transform, one bit at a time in this fixed order, so
// every kernel that keeps them gets the same bits). The interpolation over
// the group's leaves is then 2^G - 1 FMAs (conv_tree_eval) where the lerp
// tree takes 2^(G-1) FMAs and 2^(G-1) - 1 subtract-FMA pairs.
template <int G>
__device__ inline void lut_group_coeffs(float (&c)[1 << G]) {
#pragma unroll
  for (int b = 0; b < G; ++b)
#pragma unroll
    for (int i = 0; i < (1 << G); ++i)
      if ((i >> b) & 1) c[i] = c[i] - c[i ^ (1 << b)];
}

// Tree value at leaf values v with kept parameters par (ConvNode::NPR).
template <int NODE, int NLEAF>
__device__ inline float conv_tree_eval(const float (&v)[NLEAF], const float* par) {
  if constexpr (NODE == SLG_NODE_GATE16) {
    // level i combines children 2m (a) and 2m+1 (b), node ids level-major
    // (silogic/layers.py:388-401, 408-417); c0 + c1 a + c2 b + c3 ab as
    // c0 + c1 a + b (c2 + c3 a), three FMAs
    float u[NLEAF];
#pragma unroll
    for (int l = 0; l < NLEAF; ++l) u[l] = v[l];
    int nb = 0;
#pragma unroll
    for (int cnt = NLEAF; cnt > 1; cnt >>= 1) {
#pragma unroll
      for (int m = 0; m < cnt / 2; ++m) {
        const float a = u[2 * m], b = u[2 * m + 1];
        const float* c = par + 4 * (nb + m);
        u[m] = fmaf(b, fmaf(a, c[3], c[2]), fmaf(a, c[1], c[0]));
      }
      nb += cnt / 2;
    }
    return u[0];
  } else if constexpr (NODE == SLG_NODE_HYBRID) {
    int addr = 0;
#pragma unroll
    for (int l = 0; l < NLEAF; ++l) addr |= (v[l] >= 0.5f ? 1 : 0) << l;
    return par[addr];
  } else {
    // multilinear interpolation of s over the leaves (corner bit j = leaf
    // j), silogic/nodes.py:174-178: each group's polynomial in leaves
    // 0..LG-1 nested in Horner form, then a lerp tree over the rest
    constexpr int LG = ConvNode<NODE, NLEAF>::LG;
    constexpr int NG = 1 << (NLEAF - LG);
    float t[NG];
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      const float* c = par + (g << LG);
      if constexpr (LG == 3) {
        const float p = fmaf(v[1], fmaf(v[0], c[3], c[2]), fmaf(v[0], c[1], c[0]));
        const float q = fmaf(v[1], fmaf(v[0], c[7], c[6]), fmaf(v[0], c[5], c[4]));
        t[g] = fmaf(v[2], q, p);
      } else if constexpr (LG == 2) {
        t[g] = fmaf(v[1], fmaf(v[0], c[3], c[2]), fmaf(v[0], c[1], c[0]));
      } else {
        t[g] = fmaf(v[0], c[1], c[0]);
      }
    }
#pragma unroll
    for (int j = LG; j < NLEAF; ++j) {
#pragma unroll
      for (int m = 0; m < (1 << (NLEAF - 1 - j)); ++m)
        t[m] = fmaf(v[j], t[2 * m + 1] - t[2 * m], t[2 * m]);
    }
    return t[0];
  }
}

// Node trees on the generic kernels (conv_generic.hip): gate16 and walsh
// binary trees of depth 1-5, multilinear and hybrid LUT trees with at most
// 36 leaves (arity 2: depth <= 5; 3: <= 3; 4-6: <= 2), any image size.
// Parameters [N][nodes][P] level-major, P = 4 (gate16 coefficients, walsh
// coefficients times 1/tau) or 2^arity (LUT values).
bool conv_generic_supported(int node, int depth, int arity);
int conv_generic_params(int node, int depth, int arity);
int conv_generic_fwd(const float* x, int64_t B, int64_t C, int64_t H, int64_t W, int64_t N,
                     int node, int depth, int arity, int K, int kernel, int pad, bool pool,
                     const float* np, const float* w, const int* cm, const int* ch, const int* cw,
                     float* out, int64_t Ho, int64_t Wo, hipStream_t st);
int64_t conv_generic_bwd_workspace(int64_t B, int64_t C, int64_t H, int64_t W, int64_t N, int node,
                                   int depth, int arity, int K, int pad, bool pool);
int conv_generic_bwd(const float* x, int64_t B, int64_t C, int64_t H, int64_t W, int64_t N,
                     int node, int depth, int arity, int K, int pad, bool pool, const float* np,
                     const float* w, const int* cm, const int* ch, const int* cw, const float* gy,
                     float* gx, float* gw, float* gnp, float* ws, int64_t ws_floats,
                     hipStream_t st);

}  // namespace slg
