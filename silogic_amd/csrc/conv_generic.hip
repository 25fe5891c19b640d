// ConvLogicTree node trees of any kind the reference builds, soft forward
// and backward for gfx950, reading the input image through the caches
// instead of staging it in LDS (so it also takes images larger than LDS):
//   * gate16 trees (binary BasisProj nodes, silogic/layers.py:388-401),
//   * walsh trees (binary nodes y = sigmoid(z / tau), nodes.py:145-150; the
//     caller passes z's (a, b)-space coefficients times 1/tau),
//   * multilinear and hybrid LUT trees of arity A and depth D
//     (layers.py:432-446 over nodes.py:174-178 / 202-206): level i has
//     A^(D-1-i) nodes per channel, node m combines values A*m .. A*m+A-1 of
//     the level below, leaf j of a node is address bit j.
// Node parameters per channel are level-major, [N][NN][P] with NN the node
// count and P = 4 (gate16 / walsh coefficients) or 2^A (LUT values).
//
// Forward: one thread per (sample, channel, output position); the channel
// is uniform over a workgroup, so taps, weights and node parameters are
// uniform loads. For a pooled output the tree is evaluated at the four
// window positions and the maximum kept (the fused OrPool, layers.py:558).
//
// Backward (atomic-free, every sum in a fixed order): the same threads
// route the pooled gradient to the first window position holding the
// maximum (F.max_pool2d), back-propagate through the tree, and
//   * reduce the node-parameter and leaf-weight gradients over the wave with
//     a xor butterfly; lane 0 writes one partial per wave, and a second
//     kernel adds the partials of each channel in slot order;
//   * write each leaf's gradient at its (unpooled) position to gleaf, which
//     a gather kernel turns into the input gradient: every input pixel sums,
//     in ascending reference order, the leaf gradients of the taps that read
//     it (the reference's two-pass atomic-free scheme, kernels/conv.py:
//     247-345, built here on the shared reference table).
#include <math.h>

#include <type_traits>

#include "ref_table.h"

namespace slg {

__host__ __device__ constexpr int ipow(int a, int d) { return d == 0 ? 1 : a * ipow(a, d - 1); }

template <int NODE, int A, int D>
struct GenTree {
  static constexpr int NLEAF = ipow(A, D);
  static constexpr int NN = (NLEAF - 1) / (A - 1);
  static constexpr int P = (NODE == SLG_NODE_GATE16 || NODE == SLG_NODE_WALSH) ? 4 : (1 << A);
};

// Node ids of level i start at lvl_off[i] (level 0 is the level above the
// leaves) and its inputs at value index lvl_in[i] (0 = the leaves).
template <int A, int D>
struct GenLevels {
  int off[D], in[D], cnt[D];
  __host__ __device__ constexpr GenLevels() : off(), in(), cnt() {
    int o = 0, c = ipow(A, D - 1);
    for (int i = 0; i < D; ++i) {
      off[i] = o;
      cnt[i] = c;
      in[i] = i == 0 ? 0 : ipow(A, D) + off[i - 1];
      o += c;
      c /= A;
    }
  }
};

__device__ inline float gen_sigmoid(float z) { return 1.0f / (1.0f + expf(-z)); }

// Value of one node with children c[0..A) and parameters p (uniform).
template <int NODE, int A>
__device__ inline float gen_node(const float* c, const float* __restrict__ p) {
  if constexpr (NODE == SLG_NODE_GATE16 || NODE == SLG_NODE_WALSH) {
    const float a = c[0], b = c[1];
    const float z = p[0] + p[1] * a + p[2] * b + p[3] * (a * b);
    if constexpr (NODE == SLG_NODE_WALSH) return gen_sigmoid(z);
    return z;
  } else if constexpr (NODE == SLG_NODE_HYBRID) {
    int addr = 0;
#pragma unroll
    for (int j = 0; j < A; ++j) addr |= (c[j] >= 0.5f ? 1 : 0) << j;
    return p[addr];
  } else {
    // the reference's product form (nodes.py:174-178): corner factors a_j or
    // (1 - a_j) multiplied in leaf order, then sum_p w_p * s_p added in
    // corner order, each operation rounded on its own (no contraction), so
    // that values the reference computes as equal (near-ties of a flat tree
    // at binary leaves) are equal here too: the pooled routing depends on it
#pragma clang fp contract(off)
    constexpr int PP = 1 << A;
    float acc = 0.0f;
#pragma unroll
    for (int e = 0; e < PP; ++e) {
      float w = (e & 1) ? c[0] : 1.0f - c[0];
#pragma unroll
      for (int j = 1; j < A; ++j) w = w * ((e >> j) & 1 ? c[j] : 1.0f - c[j]);
      const float term = w * p[e];
      acc = e == 0 ? term : acc + term;
    }
    return acc;
  }
}

// Leaf values at output position (yy, xx) of sample b, channel n: the
// softmax-weighted sum over K taps (zero padding outside the image).
template <int NLEAF>
__device__ inline void gen_leaves(float (&v)[NLEAF], const float* __restrict__ xb, int C, int H,
                                  int W, int n, int K, int kernel, int pad, int yy, int xx,
                                  const float* __restrict__ w, const int* __restrict__ cm,
                                  const int* __restrict__ ch, const int* __restrict__ cw) {
#pragma unroll
  for (int l = 0; l < NLEAF; ++l) {
    float acc = 0.0f;
    for (int k = 0; k < K; ++k) {
      const int r = (n * NLEAF + l) * K + k;
      const int c = min(max(cm[r], 0), C - 1);
      const int iy = yy + min(max(ch[r], 0), kernel - 1) - pad;
      const int ix = xx + min(max(cw[r], 0), kernel - 1) - pad;
      const bool in = iy >= 0 && iy < H && ix >= 0 && ix < W;
      const float xv = in ? xb[((int64_t)c * H + iy) * W + ix] : 0.0f;
      acc = fmaf(w ? w[r] : 1.0f, xv, acc);
    }
    v[l] = acc;
  }
}

// All node values of the tree (level-major after the leaves): val[0..NLEAF)
// are the leaves, val[NLEAF + id] node id.
template <int NODE, int A, int D>
__device__ inline void gen_eval(float* val, const float* __restrict__ par) {
  using T = GenTree<NODE, A, D>;
  constexpr GenLevels<A, D> L{};
#pragma unroll
  for (int i = 0; i < D; ++i) {
#pragma unroll
    for (int m = 0; m < L.cnt[i]; ++m)
      val[T::NLEAF + L.off[i] + m] =
          gen_node<NODE, A>(val + L.in[i] + A * m, par + (L.off[i] + m) * T::P);
  }
}

template <int NODE, int A, int D>
__global__ void __launch_bounds__(256)
conv_generic_fwd_kernel(const float* __restrict__ x, int C, int H, int W, int N, int K, int kernel,
                        int pad, int pool, int Ho, int Wo, int nblk, const float* __restrict__ np,
                        const float* __restrict__ w, const int* __restrict__ cm,
                        const int* __restrict__ ch, const int* __restrict__ cw,
                        float* __restrict__ out) {
  using T = GenTree<NODE, A, D>;
  const int n = blockIdx.y;
  const int b = blockIdx.x / nblk;
  const int p = (blockIdx.x - b * nblk) * 256 + threadIdx.x;
  if (p >= Ho * Wo) return;
  const int oy = p / Wo, ox = p - (p / Wo) * Wo;
  const float* xb = x + (int64_t)b * C * H * W;
  const float* par = np + (int64_t)n * T::NN * T::P;
  float best = -INFINITY;
  const int nq = pool ? 4 : 1;
  for (int q = 0; q < nq; ++q) {
    const int yy = pool ? 2 * oy + (q >> 1) : oy, xx = pool ? 2 * ox + (q & 1) : ox;
    float val[T::NLEAF + T::NN];
    float (&lv)[T::NLEAF] = *reinterpret_cast<float(*)[T::NLEAF]>(val);
    gen_leaves<T::NLEAF>(lv, xb, C, H, W, n, K, kernel, pad, yy, xx, w, cm, ch, cw);
    gen_eval<NODE, A, D>(val, par);
    best = fmaxf(best, val[T::NLEAF + T::NN - 1]);
  }
  out[((int64_t)b * N + n) * Ho * Wo + p] = best;
}

// Sum over the 64 lanes of a wave; lane 0's result is the same bits on
// every call (a fixed butterfly).
__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Gradients of one node (children c, value y, parameters p) for output
// gradient g: parameter gradients gp[0..P) and child gradients gc[0..A).
template <int NODE, int A>
__device__ inline void gen_node_bwd(const float* c, float y, const float* __restrict__ p, float g,
                                    float* gp, float* gc) {
  if constexpr (NODE == SLG_NODE_GATE16 || NODE == SLG_NODE_WALSH) {
    const float a = c[0], b = c[1];
    const float dz = NODE == SLG_NODE_WALSH ? g * (y * (1.0f - y)) : g;
    gp[0] = dz;
    gp[1] = dz * a;
    gp[2] = dz * b;
    gp[3] = dz * (a * b);
    gc[0] = dz * (p[1] + p[3] * b);
    gc[1] = dz * (p[2] + p[3] * a);
  } else {
    // multilinear form (the hybrid node's surrogate gradient too): corner
    // weights prod_j (bit_j(e) ? c_j : 1 - c_j)
    constexpr int PP = 1 << A;
    float wt[PP];
    wt[0] = 1.0f;
#pragma unroll
    for (int j = 0; j < A; ++j) {
#pragma unroll
      for (int e = 0; e < (1 << j); ++e) {
        wt[e + (1 << j)] = wt[e] * c[j];
        wt[e] = wt[e] * (1.0f - c[j]);
      }
    }
#pragma unroll
    for (int e = 0; e < PP; ++e) gp[e] = g * wt[e];
    // d/dc_j: the differences across bit j interpolated over the other leaves
#pragma unroll
    for (int j = 0; j < A; ++j) {
      float acc = 0.0f;
#pragma unroll
      for (int e = 0; e < PP; ++e) {
        if (e & (1 << j)) continue;
        float o = 1.0f;
#pragma unroll
        for (int i = 0; i < A; ++i) {
          if (i == j) continue;
          o *= (e >> i) & 1 ? c[i] : 1.0f - c[i];
        }
        acc = fmaf(p[e | (1 << j)] - p[e], o, acc);
      }
      gc[j] = g * acc;
    }
  }
}

template <int NODE, int A, int D>
__global__ void __launch_bounds__(256)
conv_generic_bwd_kernel(const float* __restrict__ x, int C, int H, int W, int N, int K, int kernel,
                        int pad, int pool, int Hf, int Wf, int Ho, int Wo, int nblk, int b_base,
                        const float* __restrict__ np, const float* __restrict__ w,
                        const int* __restrict__ cm, const int* __restrict__ ch,
                        const int* __restrict__ cw, const float* __restrict__ gy,
                        float* __restrict__ part, int64_t slots, float* __restrict__ gleaf) {
  using T = GenTree<NODE, A, D>;
  constexpr int NV = T::NLEAF + T::NN;
  const int n = blockIdx.y;
  const int bl = blockIdx.x / nblk;  // sample within the chunk
  const int pb = blockIdx.x - bl * nblk;
  const int b = b_base + bl;
  const int p = pb * 256 + threadIdx.x;
  const bool active = p < Ho * Wo;
  const int pc = active ? p : 0;
  const int oy = pc / Wo, ox = pc - (pc / Wo) * Wo;
  const float* xb = x + (int64_t)b * C * H * W;
  const float* par = np + (int64_t)n * T::NN * T::P;
  float val[NV];
  float (&lv)[T::NLEAF] = *reinterpret_cast<float(*)[T::NLEAF]>(val);
  // routed window position: the first (row-major) holding the maximum
  int qs = 0;
  if (pool) {
    float best = -INFINITY;
    for (int q = 0; q < 4; ++q) {
      gen_leaves<T::NLEAF>(lv, xb, C, H, W, n, K, kernel, pad, 2 * oy + (q >> 1), 2 * ox + (q & 1),
                           w, cm, ch, cw);
      gen_eval<NODE, A, D>(val, par);
      const float v = val[NV - 1];
      if (v > best || q == 0) {
        best = v;
        qs = q;
      }
    }
  }
  const int yy = pool ? 2 * oy + (qs >> 1) : oy, xx = pool ? 2 * ox + (qs & 1) : ox;
  gen_leaves<T::NLEAF>(lv, xb, C, H, W, n, K, kernel, pad, yy, xx, w, cm, ch, cw);
  gen_eval<NODE, A, D>(val, par);

  float gv[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) gv[i] = 0.0f;
  gv[NV - 1] = active ? gy[((int64_t)b * N + n) * Ho * Wo + p] : 0.0f;

  const int lane = threadIdx.x & 63;
  const int64_t slot = ((int64_t)blockIdx.x) * 4 + (threadIdx.x >> 6);
  constexpr int R = T::NN * T::P + T::NLEAF * 8;  // row stride of part (K <= 8)
  float* prow = part + ((int64_t)n * slots + slot) * R;
  constexpr GenLevels<A, D> L{};
#pragma unroll
  for (int i = D - 1; i >= 0; --i) {
#pragma unroll
    for (int m = 0; m < L.cnt[i]; ++m) {
      const int id = L.off[i] + m;
      float gp[T::P], gc[A];
      gen_node_bwd<NODE, A>(val + L.in[i] + A * m, val[T::NLEAF + id], par + id * T::P,
                            gv[T::NLEAF + id], gp, gc);
#pragma unroll
      for (int j = 0; j < A; ++j) gv[L.in[i] + A * m + j] = gc[j];
#pragma unroll
      for (int e = 0; e < T::P; ++e) {
        const float s = wave_sum(gp[e]);
        if (lane == 0) prow[id * T::P + e] = s;
      }
    }
  }
  // leaf weights and the leaf gradients at the routed position
  const int HfWf = Hf * Wf;
  float* gl = gleaf + (((int64_t)bl * N + n) * T::NLEAF) * HfWf + yy * Wf + xx;
#pragma unroll
  for (int l = 0; l < T::NLEAF; ++l) {
    if (active) gl[(int64_t)l * HfWf] = gv[l];
    for (int k = 0; k < K; ++k) {
      const int r = (n * T::NLEAF + l) * K + k;
      const int c = min(max(cm[r], 0), C - 1);
      const int iy = yy + min(max(ch[r], 0), kernel - 1) - pad;
      const int ix = xx + min(max(cw[r], 0), kernel - 1) - pad;
      const bool in = iy >= 0 && iy < H && ix >= 0 && ix < W;
      const float xv = in ? xb[((int64_t)c * H + iy) * W + ix] : 0.0f;
      const float s = wave_sum(gv[l] * xv);
      if (lane == 0) prow[T::NN * T::P + l * 8 + k] = s;
    }
  }
}

// Fill n floats with zero (a kernel, not hipMemsetAsync, so that a captured
// graph holds no memset node).
__global__ void __launch_bounds__(256) gen_zero_kernel(float* __restrict__ p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t j = i; j < n; j += stride) p[j] = 0.0f;
}

// Keys of the reference table: the (clamped) input channel of every tap.
__global__ void __launch_bounds__(256) gen_keys_kernel(const int* __restrict__ cm, int64_t R, int C,
                                                       int* __restrict__ keys) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r < R) keys[r] = min(max(cm[r], 0), C - 1);
}

// Sum of the wave partials per channel, in slot order, into gnp / gw.
__global__ void __launch_bounds__(256) gen_reduce_kernel(const float* __restrict__ part, int N,
                                                         int64_t slots, int R, int NPAR, int NLEAF,
                                                         int K, float* __restrict__ gnp,
                                                         float* __restrict__ gw) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int per = NPAR + NLEAF * K;
  if (t >= (int64_t)N * per) return;
  const int n = (int)(t / per), j = (int)(t - (int64_t)n * per);
  int col;
  float* dst;
  if (j < NPAR) {
    col = j;
    dst = gnp ? gnp + (int64_t)n * NPAR + j : nullptr;
  } else {
    const int l = (j - NPAR) / K, k = (j - NPAR) - ((j - NPAR) / K) * K;
    col = NPAR + l * 8 + k;
    dst = gw ? gw + ((int64_t)n * NLEAF + l) * K + k : nullptr;
  }
  if (!dst) return;
  const float* src = part + (int64_t)n * slots * R + col;
  float acc = 0.0f;
  for (int64_t s = 0; s < slots; ++s) acc += src[s * R];
  *dst = acc;
}

// Input gradient of Bc samples: pixel (b, c, iy, ix) sums gleaf at the
// positions of the taps that read it, taps in ascending reference order.
__global__ void __launch_bounds__(256)
gen_gather_gx_kernel(const float* __restrict__ gleaf, RefTable tab, const int* __restrict__ ch,
                     const int* __restrict__ cw, const float* __restrict__ w, int Bc, int C, int H,
                     int W, int N, int NLEAF, int K, int kernel, int pad, int Hf, int Wf,
                     float* __restrict__ gx) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t HW = (int64_t)H * W;
  if (t >= (int64_t)Bc * C * HW) return;
  const int bl = (int)(t / (C * HW));
  const int64_t rem = t - (int64_t)bl * C * HW;
  const int c = (int)(rem / HW);
  const int pix = (int)(rem - (int64_t)c * HW);
  const int iy = pix / W, ix = pix - (pix / W) * W;
  const int e0 = tab.start[c], e1 = tab.start[c + 1];
  const int64_t HfWf = (int64_t)Hf * Wf;
  float acc = 0.0f;
  for (int e = e0; e < e1; ++e) {
    const int r = tab.sorted[e];
    const int n = r / (NLEAF * K);
    const int l = (r / K) - n * NLEAF;
    const int oy = iy + pad - min(max(ch[r], 0), kernel - 1);
    const int ox = ix + pad - min(max(cw[r], 0), kernel - 1);
    if (oy >= 0 && oy < Hf && ox >= 0 && ox < Wf)
      acc = fmaf(gleaf[(((int64_t)bl * N + n) * NLEAF + l) * HfWf + oy * Wf + ox], w ? w[r] : 1.0f,
                 acc);
  }
  gx[t] = acc;
}

// (A, D) pairs with kernels: leaves A^D <= 36.
template <typename F>
static int gen_dispatch(int node, int A, int D, F&& f) {
  auto ad = [&](auto nd) -> int {
    constexpr int NODE = decltype(nd)::value;
    if (A == 2) {
      switch (D) {
        case 1: return f(nd, std::integral_constant<int, 2>{}, std::integral_constant<int, 1>{});
        case 2: return f(nd, std::integral_constant<int, 2>{}, std::integral_constant<int, 2>{});
        case 3: return f(nd, std::integral_constant<int, 2>{}, std::integral_constant<int, 3>{});
        case 4: return f(nd, std::integral_constant<int, 2>{}, std::integral_constant<int, 4>{});
        case 5: return f(nd, std::integral_constant<int, 2>{}, std::integral_constant<int, 5>{});
        default: return SLG_E_UNSUPPORTED;
      }
    }
    if constexpr (NODE == SLG_NODE_MULTILINEAR2 || NODE == SLG_NODE_HYBRID) {
      if (A == 3) {
        switch (D) {
          case 1: return f(nd, std::integral_constant<int, 3>{}, std::integral_constant<int, 1>{});
          case 2: return f(nd, std::integral_constant<int, 3>{}, std::integral_constant<int, 2>{});
          case 3: return f(nd, std::integral_constant<int, 3>{}, std::integral_constant<int, 3>{});
          default: return SLG_E_UNSUPPORTED;
        }
      }
      if (A == 4 && (D == 1 || D == 2))
        return D == 1 ? f(nd, std::integral_constant<int, 4>{}, std::integral_constant<int, 1>{})
                      : f(nd, std::integral_constant<int, 4>{}, std::integral_constant<int, 2>{});
      if (A == 5 && (D == 1 || D == 2))
        return D == 1 ? f(nd, std::integral_constant<int, 5>{}, std::integral_constant<int, 1>{})
                      : f(nd, std::integral_constant<int, 5>{}, std::integral_constant<int, 2>{});
      if (A == 6 && (D == 1 || D == 2))
        return D == 1 ? f(nd, std::integral_constant<int, 6>{}, std::integral_constant<int, 1>{})
                      : f(nd, std::integral_constant<int, 6>{}, std::integral_constant<int, 2>{});
    }
    return SLG_E_UNSUPPORTED;
  };
  switch (node) {
    case SLG_NODE_GATE16:
      return A == 2 ? ad(std::integral_constant<int, SLG_NODE_GATE16>{}) : SLG_E_UNSUPPORTED;
    case SLG_NODE_WALSH:
      return A == 2 ? ad(std::integral_constant<int, SLG_NODE_WALSH>{}) : SLG_E_UNSUPPORTED;
    case SLG_NODE_MULTILINEAR2: return ad(std::integral_constant<int, SLG_NODE_MULTILINEAR2>{});
    case SLG_NODE_HYBRID: return ad(std::integral_constant<int, SLG_NODE_HYBRID>{});
    default: return SLG_E_UNSUPPORTED;
  }
}

bool conv_generic_supported(int node, int depth, int arity) {
  const int A = (node == SLG_NODE_GATE16 || node == SLG_NODE_WALSH) ? 2 : arity;
  return gen_dispatch(node, A, depth, [](auto, auto, auto) { return 0; }) == 0;
}

int conv_generic_params(int node, int depth, int arity) {
  const int A = (node == SLG_NODE_GATE16 || node == SLG_NODE_WALSH) ? 2 : arity;
  const int nleaf = ipow(A, depth);
  const int nn = (nleaf - 1) / (A - 1);
  return nn * ((node == SLG_NODE_GATE16 || node == SLG_NODE_WALSH) ? 4 : (1 << A));
}

int conv_generic_fwd(const float* x, int64_t B, int64_t C, int64_t H, int64_t W, int64_t N,
                     int node, int depth, int arity, int K, int kernel, int pad, bool pool,
                     const float* np, const float* w, const int* cm, const int* ch, const int* cw,
                     float* out, int64_t Ho, int64_t Wo, hipStream_t st) {
  const int A = (node == SLG_NODE_GATE16 || node == SLG_NODE_WALSH) ? 2 : arity;
  const int64_t nblk = cdiv(Ho * Wo, 256);
  SLG_REQUIRE(nblk * B < (1LL << 31) && N < 65536 && C * H * W < (1LL << 31), SLG_E_SHAPE,
              "conv_soft (generic): too large");
  return gen_dispatch(node, A, depth, [&](auto nd, auto a_, auto d_) -> int {
    constexpr int NODE = decltype(nd)::value, AA = decltype(a_)::value, DD = decltype(d_)::value;
    hipLaunchKernelGGL((conv_generic_fwd_kernel<NODE, AA, DD>),
                       dim3((unsigned)(nblk * B), (unsigned)N), dim3(256), 0, st, x, (int)C, (int)H,
                       (int)W, (int)N, K, kernel, pad, (int)pool, (int)Ho, (int)Wo, (int)nblk, np, w,
                       cm, ch, cw, out);
    SLG_LAUNCH_CHECK("conv_soft (generic)");
    return 0;
  });
}

// Backward plan: workspace (floats) = part | gleaf chunk | keys | table.
struct GenBwdPlan {
  int64_t nblk, slots, R, Bc, part, gleaf, keys, table;
  int64_t total() const { return part + gleaf + keys + table; }
};

static constexpr int64_t kGleafCap = int64_t(64) << 20;  // floats per sample chunk

static GenBwdPlan gen_bwd_plan(int64_t B, int64_t C, int64_t Hf, int64_t Wf, int64_t N, int node,
                               int depth, int arity, int K, int64_t Ho, int64_t Wo) {
  GenBwdPlan p{};
  const int A = (node == SLG_NODE_GATE16 || node == SLG_NODE_WALSH) ? 2 : arity;
  const int64_t nleaf = ipow(A, depth);
  p.nblk = cdiv(Ho * Wo, 256);
  p.slots = std::max<int64_t>(B, 1) * p.nblk * 4;
  p.R = conv_generic_params(node, depth, arity) + nleaf * 8;
  const int64_t per_sample = N * nleaf * Hf * Wf;
  p.Bc = std::max<int64_t>(1, std::min<int64_t>(std::max<int64_t>(B, 1), kGleafCap / std::max<int64_t>(per_sample, 1)));
  p.part = (N * p.slots * p.R + 3) & ~int64_t(3);
  p.gleaf = (p.Bc * per_sample + 3) & ~int64_t(3);
  const int64_t refs = N * nleaf * K;
  p.keys = (refs + 3) & ~int64_t(3);
  p.table = ref_table_ints(refs, C);
  return p;
}

int64_t conv_generic_bwd_workspace(int64_t B, int64_t C, int64_t H, int64_t W, int64_t N, int node,
                                   int depth, int arity, int K, int pad, bool pool) {
  if (!conv_generic_supported(node, depth, arity)) return -1;
  const int64_t kernel = 2 * pad + 1;
  const int64_t Hf = H + 2 * pad - kernel + 1, Wf = W + 2 * pad - kernel + 1;
  const int64_t Ho = pool ? Hf / 2 : Hf, Wo = pool ? Wf / 2 : Wf;
  return gen_bwd_plan(B, C, Hf, Wf, N, node, depth, arity, K, Ho, Wo).total();
}

int conv_generic_bwd(const float* x, int64_t B, int64_t C, int64_t H, int64_t W, int64_t N,
                     int node, int depth, int arity, int K, int pad, bool pool, const float* np,
                     const float* w, const int* cm, const int* ch, const int* cw, const float* gy,
                     float* gx, float* gw, float* gnp, float* ws, int64_t ws_floats,
                     hipStream_t st) {
  const int A = (node == SLG_NODE_GATE16 || node == SLG_NODE_WALSH) ? 2 : arity;
  const int kernel = 2 * pad + 1;
  const int64_t Hf = H + 2 * pad - kernel + 1, Wf = W + 2 * pad - kernel + 1;
  const int64_t Ho = pool ? Hf / 2 : Hf, Wo = pool ? Wf / 2 : Wf;
  SLG_REQUIRE(K >= 1 && K <= 8, SLG_E_SHAPE, "conv_soft_bwd (generic): K=%d outside 1..8", K);
  const GenBwdPlan p = gen_bwd_plan(B, C, Hf, Wf, N, node, depth, arity, K, Ho, Wo);
  SLG_REQUIRE(ws_floats >= p.total(), SLG_E_ARG, "conv_soft_bwd (generic): workspace of %lld floats, %lld needed",
              (long long)ws_floats, (long long)p.total());
  SLG_REQUIRE(p.nblk * p.Bc < (1LL << 31) && N < 65536 && p.slots < (1LL << 40), SLG_E_SHAPE,
              "conv_soft_bwd (generic): too large");
  const int nleaf = ipow(A, depth);
  const int npar = conv_generic_params(node, depth, arity);
  float* part = ws;
  float* gleaf = part + p.part;
  int* keys = reinterpret_cast<int*>(gleaf + p.gleaf);
  int* tab_ws = keys + p.keys;
  const int64_t refs = N * nleaf * K;
  RefTable tab{};
  if (gx) {
    hipLaunchKernelGGL(gen_keys_kernel, dim3((unsigned)cdiv(refs, 256)), dim3(256), 0, st, cm, refs,
                       (int)C, keys);
    SLG_LAUNCH_CHECK("conv_soft_bwd (generic) keys");
    const int rc = build_ref_table(keys, refs, C, tab_ws, st, &tab);
    if (rc) return rc;
  }
  if (B == 0) {
    // no samples: zero parameter gradients (a sum over no slots)
    if (gw || gnp) {
      hipLaunchKernelGGL(gen_reduce_kernel, dim3((unsigned)cdiv(N * (npar + nleaf * K), 256)),
                         dim3(256), 0, st, part, (int)N, (int64_t)0, (int)p.R, npar, nleaf, K, gnp, gw);
      SLG_LAUNCH_CHECK("conv_soft_bwd (generic) reduce");
    }
    return 0;
  }
  const int64_t per_sample = N * nleaf * Hf * Wf;
  for (int64_t b0 = 0; b0 < B; b0 += p.Bc) {
    const int64_t bc = std::min<int64_t>(p.Bc, B - b0);
    const int64_t nz = bc * per_sample;
    hipLaunchKernelGGL(gen_zero_kernel, dim3((unsigned)std::min<int64_t>(cdiv(nz, 256), 65536)),
                       dim3(256), 0, st, gleaf, nz);
    SLG_LAUNCH_CHECK("conv_soft_bwd (generic) zero");
    const int rc = gen_dispatch(node, A, depth, [&](auto nd, auto a_, auto d_) -> int {
      constexpr int NODE = decltype(nd)::value, AA = decltype(a_)::value, DD = decltype(d_)::value;
      // part rows of this chunk start at slot b0 * nblk * 4
      hipLaunchKernelGGL((conv_generic_bwd_kernel<NODE, AA, DD>),
                         dim3((unsigned)(p.nblk * bc), (unsigned)N), dim3(256), 0, st, x, (int)C,
                         (int)H, (int)W, (int)N, K, kernel, pad, (int)pool, (int)Hf, (int)Wf, (int)Ho,
                         (int)Wo, (int)p.nblk, (int)b0, np, w, cm, ch, cw, gy,
                         part + b0 * p.nblk * 4 * p.R, p.slots, gleaf);
      SLG_LAUNCH_CHECK("conv_soft_bwd (generic)");
      return 0;
    });
    if (rc) return rc;
    if (gx) {
      const int64_t nt = bc * C * H * W;
      hipLaunchKernelGGL(gen_gather_gx_kernel, dim3((unsigned)cdiv(nt, 256)), dim3(256), 0, st,
                         gleaf, tab, ch, cw, w, (int)bc, (int)C, (int)H, (int)W, (int)N, nleaf, K,
                         kernel, pad, (int)Hf, (int)Wf, gx + b0 * C * H * W);
      SLG_LAUNCH_CHECK("conv_soft_bwd (generic) gather");
    }
  }
  if (gw || gnp) {
    hipLaunchKernelGGL(gen_reduce_kernel, dim3((unsigned)cdiv(N * (npar + nleaf * K), 256)),
                       dim3(256), 0, st, part, (int)N, p.slots, (int)p.R, npar, nleaf, K, gnp, gw);
    SLG_LAUNCH_CHECK("conv_soft_bwd (generic) reduce");
  }
  return 0;
}

// ---------------------------------------------------------------------------
// hard (bit-packed) node trees
// ---------------------------------------------------------------------------
// Per channel: the argmax leaf taps (cm << 8 | ch << 4 | cw, as the conv hard
// prep) and one truth table per node, level-major, bit e = the node's output
// at the address e = sum_j child_j << j:
//   gate16: the argmax gate's table (functional.py:50-66) with address
//     (a << 1) | b rewritten to a | b << 1;
//   walsh: z > 0 at the corner, z = ((t0 + t1 u0) + t2 u1) + t3 u0 u1 with
//     u = 2x - 1 summed left to right as the reference's fp32 sum over the
//     size-4 dim (nodes.py:152-156);
//   multilinear / hybrid: logits[e] > 0 (nodes.py:183-189).
// raw[i] holds level i's parameters, row n * m_i + m for node m of channel
// n (m_i nodes per channel at level i, layers.py:351-358, 432-446).
struct GenHardPrep {
  const int* cm;
  const int* ch;
  const int* cw;
  const float* conn;
  const float* raw[8];
  int* leaf;
  uint64_t* tables;
  int N, K, node, A, D, nleaf, nn;
};

__constant__ uint8_t c_tt16_gen[16] = {0x0, 0x8, 0x4, 0xC, 0x2, 0xA, 0x6, 0xE,
                                       0x1, 0x9, 0x5, 0xD, 0x3, 0xB, 0x7, 0xF};

__global__ void __launch_bounds__(128) conv_generic_hard_prep_kernel(GenHardPrep P) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= P.N) return;
  for (int l = 0; l < P.nleaf; ++l) {
    const int64_t base = ((int64_t)n * P.nleaf + l) * P.K;
    int c = 0;
    if (P.conn) {  // first index of the maximum, as torch.argmax (layers.py:511-513)
      float bv = P.conn[base];
      for (int j = 1; j < P.K; ++j)
        if (P.conn[base + j] > bv) { bv = P.conn[base + j]; c = j; }
    }
    P.leaf[n * P.nleaf + l] =
        (P.cm[base + c] << 8) | ((P.ch[base + c] & 15) << 4) | (P.cw[base + c] & 15);
  }
  int id = 0;
  int m_i = 1;
  for (int i = 1; i < P.D; ++i) m_i *= P.A;  // nodes per channel at level 0
  for (int i = 0; i < P.D; ++i, m_i /= P.A) {
    for (int m = 0; m < m_i; ++m, ++id) {
      const int64_t row = (int64_t)n * m_i + m;
      uint64_t t = 0;
      if (P.node == SLG_NODE_GATE16) {
        const float* g = P.raw[i] + row * 16;
        int bi = 0;
        float bv = g[0];
        for (int q = 1; q < 16; ++q)
          if (g[q] > bv) { bv = g[q]; bi = q; }
        const uint32_t tt = c_tt16_gen[bi];  // bit (a << 1) | b
        for (int e = 0; e < 4; ++e) {
          const int a = e & 1, b = e >> 1;
          if ((tt >> ((a << 1) | b)) & 1u) t |= 1ull << e;
        }
      } else if (P.node == SLG_NODE_WALSH) {
        const float* th = P.raw[i] + row * 4;
        for (int e = 0; e < 4; ++e) {
          const float u0 = (e & 1) ? 1.0f : -1.0f, u1 = (e >> 1) ? 1.0f : -1.0f;
          float z = th[0];  // products by +-1 are exact
          z = z + th[1] * u0;
          z = z + th[2] * u1;
          z = z + th[3] * (u0 * u1);
          if (z > 0.0f) t |= 1ull << e;
        }
      } else {
        const int pn = 1 << P.A;
        for (int e = 0; e < pn; ++e)
          if (P.raw[i][row * pn + e] > 0.0f) t |= 1ull << e;
      }
      P.tables[(int64_t)n * P.nn + id] = t;
    }
  }
}

// Node output words: a Shannon multiplexer tree over the node's children,
// child j = address bit j.
template <int A>
__device__ inline uint64_t gen_mux(const uint64_t* c, uint64_t T) {
  uint64_t t[1 << (A - 1)];
#pragma unroll
  for (int m = 0; m < (1 << (A - 1)); ++m) {
    const uint64_t e0 = 0ull - ((T >> (2 * m)) & 1ull);
    const uint64_t e1 = 0ull - ((T >> (2 * m + 1)) & 1ull);
    t[m] = (c[0] & e1) | (~c[0] & e0);
  }
#pragma unroll
  for (int j = 1; j < A; ++j) {
#pragma unroll
    for (int m = 0; m < (1 << (A - 1 - j)); ++m) t[m] = (c[j] & t[2 * m + 1]) | (~c[j] & t[2 * m]);
  }
  return t[0];
}

// Packed conv tree + optional 2x2 OR pool: xp [C,H,W,nw] -> out [N,Ho,Wo,nw].
// Threads walk (output position, word), word fastest; the channel is the
// grid's y index, so leaf taps and tables are uniform.
template <int A, int D>
__global__ void __launch_bounds__(256)
conv_generic_hard_kernel(const uint64_t* __restrict__ xp, int C, int H, int W, int nw, int N,
                         const int* __restrict__ leaf, const uint64_t* __restrict__ tables,
                         int kernel, int pad, int pool, uint64_t* __restrict__ out, int Ho, int Wo) {
  constexpr int NLEAF = ipow(A, D);
  constexpr int NN = (NLEAF - 1) / (A - 1);
  constexpr GenLevels<A, D> L{};
  const int n = blockIdx.y;
  const int P = Ho * Wo;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)P * nw) return;
  const int p = (int)(i / nw), wd = (int)(i - (int64_t)p * nw);
  const int oy = (p / Wo) * (pool ? 2 : 1), ox = (p % Wo) * (pool ? 2 : 1);
  const uint64_t* T = tables + (int64_t)n * NN;
  uint64_t acc = 0;
  const int nq = pool ? 4 : 1;
  for (int q = 0; q < nq; ++q) {
    const int py = oy + (q >> 1), px = ox + (q & 1);
    uint64_t v[NLEAF + NN];
#pragma unroll
    for (int l = 0; l < NLEAF; ++l) {
      const int code = leaf[n * NLEAF + l];
      const int lc = min(max(code >> 8, 0), C - 1);
      const int iy = py + min((code >> 4) & 15, kernel - 1) - pad;
      const int ix = px + min(code & 15, kernel - 1) - pad;
      v[l] = (iy >= 0 && iy < H && ix >= 0 && ix < W)
                 ? xp[(((int64_t)lc * H + iy) * W + ix) * nw + wd]
                 : 0ull;
    }
#pragma unroll
    for (int lv = 0; lv < D; ++lv) {
#pragma unroll
      for (int m = 0; m < L.cnt[lv]; ++m)
        v[NLEAF + L.off[lv] + m] = gen_mux<A>(v + L.in[lv] + A * m, T[L.off[lv] + m]);
    }
    acc |= v[NLEAF + NN - 1];
  }
  out[((int64_t)n * P + p) * nw + wd] = acc;
}

template <typename F>
static int gen_hard_dispatch(int A, int D, F&& f) {
  // the node kind only changes the tables, so any kind with these (A, D)
  return gen_dispatch(SLG_NODE_MULTILINEAR2, A, D, [&](auto, auto a_, auto d_) { return f(a_, d_); });
}

}  // namespace slg

using namespace slg;

extern "C" {

int slg_conv_tree_hard_prep(const int32_t* cm, const int32_t* ch, const int32_t* cw,
                            const float* conn, int64_t N, int32_t K, int32_t node_kind,
                            int32_t depth, int32_t arity, const float* const* raw, int32_t* leaf,
                            uint64_t* tables, slg_stream_t stream) {
  SLG_REQUIRE(cm && ch && cw && raw && leaf && tables, SLG_E_ARG, "conv_tree_hard_prep: null pointer");
  SLG_REQUIRE(node_kind >= SLG_NODE_GATE16 && node_kind <= SLG_NODE_HYBRID, SLG_E_ARG,
              "conv_tree_hard_prep: node_kind %d", node_kind);
  SLG_REQUIRE(conv_generic_supported(node_kind, depth, arity), SLG_E_UNSUPPORTED,
              "conv_tree_hard_prep: node %d depth %d arity %d", node_kind, depth, arity);
  SLG_REQUIRE(N > 0 && N < (1LL << 20) && K >= 1 && K <= 64, SLG_E_SHAPE,
              "conv_tree_hard_prep: sizes");
  GenHardPrep P{};
  P.cm = cm; P.ch = ch; P.cw = cw; P.conn = conn;
  P.A = (node_kind == SLG_NODE_GATE16 || node_kind == SLG_NODE_WALSH) ? 2 : arity;
  P.D = depth;
  for (int i = 0; i < depth; ++i) {
    SLG_REQUIRE(raw[i], SLG_E_ARG, "conv_tree_hard_prep: null level %d", i);
    P.raw[i] = raw[i];
  }
  P.leaf = leaf; P.tables = tables;
  P.N = (int)N; P.K = K; P.node = node_kind;
  P.nleaf = ipow(P.A, depth);
  P.nn = (P.nleaf - 1) / (P.A - 1);
  hipLaunchKernelGGL(conv_generic_hard_prep_kernel, dim3((unsigned)cdiv(N, 128)), dim3(128), 0,
                     as_stream(stream), P);
  SLG_LAUNCH_CHECK("conv_tree_hard_prep");
  return 0;
}

int slg_conv_tree_hard_fwd(const uint64_t* xp, int64_t C, int64_t H, int64_t W, int64_t nw,
                           int64_t N, int32_t arity, int32_t depth, const int32_t* leaf,
                           const uint64_t* tables, int32_t kernel, int32_t pad, int32_t pool,
                           uint64_t* out, slg_stream_t stream) {
  SLG_REQUIRE(xp && leaf && tables && out, SLG_E_ARG, "conv_tree_hard: null pointer");
  SLG_REQUIRE(conv_generic_supported(SLG_NODE_MULTILINEAR2, depth, arity), SLG_E_UNSUPPORTED,
              "conv_tree_hard: arity %d depth %d", arity, depth);
  SLG_REQUIRE(C > 0 && H > 0 && W > 0 && nw > 0 && N > 0 && N < 65536 && kernel >= 1 &&
                  kernel <= 15 && pad >= 0 && 2 * pad + 1 == kernel,
              SLG_E_SHAPE, "conv_tree_hard: bad sizes");
  const int64_t Hf = H + 2 * pad - kernel + 1, Wf = W + 2 * pad - kernel + 1;
  const int64_t Ho = pool ? Hf / 2 : Hf, Wo = pool ? Wf / 2 : Wf;
  if (Ho == 0 || Wo == 0) return 0;
  const int64_t n = Ho * Wo * nw;
  SLG_REQUIRE(n < (1LL << 40) && C * H * W * nw < (1LL << 40), SLG_E_SHAPE, "conv_tree_hard: too large");
  return gen_hard_dispatch(arity, depth, [&](auto a_, auto d_) -> int {
    constexpr int AA = decltype(a_)::value, DD = decltype(d_)::value;
    hipLaunchKernelGGL((conv_generic_hard_kernel<AA, DD>), dim3((unsigned)cdiv(n, 256), (unsigned)N),
                       dim3(256), 0, as_stream(stream), xp, (int)C, (int)H, (int)W, (int)nw, (int)N,
                       leaf, tables, kernel, pad, (int)pool, out, (int)Ho, (int)Wo);
    SLG_LAUNCH_CHECK("conv_tree_hard");
    return 0;
  });
}

}  // extern "C"
