// Bit-packed building blocks behind the silogic.bitpacking API on gfx950:
// FC LUT layers of arity up to 6, packed unfold, packed OR-pool of any
// window, and k-ary LUT trees over unfolded conv inputs.
//
// Packed layouts (64 samples per word, sample b at bit b % 64 of word
// b / 64): FC activations [dim, nw]; conv activations [C, L, nw] with
// L = H * W row-major. Every kernel walks (row, word) with the word index
// fastest, so the lanes of a wave read and write consecutive words.
//
// LUT convention (silogic/nodes.py:186-187, functional.py:169-173): the
// address of a k-input node is sum_j x_j << j (input 0 is the least
// significant bit). A truth table of up to 64 entries is one uint64 word,
// entry e at bit e. It is evaluated as a multiplexer tree: level 0 picks
// between entries 2m and 2m+1 by input 0, level j by input j, so a k-input
// node costs 2^k - 1 bit-selects per 32-bit half.
#include "slg_common.h"

namespace slg {

constexpr int kMaxLutArity = 6;
constexpr int kMaxTreeLeaves = 64;
constexpr int kMaxTreeNodes = 64;

__device__ inline uint32_t sel32(uint32_t m, uint32_t x, uint32_t y) { return (m & x) | (~m & y); }

// One k-input LUT on packed words: in[j] is input j's word.
__device__ inline uint64_t lut_word(const uint64_t* in, int k, uint64_t tt) {
  uint32_t tlo[32], thi[32];  // level values, low and high halves
  const int half = 1 << (k - 1);
#pragma unroll
  for (int m = 0; m < 32; ++m) {
    if (m < half) {
      const uint32_t e0 = (tt >> (2 * m)) & 1ull ? 0xFFFFFFFFu : 0u;
      const uint32_t e1 = (tt >> (2 * m + 1)) & 1ull ? 0xFFFFFFFFu : 0u;
      tlo[m] = sel32((uint32_t)in[0], e1, e0);
      thi[m] = sel32((uint32_t)(in[0] >> 32), e1, e0);
    }
  }
#pragma unroll
  for (int j = 1; j < kMaxLutArity; ++j) {
    if (j < k) {
      const uint32_t xl = (uint32_t)in[j], xh = (uint32_t)(in[j] >> 32);
      const int cnt = 1 << (k - 1 - j);
#pragma unroll
      for (int m = 0; m < 16; ++m) {
        if (m < cnt) {
          tlo[m] = sel32(xl, tlo[2 * m + 1], tlo[2 * m]);
          thi[m] = sel32(xh, thi[2 * m + 1], thi[2 * m]);
        }
      }
    }
  }
  return ((uint64_t)thi[0] << 32) | tlo[0];
}

// out[o][w] = LUT_o(x[idx[o][0]][w], ..., x[idx[o][k-1]][w])
// (silogic/bitpacking/packed_layer.py:121-178 semantics).
__global__ void __launch_bounds__(256) fc_lut_kernel(const uint64_t* __restrict__ x, int IN, int nw,
                                                     const int* __restrict__ idx, int k,
                                                     const uint64_t* __restrict__ tt, int OUT,
                                                     uint64_t* __restrict__ out) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (int64_t)OUT * nw) return;
  const int o = (int)(t / nw), w = (int)(t - (int64_t)o * nw);
  uint64_t in[kMaxLutArity];
#pragma unroll
  for (int j = 0; j < kMaxLutArity; ++j) {
    if (j < k) {
      const int i = min(max(idx[(int64_t)o * k + j], 0), IN - 1);
      in[j] = x[(int64_t)i * nw + w];
    } else {
      in[j] = 0;
    }
  }
  out[t] = lut_word(in, k, tt[o]);
}

// out[c*kh*kw + dy*kw + dx][l][w] = x[c][(hy*stride - pad + dy) * W + ...][w],
// zero outside the image (packed_layer.py:224-283).
__global__ void __launch_bounds__(256) packed_unfold_kernel(const uint64_t* __restrict__ x, int C,
                                                            int H, int W, int nw, int kh, int kw,
                                                            int stride, int pad, int Ho, int Wo,
                                                            uint64_t* __restrict__ out) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t Lo = (int64_t)Ho * Wo;
  if (t >= (int64_t)C * kh * kw * Lo * nw) return;
  const int w = (int)(t % nw);
  const int64_t r = t / nw;
  const int l = (int)(r % Lo);
  const int p = (int)(r / Lo);
  const int c = p / (kh * kw), q = p - c * kh * kw;
  const int dy = q / kw, dx = q - dy * kw;
  const int hy = (l / Wo) * stride - pad + dy, hx = (l % Wo) * stride - pad + dx;
  uint64_t v = 0;
  if (hy >= 0 && hy < H && hx >= 0 && hx < W) v = x[((int64_t)c * H * W + hy * W + hx) * nw + w];
  out[t] = v;
}

// OR over ps x ps windows, floor sizes (packed_layer.py:286-319).
__global__ void __launch_bounds__(256) packed_or_pool_kernel(const uint64_t* __restrict__ x, int C,
                                                             int H, int W, int nw, int ps,
                                                             uint64_t* __restrict__ out) {
  const int Ho = H / ps, Wo = W / ps;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (int64_t)C * Ho * Wo * nw) return;
  const int w = (int)(t % nw);
  const int64_t r = t / nw;
  const int l = (int)(r % ((int64_t)Ho * Wo));
  const int c = (int)(r / ((int64_t)Ho * Wo));
  const int oy = (l / Wo) * ps, ox = (l % Wo) * ps;
  const uint64_t* base = x + (int64_t)c * H * W * nw + w;
  uint64_t v = 0;
  for (int dy = 0; dy < ps; ++dy)
    for (int dx = 0; dx < ps; ++dx) v |= base[((int64_t)(oy + dy) * W + ox + dx) * nw];
  out[t] = v;
}

// LUT tree over unfolded input xu [P, L, nw]: output n gathers its k^d
// leaves leaf[n][.] (flat P indices), then level i combines k consecutive
// values per node; tables [N][nodes] hold the nodes level-major (level 0
// first, node m of a level combines values k*m .. k*m+k-1 of the level
// below), one LUT word per node (packed_layer.py:324-540).
__global__ void __launch_bounds__(256) lut_tree_kernel(const uint64_t* __restrict__ xu, int P, int L,
                                                       int nw, int N, const int* __restrict__ leaf,
                                                       int leaves, int k, int depth, int nodes,
                                                       const uint64_t* __restrict__ tables,
                                                       uint64_t* __restrict__ out) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (int64_t)N * L * nw) return;
  const int w = (int)(t % nw);
  const int64_t r = t / nw;
  const int l = (int)(r % L);
  const int n = (int)(r / L);
  uint64_t v[kMaxTreeLeaves];
  for (int j = 0; j < leaves; ++j) {
    const int p = min(max(leaf[(int64_t)n * leaves + j], 0), P - 1);
    v[j] = xu[((int64_t)p * L + l) * nw + w];
  }
  int cnt = leaves, nb = 0;
  for (int i = 0; i < depth; ++i) {
    const int m_cnt = cnt / k;
    for (int m = 0; m < m_cnt; ++m)
      v[m] = lut_word(v + k * m, k, tables[(int64_t)n * nodes + nb + m]);
    nb += m_cnt;
    cnt = m_cnt;
  }
  out[t] = v[0];
}

}  // namespace slg

using namespace slg;

extern "C" {

int slg_fc_lut_hard(const uint64_t* x, int64_t IN, int64_t nw, const int32_t* idx, int32_t arity,
                    const uint64_t* tt, int64_t OUT, uint64_t* out, slg_stream_t stream) {
  SLG_REQUIRE(idx && tt && ((x && out) || nw == 0), SLG_E_ARG, "fc_lut_hard: null pointer");
  SLG_REQUIRE(arity >= 1 && arity <= kMaxLutArity, SLG_E_UNSUPPORTED, "fc_lut_hard: arity %d",
              arity);
  SLG_REQUIRE(IN > 0 && OUT > 0 && nw >= 0 && IN < (1LL << 31) && OUT * nw < (1LL << 40),
              SLG_E_SHAPE, "fc_lut_hard: bad sizes");
  if (nw == 0) return 0;
  const int64_t n = OUT * nw;
  hipLaunchKernelGGL(fc_lut_kernel, dim3((unsigned)cdiv(n, 256)), dim3(256), 0, as_stream(stream),
                     x, (int)IN, (int)nw, idx, arity, tt, (int)OUT, out);
  SLG_LAUNCH_CHECK("fc_lut_hard");
  return 0;
}

int slg_packed_unfold(const uint64_t* x, int64_t C, int64_t H, int64_t W, int64_t nw, int32_t kh,
                      int32_t kw, int32_t stride, int32_t pad, uint64_t* out,
                      slg_stream_t stream) {
  SLG_REQUIRE(C > 0 && H > 0 && W > 0 && nw >= 0 && kh > 0 && kw > 0 && stride > 0 && pad >= 0 &&
                  C * H * W < (1LL << 31),
              SLG_E_SHAPE, "packed_unfold: bad sizes");
  const int64_t Ho = (H + 2 * pad - kh) / stride + 1, Wo = (W + 2 * pad - kw) / stride + 1;
  SLG_REQUIRE(Ho > 0 && Wo > 0, SLG_E_SHAPE, "packed_unfold: empty output");
  const int64_t n = C * kh * kw * Ho * Wo * nw;
  if (n == 0) return 0;
  SLG_REQUIRE(x && out, SLG_E_ARG, "packed_unfold: null pointer");
  SLG_REQUIRE(n < (1LL << 40), SLG_E_SHAPE, "packed_unfold: too large");
  hipLaunchKernelGGL(packed_unfold_kernel, dim3((unsigned)cdiv(n, 256)), dim3(256), 0,
                     as_stream(stream), x, (int)C, (int)H, (int)W, (int)nw, kh, kw, stride, pad,
                     (int)Ho, (int)Wo, out);
  SLG_LAUNCH_CHECK("packed_unfold");
  return 0;
}

int slg_packed_or_pool(const uint64_t* x, int64_t C, int64_t H, int64_t W, int64_t nw, int32_t ps,
                       uint64_t* out, slg_stream_t stream) {
  SLG_REQUIRE(C > 0 && H > 0 && W > 0 && nw >= 0 && ps > 0 && C * H * W < (1LL << 31),
              SLG_E_SHAPE, "packed_or_pool: bad sizes");
  const int64_t n = C * (H / ps) * (W / ps) * nw;
  if (n == 0) return 0;  // empty output: nothing to read or write
  SLG_REQUIRE(x && out, SLG_E_ARG, "packed_or_pool: null pointer");
  hipLaunchKernelGGL(packed_or_pool_kernel, dim3((unsigned)cdiv(n, 256)), dim3(256), 0,
                     as_stream(stream), x, (int)C, (int)H, (int)W, (int)nw, ps, out);
  SLG_LAUNCH_CHECK("packed_or_pool");
  return 0;
}

int slg_lut_tree_hard(const uint64_t* xu, int64_t P, int64_t L, int64_t nw, int64_t N,
                      const int32_t* leaf, int32_t arity, int32_t depth, const uint64_t* tables,
                      uint64_t* out, slg_stream_t stream) {
  SLG_REQUIRE(leaf && tables && ((xu && out) || nw == 0), SLG_E_ARG, "lut_tree: null pointer");
  SLG_REQUIRE(arity >= 2 && arity <= kMaxLutArity && depth >= 1, SLG_E_UNSUPPORTED,
              "lut_tree: arity %d depth %d", arity, depth);
  int64_t leaves = 1, nodes = 0;
  for (int i = 0; i < depth; ++i) {
    nodes += leaves;
    leaves *= arity;
    SLG_REQUIRE(leaves <= kMaxTreeLeaves, SLG_E_UNSUPPORTED, "lut_tree: more than %d leaves",
                kMaxTreeLeaves);
  }
  SLG_REQUIRE(nodes <= kMaxTreeNodes, SLG_E_UNSUPPORTED, "lut_tree: too many nodes");
  SLG_REQUIRE(P > 0 && L > 0 && N > 0 && nw >= 0 && P * L < (1LL << 31) && N * L * nw < (1LL << 40),
              SLG_E_SHAPE, "lut_tree: bad sizes");
  const int64_t n = N * L * nw;
  if (n == 0) return 0;
  hipLaunchKernelGGL(lut_tree_kernel, dim3((unsigned)cdiv(n, 256)), dim3(256), 0,
                     as_stream(stream), xu, (int)P, (int)L, (int)nw, (int)N, leaf, (int)leaves,
                     arity, depth, (int)nodes, tables, out);
  SLG_LAUNCH_CHECK("lut_tree");
  return 0;
}

}  // extern "C"
