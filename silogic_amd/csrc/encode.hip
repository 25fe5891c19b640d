// Input encoders on the GPU (the step before the gate layers): fixed
// thermometer codes (silogic/data.py:23-40 binarize, 75-89 binarize_spatial),
// edge-detector bits (data.py:102-131 edge_bits) and the learnable
// thermometer (silogic/encoders.py:12-49). Each writes the reference's uint8
// layout, and the thermometers also write the packed layouts the hard kernels
// read ([F, nw] rows, which is also the conv [C, H*W, nw] layout, or [nw, F]
// word-major for the fused FC network), so a batch goes from pixels to
// packed bits in one pass.
//
// binarize / binarize_spatial share one memory order: feature t*D + d is
// (x[b][d] >= thr[t]) for D = C*H*W (the spatial form's channel t*C + c).
// The learnable thermometer orders f*bits + i: (x[b][f] - thr[f][i] > 0).
#include <math.h>

#include "pack_cols.h"
#include "slg_common.h"

namespace slg {

// Input value: fp32, or a pixel byte taken as x / 255 in fp32 (the value
// the reference's loaders compute, data.py:49-57, before encoding).
template <typename TX>
__device__ inline float in_val(const TX* __restrict__ x, int64_t i) {
  if constexpr (sizeof(TX) == 1) return (float)x[i] / 255.0f;
  else return x[i];
}

// Bit of feature j of sample b. FIXED: j = t*D + d, x >= thr[t]; else
// (learned): j = f*T + i, x[f] - thr[f*T + i] > 0.
template <bool FIXED, typename TX>
__device__ inline bool encode_bit(const TX* __restrict__ x, int64_t b, int D, int T,
                                  const float* __restrict__ thr, int j) {
  if constexpr (FIXED) {
    const int t = j / D, d = j - t * D;
    return in_val(x, b * D + d) >= thr[t];
  } else {
    const int f = j / T;
    return in_val(x, b * D + f) - thr[j] > 0.0f;
  }
}

template <typename TX>
__global__ void __launch_bounds__(256) encode_u8_kernel(const TX* __restrict__ x, int B, int D,
                                                        int T, const float* __restrict__ thr,
                                                        int fixed, uint8_t* __restrict__ out) {
  const int64_t F = (int64_t)D * T;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)B * F) return;
  const int64_t b = i / F;
  const int j = (int)(i - b * F);
  out[i] = (fixed ? encode_bit<true>(x, b, D, T, thr, j) : encode_bit<false>(x, b, D, T, thr, j))
               ? 1 : 0;
}

// Smallest byte k in [0, 256] whose value k / 255 passes the test against
// threshold t (256: none). The test is monotone in the byte (a correctly
// rounded k / 255 does not decrease with k), so byte >= k is the same bit
// as the fp32 test on byte / 255.
template <bool FIXED>
__device__ inline int byte_cut(float t) {
  int lo = 0, hi = 256;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    const float v = (float)mid / 255.0f;
    const bool pass = FIXED ? (v >= t) : (v - t > 0.0f);
    if (pass) hi = mid; else lo = mid + 1;
  }
  return lo;
}

template <bool FIXED, typename TX>
__device__ inline bool pass_bit(TX v, float th, int cut) {
  if constexpr (sizeof(TX) == 1) return (int)v >= cut;
  else return FIXED ? (v >= th) : (v - th > 0.0f);
}

// Packed: a lane takes V consecutive features and builds their words over
// the 64 samples of one word in registers (pack_cols); the four waves of a
// workgroup take four consecutive words. V = 4 reads the four features of a
// row as one vector (fixed thresholds, D % 4 == 0, aligned input).
// LAYOUT 0: xp [F, nw]; 1: xp [nw, F].
template <bool FIXED, int LAYOUT, typename TX, int V>
__global__ void __launch_bounds__(256) encode_pack_kernel(const TX* __restrict__ x, int B, int D,
                                                          int T, const float* __restrict__ thr,
                                                          int nw, int ftiles,
                                                          uint64_t* __restrict__ xp) {
  const int lane = threadIdx.x & 63;
  const int w = (int)(blockIdx.x / (uint32_t)ftiles) * 4 + (int)(threadIdx.x >> 6);
  const int F = D * T;
  const int j0 = (int)(blockIdx.x % (uint32_t)ftiles) * 64 * V + lane * V;
  if (w >= nw || j0 >= F) return;                       // no barriers below
  int src[V], cut[V];
  float th[V];
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const int j = min(j0 + v, F - 1);                    // tail lanes: stores are guarded
    if constexpr (FIXED) {
      const int t = j / D;
      src[v] = j - t * D;
      th[v] = thr[t];
    } else {
      src[v] = j / T;
      th[v] = thr[j];
    }
    cut[v] = sizeof(TX) == 1 ? byte_cut<FIXED>(th[v]) : 0;
  }
  uint64_t word[V];
  pack_cols<V, V == 4>(x + (int64_t)w * 64 * D, D, min(64, B - w * 64), src,
                       [&](TX v, int f) { return pass_bit<FIXED>(v, th[f], cut[f]); }, word);
#pragma unroll
  for (int v = 0; v < V; ++v) {
    if (j0 + v < F) {
      if constexpr (LAYOUT == 0) xp[(int64_t)(j0 + v) * nw + w] = word[v];
      else xp[(int64_t)w * F + j0 + v] = word[v];
    }
  }
}

// Edge bits: per colour channel c the 3x3 responses Sobel-x, Sobel-y,
// Laplacian (zero padding), channel-major as the grouped convolution
// (data.py:123-126), then per level t two planes (> t, < -t); output channel
// (ti*2 + s) * 3C + c*3 + det (data.py:127-131). One thread per pixel of
// one (sample, colour); the three responses are sums of the nine taps in
// row-major order.
__constant__ float c_edge_k[3][9] = {
    {-1.f, 0.f, 1.f, -2.f, 0.f, 2.f, -1.f, 0.f, 1.f},   // Sobel-x
    {-1.f, -2.f, -1.f, 0.f, 0.f, 0.f, 1.f, 2.f, 1.f},   // Sobel-y (its transpose)
    {0.f, 1.f, 0.f, 1.f, -4.f, 1.f, 0.f, 1.f, 0.f}};    // Laplacian

__global__ void __launch_bounds__(256) edge_bits_kernel(const float* __restrict__ x, int N, int C,
                                                        int H, int W, const float* __restrict__ thr,
                                                        int T, uint8_t* __restrict__ out) {
  const int64_t HW = (int64_t)H * W;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)N * C * HW) return;
  const int64_t nc = i / HW;
  const int hw = (int)(i - nc * HW);
  const int n = (int)(nc / C), c = (int)(nc - (int64_t)n * C);
  const int h = hw / W, w = hw - h * W;
  const float* xc = x + nc * HW;
  float v[9];
#pragma unroll
  for (int dy = 0; dy < 3; ++dy)
#pragma unroll
    for (int dx = 0; dx < 3; ++dx) {
      const int y = h + dy - 1, xx = w + dx - 1;
      v[dy * 3 + dx] = (y >= 0 && y < H && xx >= 0 && xx < W) ? xc[(int64_t)y * W + xx] : 0.0f;
    }
  float r[3];
#pragma unroll
  for (int det = 0; det < 3; ++det) {
    float s = 0.0f;
#pragma unroll
    for (int q = 0; q < 9; ++q) s = fmaf(c_edge_k[det][q], v[q], s);
    r[det] = s;
  }
  const int64_t planes = (int64_t)2 * T * 3 * C;
  uint8_t* on = out + (int64_t)n * planes * HW + hw;
  for (int ti = 0; ti < T; ++ti) {
    const float t = thr[ti];
#pragma unroll
    for (int det = 0; det < 3; ++det) {
      on[((int64_t)(ti * 2) * 3 * C + c * 3 + det) * HW] = r[det] > t ? 1 : 0;
      on[((int64_t)(ti * 2 + 1) * 3 * C + c * 3 + det) * HW] = r[det] < -t ? 1 : 0;
    }
  }
}

// Learnable thermometer, soft path: the value is the hard bit (the
// reference's hard + soft - soft.detach(), encoders.py:40-44, without its
// fp32 rounding); the gradient is that of sigmoid((x - t) * scale).
// gx [B,F] = sum_i g[b][f*T+i] * ds; gt partials over sample ranges.
__global__ void __launch_bounds__(256) learned_thermo_bwd_x_kernel(
    const float* __restrict__ x, int B, int F, int T, const float* __restrict__ thr, float scale,
    const float* __restrict__ g, float* __restrict__ gx) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)B * F) return;
  const int64_t b = i / F;
  const int f = (int)(i - b * F);
  const float xv = x[i];
  float acc = 0.0f;
  for (int k = 0; k < T; ++k) {
    const float s = 1.0f / (1.0f + expf(-(xv - thr[f * T + k]) * scale));
    acc = fmaf(g[b * (int64_t)F * T + f * T + k], s * (1.0f - s) * scale, acc);
  }
  gx[i] = acc;
}

// part [NR][F*T]: range r sums samples [r*spr, (r+1)*spr) in order.
__global__ void __launch_bounds__(256) learned_thermo_bwd_t_kernel(
    const float* __restrict__ x, int B, int F, int T, const float* __restrict__ thr, float scale,
    const float* __restrict__ g, int spr, float* __restrict__ part) {
  const int j = blockIdx.x * blockDim.x + threadIdx.x;
  const int r = blockIdx.y;
  if (j >= F * T) return;
  const int f = j / T;
  const float t = thr[j];
  float acc = 0.0f;
  const int b1 = min(B, (r + 1) * spr);
  for (int b = r * spr; b < b1; ++b) {
    const float s = 1.0f / (1.0f + expf(-(x[(int64_t)b * F + f] - t) * scale));
    acc = fmaf(g[(int64_t)b * F * T + j], -(s * (1.0f - s) * scale), acc);
  }
  part[(int64_t)r * F * T + j] = acc;
}

__global__ void __launch_bounds__(256) learned_thermo_sum_kernel(const float* __restrict__ part,
                                                                 int NR, int n,
                                                                 float* __restrict__ gt) {
  const int j = blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= n) return;
  float s = 0.0f;
  for (int r = 0; r < NR; ++r) s += part[(int64_t)r * n + j];
  gt[j] = s;
}

static int learned_ranges(int64_t B, int64_t FT) {
  const int64_t tiles = cdiv(FT, 256);
  return (int)std::max<int64_t>(1, std::min<int64_t>(std::min<int64_t>(B, 1024),
                                                     cdiv(8 * device_cus(), tiles)));
}

template <typename TX>
static int encode_thermo_t(const TX* x, int64_t B, int64_t D, const float* thr, int T,
                           int learned, int layout, void* out, hipStream_t st) {
  const int64_t F = D * T;
  if (layout == 2) {
    hipLaunchKernelGGL(encode_u8_kernel<TX>, dim3((unsigned)cdiv(B * F, 256)), dim3(256), 0, st,
                       x, (int)B, (int)D, T, thr, learned ? 0 : 1, (uint8_t*)out);
    SLG_LAUNCH_CHECK("encode_thermometer");
    return 0;
  }
  const bool vec = !learned && D % 4 == 0 && (uintptr_t)x % (4 * sizeof(TX)) == 0;
  const int64_t nw = cdiv(B, 64), ftiles = cdiv(F, vec ? 256 : 64);
  SLG_REQUIRE(cdiv(nw, 4) * ftiles < (1LL << 31), SLG_E_SHAPE,
              "encode_thermometer: grid too large");
  const dim3 grid((unsigned)(cdiv(nw, 4) * ftiles));
  uint64_t* xp = (uint64_t*)out;
#define SLG_ENC(FX, LY, V)                                                                 \
  hipLaunchKernelGGL((encode_pack_kernel<FX, LY, TX, V>), grid, dim3(256), 0, st, x, (int)B, \
                     (int)D, T, thr, (int)nw, (int)ftiles, xp)
  if (vec) {
    if (layout == 0) SLG_ENC(true, 0, 4); else SLG_ENC(true, 1, 4);
  } else if (!learned) {
    if (layout == 0) SLG_ENC(true, 0, 1); else SLG_ENC(true, 1, 1);
  } else {
    if (layout == 0) SLG_ENC(false, 0, 1); else SLG_ENC(false, 1, 1);
  }
#undef SLG_ENC
  SLG_LAUNCH_CHECK("encode_thermometer");
  return 0;
}

}  // namespace slg

using namespace slg;

extern "C" {

int slg_encode_thermometer(const void* x, int32_t dtype, int64_t B, int64_t D, const float* thr,
                           int32_t T, int32_t learned, int32_t layout, void* out,
                           slg_stream_t stream) {
  SLG_REQUIRE(thr && out && (x || B == 0), SLG_E_ARG, "encode_thermometer: null pointer");
  SLG_REQUIRE(B >= 0 && D > 0 && T >= 1 && layout >= 0 && layout <= 2 && (dtype == 0 || dtype == 1) &&
                  D * T < (1LL << 31) && B < (1LL << 31) && B * D * T < (1LL << 46),
              SLG_E_SHAPE, "encode_thermometer: bad sizes");
  if (B == 0) return 0;
  hipStream_t st = as_stream(stream);
  return dtype == 1 ? encode_thermo_t((const uint8_t*)x, B, D, thr, T, learned, layout, out, st)
                    : encode_thermo_t((const float*)x, B, D, thr, T, learned, layout, out, st);
}

int slg_edge_bits(const float* x, int64_t N, int64_t C, int64_t H, int64_t W, const float* thr,
                  int32_t T, uint8_t* out, slg_stream_t stream) {
  SLG_REQUIRE(thr && ((x && out) || N == 0), SLG_E_ARG, "edge_bits: null pointer");
  SLG_REQUIRE(N >= 0 && C > 0 && H > 0 && W > 0 && T >= 1 && N * C * H * W < (1LL << 40) &&
                  H * W < (1LL << 31),
              SLG_E_SHAPE, "edge_bits: bad sizes");
  if (N == 0) return 0;
  const int64_t n = N * C * H * W;
  hipLaunchKernelGGL(edge_bits_kernel, dim3((unsigned)cdiv(n, 256)), dim3(256), 0,
                     as_stream(stream), x, (int)N, (int)C, (int)H, (int)W, thr, T, out);
  SLG_LAUNCH_CHECK("edge_bits");
  return 0;
}

int64_t slg_learned_thermo_bwd_workspace(int64_t B, int64_t F, int32_t T) {
  if (B < 0 || F <= 0 || T < 1) return -1;
  return (int64_t)learned_ranges(std::max<int64_t>(B, 1), F * T) * F * T;
}

int slg_learned_thermo_bwd(const float* x, int64_t B, int64_t F, int32_t T, const float* thr,
                           float scale, const float* g, float* gx, float* gt, float* workspace,
                           int64_t workspace_floats, slg_stream_t stream) {
  SLG_REQUIRE(thr && ((x && g) || B == 0) && (workspace || !gt), SLG_E_ARG,
              "learned_thermo_bwd: null pointer");
  SLG_REQUIRE(B >= 0 && F > 0 && T >= 1 && F * T < (1LL << 31) && B < (1LL << 31), SLG_E_SHAPE,
              "learned_thermo_bwd: bad sizes");
  hipStream_t st = as_stream(stream);
  const int64_t FT = F * T;
  if (gx && B > 0) {
    hipLaunchKernelGGL(learned_thermo_bwd_x_kernel, dim3((unsigned)cdiv(B * F, 256)), dim3(256),
                       0, st, x, (int)B, (int)F, T, thr, scale, g, gx);
  }
  if (gt) {
    const int NR = learned_ranges(std::max<int64_t>(B, 1), FT);
    SLG_REQUIRE(workspace_floats >= (int64_t)NR * FT, SLG_E_ARG,
                "learned_thermo_bwd: workspace of %lld floats, %lld needed",
                (long long)workspace_floats, (long long)NR * FT);
    const int spr = (int)cdiv(std::max<int64_t>(B, 1), NR);
    if (B > 0)
      hipLaunchKernelGGL(learned_thermo_bwd_t_kernel, dim3((unsigned)cdiv(FT, 256), (unsigned)NR),
                         dim3(256), 0, st, x, (int)B, (int)F, T, thr, scale, g, spr, workspace);
    hipLaunchKernelGGL(learned_thermo_sum_kernel, dim3((unsigned)cdiv(FT, 256)), dim3(256), 0, st,
                       workspace, B > 0 ? NR : 0, (int)FT, gt);
  }
  SLG_LAUNCH_CHECK("learned_thermo_bwd");
  return 0;
}

}  // extern "C"
