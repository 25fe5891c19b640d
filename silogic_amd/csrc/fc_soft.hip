// FC soft forward for gfx950: Top-K gather + 4-coefficient node, and the
// parameter prep / GroupSum kernels around it.
//
// Design (one layer, x [B,IN] -> y [B,OUT]):
//   * A workgroup owns a tile of S consecutive samples and a chunk of
//     outputs. It stages the S input rows in LDS transposed and
//     sample-interleaved, lds[i][g] = float4 of samples 4g..4g+3 of input i
//     (S = 1, 2 use float / float2), so one ds_read_b128 per candidate
//     fetches 4 samples. Random-address b128 reads measured on gfx950 reach
//     ~80 B/clk/CU, b64 ~68, b32 ~33: wider is better for random gathers.
//   * Lanes walk outputs. Each lane holds its output's 2K candidate indices,
//     2K weights and 4 node coefficients in registers and reuses them for all
//     S samples, so parameter traffic is 144/S bytes per sample-output.
//   * Output stores are coalesced along the output dimension.
//   * The tile/chunk index is remapped so chunks of one tile run on the same
//     XCD and share its L2 copy of the input rows.
#include "slg_common.h"

namespace slg {

template <int V> struct vecf;
template <> struct vecf<1> { using t = float; };
template <> struct vecf<2> { using t = float2; };
template <> struct vecf<4> { using t = float4; };

__device__ inline float lanev(float v, int) { return v; }
__device__ inline float lanev(float2 v, int i) { return i == 0 ? v.x : v.y; }
__device__ inline float lanev(float4 v, int i) {
  return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w));
}
__device__ inline void fma_acc(float& acc, float w, float v) { acc = fmaf(w, v, acc); }
__device__ inline void fma_acc(float2& acc, float w, float2 v) {
  acc.x = fmaf(w, v.x, acc.x);
  acc.y = fmaf(w, v.y, acc.y);
}
__device__ inline void fma_acc(float4& acc, float w, float4 v) {
  acc.x = fmaf(w, v.x, acc.x);
  acc.y = fmaf(w, v.y, acc.y);
  acc.z = fmaf(w, v.z, acc.z);
  acc.w = fmaf(w, v.w, acc.w);
}
template <typename T> __device__ inline T zero_vec();
template <> __device__ inline float zero_vec<float>() { return 0.f; }
template <> __device__ inline float2 zero_vec<float2>() { return make_float2(0.f, 0.f); }
template <> __device__ inline float4 zero_vec<float4>() { return make_float4(0.f, 0.f, 0.f, 0.f); }

__device__ inline float sigmoidf_(float z) { return 1.0f / (1.0f + expf(-z)); }

// Node evaluation on the two gathered operands (silogic/nodes.py:86-91 for
// gate16, the warp_logic form of kernels/warp.py:14-31 for walsh,
// nodes.py:174-178 with n = 2 for multilinear).
template <int NODE>
__device__ inline float node_eval(float a, float b, const float4& p, float inv_tau) {
  if constexpr (NODE == SLG_NODE_GATE16) {
    return p.x + p.y * a + p.z * b + p.w * (a * b);
  } else if constexpr (NODE == SLG_NODE_WALSH) {
    return sigmoidf_((p.x + p.y * a + p.z * b + p.w * (a * b)) * inv_tau);
  } else {
    // corners P = 0:(0,0) 1:(1,0) 2:(0,1) 3:(1,1) (bit j of P = slot j)
    const float ua = 1.0f - a, ub = 1.0f - b;
    return (((ua * ub) * p.x + (a * ub) * p.y) + (ua * b) * p.z) + (a * b) * p.w;
  }
}

// KC = compile-time candidate count (0 = runtime K <= 16, scalar loads).
template <int NODE, int KC, int S>
__global__ void __launch_bounds__(1024)
fc_soft_kernel(const float* __restrict__ x, int B, int IN, int OUT, int Kr,
               const int* __restrict__ ca, const int* __restrict__ cb, int cstride,
               const float* __restrict__ wa, const float* __restrict__ wb, int wstride,
               const float* __restrict__ np, float inv_tau, float* __restrict__ y,
               int n_chunks, int chunk) {
  constexpr int V = S >= 4 ? 4 : S;
  constexpr int G = S / V;
  constexpr int KM = KC > 0 ? KC : 16;
  using vt = typename vecf<V>::t;
  extern __shared__ __align__(16) unsigned char smem[];
  vt* lds = reinterpret_cast<vt*>(smem);
  const int K = KC > 0 ? KC : Kr;

  const uint32_t lid = xcd_logical_id(blockIdx.x, gridDim.x);
  const int tile = (int)(lid / (uint32_t)n_chunks);
  const int ch = (int)(lid % (uint32_t)n_chunks);
  const int b0 = tile * S;

  // Stage S rows transposed: lds[i*G + g] = samples b0+gV .. b0+gV+V-1 of input i.
  for (int g = 0; g < G; ++g) {
    for (int i = threadIdx.x; i < IN; i += blockDim.x) {
      float t[V];
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const int b = b0 + g * V + v;
        t[v] = (b < B) ? __builtin_nontemporal_load(x + (int64_t)b * IN + i) : 0.0f;
      }
      vt val;
      if constexpr (V == 1) val = t[0];
      else if constexpr (V == 2) val = make_float2(t[0], t[1]);
      else val = make_float4(t[0], t[1], t[2], t[3]);
      lds[i * G + g] = val;
    }
  }
  __syncthreads();

  const int o_begin = ch * chunk;
  const int o_end = min(OUT, o_begin + chunk);
  for (int o = o_begin + threadIdx.x; o < o_end; o += blockDim.x) {
    int ia[KM], ib[KM];
    float fa[KM], fb[KM];
    if constexpr (KC > 0 && (KC % 4) == 0) {
#pragma unroll
      for (int q = 0; q < KC / 4; ++q) {
        const int4 a4 = *reinterpret_cast<const int4*>(ca + (int64_t)o * cstride + 4 * q);
        const int4 b4 = *reinterpret_cast<const int4*>(cb + (int64_t)o * cstride + 4 * q);
        const float4 u4 = *reinterpret_cast<const float4*>(wa + (int64_t)o * wstride + 4 * q);
        const float4 v4 = *reinterpret_cast<const float4*>(wb + (int64_t)o * wstride + 4 * q);
        ia[4 * q + 0] = a4.x; ia[4 * q + 1] = a4.y; ia[4 * q + 2] = a4.z; ia[4 * q + 3] = a4.w;
        ib[4 * q + 0] = b4.x; ib[4 * q + 1] = b4.y; ib[4 * q + 2] = b4.z; ib[4 * q + 3] = b4.w;
        fa[4 * q + 0] = u4.x; fa[4 * q + 1] = u4.y; fa[4 * q + 2] = u4.z; fa[4 * q + 3] = u4.w;
        fb[4 * q + 0] = v4.x; fb[4 * q + 1] = v4.y; fb[4 * q + 2] = v4.z; fb[4 * q + 3] = v4.w;
      }
    } else {
#pragma unroll
      for (int k = 0; k < KM; ++k) {
        if (k < K) {
          ia[k] = ca[(int64_t)o * cstride + k];
          ib[k] = cb[(int64_t)o * cstride + k];
          fa[k] = wa ? wa[(int64_t)o * wstride + k] : 1.0f;
          fb[k] = wb ? wb[(int64_t)o * wstride + k] : 1.0f;
        } else {
          ia[k] = 0; ib[k] = 0; fa[k] = 0.f; fb[k] = 0.f;
        }
      }
    }
#pragma unroll
    for (int k = 0; k < KM; ++k) {  // clamp into the staged rows, scale to slots
      ia[k] = min(max(ia[k], 0), IN - 1) * G;
      ib[k] = min(max(ib[k], 0), IN - 1) * G;
    }
    const float4 p = reinterpret_cast<const float4*>(np)[o];
    for (int g = 0; g < G; ++g) {
      vt A = zero_vec<vt>(), Bv = zero_vec<vt>();
#pragma unroll
      for (int k = 0; k < KM; ++k) {
        if (KC > 0 || k < K) {
          fma_acc(A, fa[k], lds[ia[k] + g]);
          fma_acc(Bv, fb[k], lds[ib[k] + g]);
        }
      }
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const int b = b0 + g * V + v;
        if (b < B) y[(int64_t)b * OUT + o] = node_eval<NODE>(lanev(A, v), lanev(Bv, v), p, inv_tau);
      }
    }
  }
}

struct SoftArgs {
  const float* x; int64_t B, IN, OUT; int K;
  const int* ca; const int* cb; int cstride;
  const float* wa; const float* wb; int wstride;
  const float* np; float inv_tau; float* y;
  int S, threads;
};

template <int NODE, int KC, int S>
static int launch_soft_s(const SoftArgs& a, hipStream_t st) {
  const int64_t tiles = cdiv(a.B, S);
  const int cus = device_cus();
  const size_t lds = (size_t)a.IN * S * sizeof(float);
  const int per_cu = (int)std::max<int64_t>(1, (int64_t)device_lds_bytes() / std::max<size_t>(lds, 1));
  const int64_t target = (int64_t)cus * std::min(per_cu, 4) * 2;
  int64_t n_chunks = std::max<int64_t>(1, cdiv(target, tiles));
  n_chunks = std::min<int64_t>(n_chunks, std::max<int64_t>(1, cdiv(a.OUT, 64)));
  int64_t chunk = cdiv(cdiv(a.OUT, n_chunks), 64) * 64;
  n_chunks = cdiv(a.OUT, chunk);
  const int64_t grid = tiles * n_chunks;
  SLG_REQUIRE(grid < (1LL << 31), SLG_E_SHAPE, "fc_soft: grid too large");
  auto kern = fc_soft_kernel<NODE, KC, S>;
  if (lds > 65536) {
    hipError_t e = hipFuncSetAttribute((const void*)kern,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) {
      set_error("fc_soft: cannot reserve %zu B LDS: %s", lds, hipGetErrorString(e));
      return (int)e;
    }
  }
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(a.threads), lds, st, a.x, (int)a.B,
                     (int)a.IN, (int)a.OUT, a.K, a.ca, a.cb, a.cstride, a.wa, a.wb, a.wstride,
                     a.np, a.inv_tau, a.y, (int)n_chunks, (int)chunk);
  SLG_LAUNCH_CHECK("fc_soft");
  return 0;
}

template <int NODE, int KC>
static int launch_soft_k(const SoftArgs& a, hipStream_t st) {
  switch (a.S) {
    case 1: return launch_soft_s<NODE, KC, 1>(a, st);
    case 2: return launch_soft_s<NODE, KC, 2>(a, st);
    case 4: return launch_soft_s<NODE, KC, 4>(a, st);
    case 8: return launch_soft_s<NODE, KC, 8>(a, st);
    case 16: return launch_soft_s<NODE, KC, 16>(a, st);
    default: break;
  }
  set_error("fc_soft: unsupported tile_samples %d (1,2,4,8,16)", a.S);
  return SLG_E_ARG;
}

template <int NODE>
static int launch_soft_node(const SoftArgs& a, hipStream_t st) {
  const bool aligned = ((uintptr_t)a.ca % 16 == 0) && ((uintptr_t)a.cb % 16 == 0) &&
                       ((uintptr_t)a.wa % 16 == 0) && ((uintptr_t)a.wb % 16 == 0) &&
                       (a.cstride % 4 == 0) && (a.wstride % 4 == 0) && a.wa && a.wb;
  if (a.K == 8 && aligned) return launch_soft_k<NODE, 8>(a, st);
  if (a.K == 4 && aligned) return launch_soft_k<NODE, 4>(a, st);
  if (a.K == 1) return launch_soft_k<NODE, 1>(a, st);
  if (a.K == 2) return launch_soft_k<NODE, 2>(a, st);
  return launch_soft_k<NODE, 0>(a, st);
}

static int pick_tile(int64_t IN, int requested) {
  if (requested > 0) return requested;
  const int64_t cap = std::min<int64_t>(device_lds_bytes(), 160 * 1024);
  for (int s : {16, 8, 4, 2, 1})
    if (IN * s * 4 <= cap && (s <= 4 || IN * s * 4 <= cap / 2)) return s;
  return 0;
}

static int fc_soft_dispatch(SoftArgs a, int node_kind, hipStream_t st) {
  SLG_REQUIRE(a.x && a.ca && a.cb && a.np && a.y, SLG_E_ARG, "fc_soft: null pointer");
  SLG_REQUIRE(a.B >= 0 && a.IN > 0 && a.OUT > 0, SLG_E_SHAPE, "fc_soft: bad sizes B=%lld IN=%lld OUT=%lld",
              (long long)a.B, (long long)a.IN, (long long)a.OUT);
  SLG_REQUIRE(a.K >= 1 && a.K <= 16, SLG_E_SHAPE, "fc_soft: K=%d outside 1..16", a.K);
  SLG_REQUIRE(a.B < (1LL << 31) && a.IN < (1LL << 28) && a.OUT < (1LL << 31), SLG_E_SHAPE,
              "fc_soft: sizes exceed 32-bit indexing");
  SLG_REQUIRE(((uintptr_t)a.np % 16) == 0, SLG_E_ARG, "fc_soft: node_param must be 16-byte aligned");
  if (a.B == 0) return 0;
  a.S = pick_tile(a.IN, a.S);
  SLG_REQUIRE(a.S > 0 && (int64_t)a.IN * a.S * 4 <= device_lds_bytes(), SLG_E_SHAPE,
              "fc_soft: IN=%lld does not fit LDS", (long long)a.IN);
  if (a.threads <= 0) a.threads = ((int64_t)a.IN * a.S * 4 > 80 * 1024) ? 1024 : 512;
  SLG_REQUIRE(a.threads % 64 == 0 && a.threads <= 1024, SLG_E_ARG, "fc_soft: threads=%d", a.threads);
  switch (node_kind) {
    case SLG_NODE_GATE16: return launch_soft_node<SLG_NODE_GATE16>(a, st);
    case SLG_NODE_WALSH: return launch_soft_node<SLG_NODE_WALSH>(a, st);
    case SLG_NODE_MULTILINEAR2: return launch_soft_node<SLG_NODE_MULTILINEAR2>(a, st);
    default: break;
  }
  set_error("fc_soft: unknown node_kind %d", node_kind);
  return SLG_E_ARG;
}

// ---------------------------------------------------------------------------
// Parameter prep: softmax over K candidates and the 4 node coefficients.
// ---------------------------------------------------------------------------
// silogic/functional.py:24-44 — {1,A,B,AB} coefficients of the 16 gates.
__constant__ float c_basis[16][4] = {
    {0, 0, 0, 0}, {0, 0, 0, 1}, {0, 1, 0, -1}, {0, 1, 0, 0}, {0, 0, 1, -1}, {0, 0, 1, 0},
    {0, 1, 1, -2}, {0, 1, 1, -1}, {1, -1, -1, 1}, {1, -1, -1, 2}, {1, 0, -1, 0},
    {1, 0, -1, 1}, {1, -1, 0, 0}, {1, -1, 0, 1}, {1, 0, 0, -1}, {1, 0, 0, 0}};

__global__ void fc_soft_prep_kernel(const float* __restrict__ conn, int OUT, int K, int node,
                                    const float* __restrict__ raw, float* __restrict__ w,
                                    float* __restrict__ np) {
  const int o = blockIdx.x * blockDim.x + threadIdx.x;
  if (o >= OUT) return;
  for (int s = 0; s < 2; ++s) {  // softmax over the K candidates of slot s
    const int64_t base = ((int64_t)o * 2 + s) * K;
    if (!conn) {
      for (int k = 0; k < K; ++k) w[base + k] = 1.0f;
      continue;
    }
    float m = conn[base];
    for (int k = 1; k < K; ++k) m = fmaxf(m, conn[base + k]);
    float sum = 0.f;
    for (int k = 0; k < K; ++k) sum += expf(conn[base + k] - m);
    for (int k = 0; k < K; ++k) w[base + k] = expf(conn[base + k] - m) / sum;
  }
  float4 c;
  if (node == SLG_NODE_GATE16) {
    const float* g = raw + (int64_t)o * 16;
    float m = g[0];
    for (int i = 1; i < 16; ++i) m = fmaxf(m, g[i]);
    float e[16], sum = 0.f;
    for (int i = 0; i < 16; ++i) { e[i] = expf(g[i] - m); sum += e[i]; }
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    for (int i = 0; i < 16; ++i) {
      const float p = e[i] / sum;
      for (int j = 0; j < 4; ++j) acc[j] += p * c_basis[i][j];
    }
    c = make_float4(acc[0], acc[1], acc[2], acc[3]);
  } else if (node == SLG_NODE_WALSH) {  // nodes.py:138-143
    const float t0 = raw[o * 4 + 0], t1 = raw[o * 4 + 1], t2 = raw[o * 4 + 2], t3 = raw[o * 4 + 3];
    c = make_float4(((t0 - t1) - t2) + t3, 2.0f * (t1 - t3), 2.0f * (t2 - t3), 4.0f * t3);
  } else {
    c = make_float4(sigmoidf_(raw[o * 4 + 0]), sigmoidf_(raw[o * 4 + 1]),
                    sigmoidf_(raw[o * 4 + 2]), sigmoidf_(raw[o * 4 + 3]));
  }
  reinterpret_cast<float4*>(np)[o] = c;
}

// ---------------------------------------------------------------------------
// GroupSum (silogic/heads.py:16-45): one workgroup per sample.
// ---------------------------------------------------------------------------
template <typename T, bool STE>
__global__ void groupsum_kernel(const T* __restrict__ x, int W, int C, float tau,
                                float* __restrict__ logits) {
  const int b = blockIdx.x;
  const int G = W / C;
  __shared__ float red[1024 / 64];
  const T* row = x + (int64_t)b * W;
  for (int c = 0; c < C; ++c) {
    float part = 0.f;
    for (int j = threadIdx.x; j < G; j += blockDim.x) {
      const float v = (float)row[c * G + j];
      part += STE ? (v > 0.5f ? 1.0f : 0.0f) : v;
    }
    for (int off = 32; off > 0; off >>= 1) part += __shfl_xor(part, off);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = part;
    __syncthreads();
    if (threadIdx.x == 0) {
      float s = 0.f;
      for (int i = 0; i < (int)(blockDim.x >> 6); ++i) s += red[i];
      logits[(int64_t)b * C + c] = s / tau;
    }
    __syncthreads();
  }
}

}  // namespace slg

using namespace slg;

extern "C" {

int slg_fc_soft_fwd(const float* x, int64_t B, int64_t IN, int64_t OUT, int32_t K,
                    const int32_t* cand, const float* w, int32_t node_kind,
                    const float* node_param, float inv_tau, float* out, int32_t tile_samples,
                    int32_t threads, slg_stream_t stream) {
  SLG_REQUIRE(cand && w, SLG_E_ARG, "fc_soft_fwd: null cand/w");
  SoftArgs a{x, B, IN, OUT, K, cand, cand + K, 2 * K, w, w + K, 2 * K, node_param, inv_tau,
             out, tile_samples, threads};
  return fc_soft_dispatch(a, node_kind, as_stream(stream));
}

int slg_dense_logic_fwd(const float* x, int64_t B, int64_t IN, int64_t OUT, int32_t K,
                        const int32_t* ca, const int32_t* cb, const float* wa, const float* wb,
                        const float* coef, float* out, slg_stream_t stream) {
  SLG_REQUIRE(wa && wb, SLG_E_ARG, "dense_logic: null weights");
  SoftArgs a{x, B, IN, OUT, K, ca, cb, K, wa, wb, K, coef, 1.0f, out, 0, 0};
  return fc_soft_dispatch(a, SLG_NODE_GATE16, as_stream(stream));
}

int slg_warp_logic_fwd(const float* x, int64_t B, int64_t IN, int64_t OUT, int32_t K,
                       const int32_t* ca, const int32_t* cb, const float* wa, const float* wb,
                       const float* coef, float inv_tau, float* out, slg_stream_t stream) {
  SLG_REQUIRE(wa && wb, SLG_E_ARG, "warp_logic: null weights");
  SoftArgs a{x, B, IN, OUT, K, ca, cb, K, wa, wb, K, coef, inv_tau, out, 0, 0};
  return fc_soft_dispatch(a, SLG_NODE_WALSH, as_stream(stream));
}

int slg_fc_soft_prep(const float* conn, int64_t OUT, int32_t K, int32_t node_kind,
                     const float* raw, float* w, float* node_param, slg_stream_t stream) {
  SLG_REQUIRE(raw && w && node_param, SLG_E_ARG, "fc_soft_prep: null pointer");
  SLG_REQUIRE(OUT > 0 && OUT < (1LL << 31) && K >= 1 && K <= 64, SLG_E_SHAPE,
              "fc_soft_prep: bad OUT/K");
  SLG_REQUIRE(node_kind >= 0 && node_kind <= 2, SLG_E_ARG, "fc_soft_prep: node_kind %d", node_kind);
  SLG_REQUIRE(((uintptr_t)node_param % 16) == 0, SLG_E_ARG, "fc_soft_prep: node_param alignment");
  const int th = 256;
  hipLaunchKernelGGL(fc_soft_prep_kernel, dim3((unsigned)cdiv(OUT, th)), dim3(th), 0,
                     as_stream(stream), conn, (int)OUT, K, node_kind, raw, w, node_param);
  SLG_LAUNCH_CHECK("fc_soft_prep");
  return 0;
}

int slg_groupsum_soft(const float* x, int64_t B, int64_t W, int32_t C, float tau, int32_t ste,
                      float* logits, slg_stream_t stream) {
  SLG_REQUIRE(x && logits, SLG_E_ARG, "groupsum_soft: null pointer");
  SLG_REQUIRE(B >= 0 && B < (1LL << 31) && C > 0 && W > 0 && W % C == 0 && W < (1LL << 31),
              SLG_E_SHAPE, "groupsum_soft: W=%lld not divisible by C=%d", (long long)W, C);
  if (B == 0) return 0;
  if (ste)
    hipLaunchKernelGGL((groupsum_kernel<float, true>), dim3((unsigned)B), dim3(256), 0,
                       as_stream(stream), x, (int)W, C, tau, logits);
  else
    hipLaunchKernelGGL((groupsum_kernel<float, false>), dim3((unsigned)B), dim3(256), 0,
                       as_stream(stream), x, (int)W, C, tau, logits);
  SLG_LAUNCH_CHECK("groupsum_soft");
  return 0;
}

int slg_groupsum_hard(const void* x, int32_t dtype, int64_t B, int64_t W, int32_t C,
                      float* logits, slg_stream_t stream) {
  SLG_REQUIRE(x && logits, SLG_E_ARG, "groupsum_hard: null pointer");
  SLG_REQUIRE(B >= 0 && B < (1LL << 31) && C > 0 && W > 0 && W % C == 0 && W < (1LL << 31),
              SLG_E_SHAPE, "groupsum_hard: W=%lld not divisible by C=%d", (long long)W, C);
  if (B == 0) return 0;
  if (dtype == 1)
    hipLaunchKernelGGL((groupsum_kernel<uint8_t, false>), dim3((unsigned)B), dim3(256), 0,
                       as_stream(stream), (const uint8_t*)x, (int)W, C, 1.0f, logits);
  else
    hipLaunchKernelGGL((groupsum_kernel<float, false>), dim3((unsigned)B), dim3(256), 0,
                       as_stream(stream), (const float*)x, (int)W, C, 1.0f, logits);
  SLG_LAUNCH_CHECK("groupsum_hard");
  return 0;
}

}  // extern "C"
