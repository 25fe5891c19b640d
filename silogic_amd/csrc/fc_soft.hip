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

// Native vector types: one ds_read_b64 / ds_read_b128 per gather (HIP's
// float2/float4 structs are split into scalar LDS reads by the compiler).
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
template <int V> struct vecf;
template <> struct vecf<1> { using t = float; };
template <> struct vecf<2> { using t = f32x2; };
template <> struct vecf<4> { using t = f32x4; };

__device__ inline float lanev(float v, int) { return v; }
__device__ inline float lanev(f32x2 v, int i) { return v[i]; }
__device__ inline float lanev(f32x4 v, int i) { return v[i]; }
__device__ inline float lanev(float4 v, int i) {
  return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w));
}
__device__ inline void fma_acc(float& acc, float w, float v) { acc = fmaf(w, v, acc); }
template <typename VT>
__device__ inline void fma_acc(VT& acc, float w, VT v) {
#pragma unroll
  for (int i = 0; i < (int)(sizeof(VT) / 4); ++i) acc[i] = fmaf(w, v[i], acc[i]);
}
template <typename T> __device__ inline T zero_vec() { return (T)0.0f; }

__device__ inline float sigmoidf_(float z) { return 1.0f / (1.0f + expf(-z)); }

template <int V> __device__ inline typename vecf<V>::t make_vec(const float (&e)[V]);
template <> __device__ inline float make_vec<1>(const float (&e)[1]) { return e[0]; }
template <> __device__ inline f32x2 make_vec<2>(const float (&e)[2]) { return f32x2{e[0], e[1]}; }
template <> __device__ inline f32x4 make_vec<4>(const float (&e)[4]) {
  return f32x4{e[0], e[1], e[2], e[3]};
}

// 16-byte streaming (non-temporal) load: the input rows are read once.
__device__ inline float4 ld_stream4(const float* p) {
  const f32x4 v = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
  return make_float4(v.x, v.y, v.z, v.w);
}

// LDS slot of (input i, sample group g). Rows of G > 1 groups are G*16 bytes
// apart, a multiple of 32 B, so random rows would hit only 64/(4G) of the
// bank groups; XOR-ing g with the low bits of i spreads them over all.
template <int G>
__device__ inline int slot(int i, int g) {
  if constexpr (G == 1) return i;
  else return i * G + (g ^ (i & (G - 1)));
}

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

// Per-output parameters held in registers: 2K candidate indices, 2K weights,
// 4 node coefficients (144 bytes for K = 8).
template <int KM>
struct FcParams {
  int ia[KM], ib[KM];
  float fa[KM], fb[KM];
  float4 p;
};

// KC = compile-time candidate count (0 = runtime K <= 16, scalar loads).
template <int KC, int KM>
__device__ inline void load_params(FcParams<KM>& P, int o, int K, const int* __restrict__ ca,
                                   const int* __restrict__ cb, int cstride,
                                   const float* __restrict__ wa, const float* __restrict__ wb,
                                   int wstride, const float* __restrict__ np) {
  if constexpr (KC > 0 && (KC % 4) == 0) {
#pragma unroll
    for (int q = 0; q < KC / 4; ++q) {
      const int4 a4 = *reinterpret_cast<const int4*>(ca + (int64_t)o * cstride + 4 * q);
      const int4 b4 = *reinterpret_cast<const int4*>(cb + (int64_t)o * cstride + 4 * q);
      const float4 u4 = *reinterpret_cast<const float4*>(wa + (int64_t)o * wstride + 4 * q);
      const float4 v4 = *reinterpret_cast<const float4*>(wb + (int64_t)o * wstride + 4 * q);
      P.ia[4 * q + 0] = a4.x; P.ia[4 * q + 1] = a4.y; P.ia[4 * q + 2] = a4.z; P.ia[4 * q + 3] = a4.w;
      P.ib[4 * q + 0] = b4.x; P.ib[4 * q + 1] = b4.y; P.ib[4 * q + 2] = b4.z; P.ib[4 * q + 3] = b4.w;
      P.fa[4 * q + 0] = u4.x; P.fa[4 * q + 1] = u4.y; P.fa[4 * q + 2] = u4.z; P.fa[4 * q + 3] = u4.w;
      P.fb[4 * q + 0] = v4.x; P.fb[4 * q + 1] = v4.y; P.fb[4 * q + 2] = v4.z; P.fb[4 * q + 3] = v4.w;
    }
  } else {
#pragma unroll
    for (int k = 0; k < KM; ++k) {
      if (k < K) {
        P.ia[k] = ca[(int64_t)o * cstride + k];
        P.ib[k] = cb[(int64_t)o * cstride + k];
        P.fa[k] = wa ? wa[(int64_t)o * wstride + k] : 1.0f;
        P.fb[k] = wb ? wb[(int64_t)o * wstride + k] : 1.0f;
      } else {
        P.ia[k] = 0; P.ib[k] = 0; P.fa[k] = 0.f; P.fb[k] = 0.f;
      }
    }
  }
  P.p = reinterpret_cast<const float4*>(np)[o];
}

// Widest workgroup per variant: 1024 threads keeps <= 128 VGPRs per lane,
// which fits the lean variants; the others get 512 threads and more registers.
template <int KC, int S>
constexpr int soft_max_threads() { return (KC == 0 || S >= 8) ? 512 : 1024; }

template <int NODE, int KC, int S>
__global__ void __launch_bounds__((soft_max_threads<KC, S>()))
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
  const int o_begin = ch * chunk;
  const int o_end = min(OUT, o_begin + chunk);

  // First output's parameters are in flight while the tile is staged.
  int o = o_begin + threadIdx.x;
  FcParams<KM> P;
  if (o < o_end) load_params<KC>(P, o, K, ca, cb, cstride, wa, wb, wstride, np);

  // Stage S rows transposed: slot(i, g) holds samples b0+gV .. b0+gV+V-1 of
  // input i. Threads load float4 runs of 4 inputs from each of the V rows of
  // a group (4 batches in flight), then scatter them to the 4 input slots.
  const bool vec_rows = (IN & 3) == 0;
  for (int g = 0; g < G; ++g) {
    if (vec_rows) {
      const int n4 = IN >> 2;
      constexpr int NBAT = V == 4 ? 2 : 4;  // float4 batches in flight per thread
      for (int q0 = threadIdx.x; q0 < n4; q0 += NBAT * blockDim.x) {
        float4 t[NBAT][V];
#pragma unroll
        for (int u = 0; u < NBAT; ++u) {
          const int q = q0 + u * blockDim.x;
#pragma unroll
          for (int v = 0; v < V; ++v) {
            const int b = b0 + g * V + v;
            t[u][v] = (b < B && q < n4)
                          ? ld_stream4(x + (int64_t)b * IN + 4 * q)
                          : make_float4(0.f, 0.f, 0.f, 0.f);
          }
        }
#pragma unroll
        for (int u = 0; u < NBAT; ++u) {
          const int q = q0 + u * blockDim.x;
          if (q < n4) {
#pragma unroll
            for (int c = 0; c < 4; ++c) {
              float e[V];
#pragma unroll
              for (int v = 0; v < V; ++v) e[v] = lanev(t[u][v], c);
              const int i = 4 * q + c;
              lds[slot<G>(i, g)] = make_vec<V>(e);
            }
          }
        }
      }
    } else {
      for (int i = threadIdx.x; i < IN; i += blockDim.x) {
        float e[V];
#pragma unroll
        for (int v = 0; v < V; ++v) {
          const int b = b0 + g * V + v;
          e[v] = (b < B) ? __builtin_nontemporal_load(x + (int64_t)b * IN + i) : 0.0f;
        }
        lds[slot<G>(i, g)] = make_vec<V>(e);
      }
    }
  }
  __syncthreads();

  while (o < o_end) {
    // prefetch the next output's parameters; they land while this one computes
    const int on = o + blockDim.x;
    FcParams<KM> Q;
    if (on < o_end) load_params<KC>(Q, on, K, ca, cb, cstride, wa, wb, wstride, np);
    int ia[KM], ib[KM];
#pragma unroll
    for (int k = 0; k < KM; ++k) {  // clamp into the staged rows
      ia[k] = min(max(P.ia[k], 0), IN - 1);
      ib[k] = min(max(P.ib[k], 0), IN - 1);
    }
    for (int g = 0; g < G; ++g) {
      vt A = zero_vec<vt>(), Bv = zero_vec<vt>();
#pragma unroll
      for (int k = 0; k < KM; ++k) {
        if (KC > 0 || k < K) {
          fma_acc(A, P.fa[k], lds[slot<G>(ia[k], g)]);
          fma_acc(Bv, P.fb[k], lds[slot<G>(ib[k], g)]);
        }
      }
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const int b = b0 + g * V + v;
        if (b < B) y[(int64_t)b * OUT + o] = node_eval<NODE>(lanev(A, v), lanev(Bv, v), P.p, inv_tau);
      }
    }
    P = Q;
    o = on;
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
  const int threads = std::min(a.threads, soft_max_threads<KC, S>());
  if (lds > 65536) {
    hipError_t e = hipFuncSetAttribute((const void*)kern,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) {
      set_error("fc_soft: cannot reserve %zu B LDS: %s", lds, hipGetErrorString(e));
      return (int)e;
    }
  }
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(threads), lds, st, a.x, (int)a.B,
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

// Samples per workgroup tile and workgroup size, from a sweep on MI355X
// (B = 4096, OUT = 10000-16380, K = 8): IN = 784 -> 4 samples / 256 threads,
// IN = 4096 -> 8 / 512, IN = 10000 -> 4 / 1024, IN = 16380 -> 2 / 1024. The
// tile takes the largest power of two <= 8 whose rows fit 160 KB of LDS (4 for
// narrow inputs, where more, smaller workgroups per CU win).
static int pick_tile(int64_t IN, int requested) {
  if (requested > 0) return requested;
  const int64_t cap = std::min<int64_t>(device_lds_bytes(), 160 * 1024);
  if (IN <= 1280) return 4;
  for (int s : {8, 4, 2, 1})
    if (IN * s * 4 <= cap) return s;
  return 0;
}

static int pick_threads(int64_t IN, int S, int requested) {
  if (requested > 0) return requested;
  const int64_t lds = IN * S * 4;
  if (lds <= 40 * 1024) return 256;
  return 1024;  // capped per variant by soft_max_threads
}

static int fc_soft_dispatch(SoftArgs a, int node_kind, hipStream_t st) {
  SLG_REQUIRE(a.ca && a.cb && a.np && ((a.x && a.y) || a.B == 0), SLG_E_ARG, "fc_soft: null pointer");
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
  a.threads = pick_threads(a.IN, a.S, a.threads);
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
__global__ void __launch_bounds__(256) groupsum_kernel(const T* __restrict__ x, int B, int W, int C,
                                                       float tau, float* __restrict__ logits) {
  // one wave per (sample, class): coalesced reads of the class block, wave sum
  const int task = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (task >= B * C) return;
  const int b = task / C, c = task % C;
  const int G = W / C;
  const T* row = x + (int64_t)b * W + (int64_t)c * G;
  float part = 0.f;
  for (int j = lane; j < G; j += 64) {
    const float v = (float)row[j];
    part += STE ? (v > 0.5f ? 1.0f : 0.0f) : v;
  }
  for (int off = 32; off > 0; off >>= 1) part += __shfl_xor(part, off);
  if (lane == 0) logits[task] = part / tau;
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
  SLG_REQUIRE((x && logits) || B == 0, SLG_E_ARG, "groupsum_soft: null pointer");
  SLG_REQUIRE(B >= 0 && B * C < (1LL << 31) && C > 0 && W > 0 && W % C == 0 && W < (1LL << 31),
              SLG_E_SHAPE, "groupsum_soft: W=%lld not divisible by C=%d", (long long)W, C);
  if (B == 0) return 0;
  const unsigned grid = (unsigned)cdiv(B * C, 4);
  if (ste)
    hipLaunchKernelGGL((groupsum_kernel<float, true>), dim3(grid), dim3(256), 0, as_stream(stream), x,
                       (int)B, (int)W, C, tau, logits);
  else
    hipLaunchKernelGGL((groupsum_kernel<float, false>), dim3(grid), dim3(256), 0, as_stream(stream),
                       x, (int)B, (int)W, C, tau, logits);
  SLG_LAUNCH_CHECK("groupsum_soft");
  return 0;
}

int slg_groupsum_hard(const void* x, int32_t dtype, int64_t B, int64_t W, int32_t C,
                      float* logits, slg_stream_t stream) {
  SLG_REQUIRE((x && logits) || B == 0, SLG_E_ARG, "groupsum_hard: null pointer");
  SLG_REQUIRE(B >= 0 && B * C < (1LL << 31) && C > 0 && W > 0 && W % C == 0 && W < (1LL << 31),
              SLG_E_SHAPE, "groupsum_hard: W=%lld not divisible by C=%d", (long long)W, C);
  if (B == 0) return 0;
  const unsigned grid = (unsigned)cdiv(B * C, 4);
  if (dtype == 1)
    hipLaunchKernelGGL((groupsum_kernel<uint8_t, false>), dim3(grid), dim3(256), 0,
                       as_stream(stream), (const uint8_t*)x, (int)B, (int)W, C, 1.0f, logits);
  else
    hipLaunchKernelGGL((groupsum_kernel<float, false>), dim3(grid), dim3(256), 0,
                       as_stream(stream), (const float*)x, (int)B, (int)W, C, 1.0f, logits);
  SLG_LAUNCH_CHECK("groupsum_hard");
  return 0;
}

}  // extern "C"
