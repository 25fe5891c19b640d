// FC soft backward for gfx950 (the gradients DenseLogicFn / WarpLogicFn
// return: kernels/dense.py:46-75, 107-120; warp.py:33-64): given x [B,IN],
// the layer's candidates / weights / node parameters and gy [B,OUT], write
//   gx  [B,IN]      = sum over (o, k) of ga[b,o] * w_a[o,k] at x[b, cand_a[o,k]]
//                     (and the b side),
//   gw  [OUT,2,K]   = sum over b of ga[b,o] * x[b, cand_a[o,k]] (and b),
//   gnp [OUT,4]     = sum over b of dL/dparam,
// where ga, gb are the node's input gradients at the recomputed operands.
//
// Three launches, each shaped for one reduction:
//   * records: the parameters repacked into the forward's chunk-major
//     records (natural candidate order), so every parameter load of a wave
//     is one coalesced 16-byte load per quad.
//   * fc_soft_bwd_x_kernel: a workgroup owns S samples and every output. It
//     stages the S rows in LDS next to an S-row gradient accumulator,
//     recomputes each output's operands, and adds its input gradients with
//     LDS float atomics; the finished rows are written once. No global
//     atomics: every contribution to a row of gx comes from this workgroup.
//   * fc_soft_bwd_w_kernel: a workgroup owns 1024 outputs (one per thread)
//     and a range of samples; it streams that range through LDS in S-sample
//     tiles and keeps its output's 2K + 4 gradient sums in registers, then
//     writes them once as one partial per sample range.
//   * fc_soft_bwd_reduce_kernel: sums the partials over sample ranges in a
//     fixed order (deterministic weight gradients).
#include "fc_soft_common.h"

namespace slg {

// dL/da, dL/db and dL/dparam of one node at operands (a, b), given dL/dy = g.
template <int NODE>
__device__ inline void node_grad(float a, float b, float g, const float4& p, float inv_tau,
                                 float& ga, float& gb, float (&gp)[4]) {
  if constexpr (NODE == SLG_NODE_MULTILINEAR2) {
    // y = (1-a)(1-b) s0 + a(1-b) s1 + (1-a) b s2 + a b s3 (nodes.py:174-178)
    const float ua = 1.0f - a, ub = 1.0f - b;
    gp[0] = g * (ua * ub);
    gp[1] = g * (a * ub);
    gp[2] = g * (ua * b);
    gp[3] = g * (a * b);
    ga = g * (ub * (p.y - p.x) + b * (p.w - p.z));
    gb = g * (ua * (p.z - p.x) + a * (p.w - p.y));
  } else {
    float gz = g;
    if constexpr (NODE == SLG_NODE_WALSH) {
      // y = sigmoid(z * inv_tau), z = c0 + c1 a + c2 b + c3 ab (warp.py:14-31)
      const float y = sigmoidf_((p.x + p.y * a + p.z * b + p.w * (a * b)) * inv_tau);
      gz = g * (y * (1.0f - y)) * inv_tau;
    }
    gp[0] = gz;
    gp[1] = gz * a;
    gp[2] = gz * b;
    gp[3] = gz * (a * b);
    ga = gz * (p.y + p.w * b);
    gb = gz * (p.z + p.w * a);
  }
}

// Records from separate arrays: cand [OUT,2,K] int32 (clamped to IN),
// w [OUT,2,K], np [OUT,4] -> the chunk-major records of fc_soft_kernel
// (quad q of output o at ((o/64)*(K+1)+q)*64 + o%64; words idx_a, idx_b,
// w_a, w_b, params). One thread per record word.
__global__ void __launch_bounds__(256) fc_soft_pack_records_kernel(const int* __restrict__ cand,
                                                                   const float* __restrict__ w,
                                                                   const float* __restrict__ np,
                                                                   int OUT, int K, int IN,
                                                                   float* __restrict__ rec) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t nq = (int64_t)((OUT + 63) / 64) * (K + 1) * 64;
  if (t >= nq * 4) return;
  const int e = (int)(t & 3);
  const int64_t Q = t >> 2;
  const int lane = (int)(Q % 64);
  const int q = (int)((Q / 64) % (K + 1));
  const int c = (int)(Q / (64 * (int64_t)(K + 1)));
  const int o = min(c * 64 + lane, OUT - 1);
  const int word = q * 4 + e;
  float v;
  if (word < 2 * K) {
    const int i = cand[(int64_t)o * 2 * K + word];  // side = word / K, k = word % K
    v = __int_as_float(min(max(i, 0), IN - 1));
  } else if (word < 4 * K) {
    v = w[(int64_t)o * 2 * K + (word - 2 * K)];
  } else {
    v = np[(int64_t)o * 4 + (word - 4 * K)];
  }
  rec[t] = v;
}

template <int KC>
constexpr int bwd_threads() { return KC > 0 && KC <= 8 ? 1024 : 512; }

// Input gradient of S samples (see the file comment).
template <int NODE, int KC, int S>
__global__ void __launch_bounds__((bwd_threads<KC>()))
fc_soft_bwd_x_kernel(const float* __restrict__ x, int B, int IN, int OUT, int Kr, ParamView pv,
                     float inv_tau, const float* __restrict__ gy, float* __restrict__ gx) {
  constexpr int KM = KC > 0 ? KC : 16;
  using vt = typename vecf<S>::t;
  extern __shared__ __align__(16) unsigned char smem[];
  vt* xs = reinterpret_cast<vt*>(smem);                                   // [IN] x S samples
  float* gs = reinterpret_cast<float*>(smem + (size_t)IN * S * sizeof(float));  // [IN][S]
  const int K = KC > 0 ? KC : Kr;
  const int b0 = blockIdx.x * S;

  for (int i = threadIdx.x; i < IN; i += blockDim.x) {
    float e[S];
#pragma unroll
    for (int s = 0; s < S; ++s) e[s] = (b0 + s < B) ? x[(int64_t)(b0 + s) * IN + i] : 0.0f;
    xs[i] = make_vec<S>(e);
#pragma unroll
    for (int s = 0; s < S; ++s) gs[i * S + s] = 0.0f;
  }
  __syncthreads();

  const uint32_t lim = (uint32_t)IN - 1u;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nwaves = blockDim.x >> 6;
  const int n64 = (OUT + 63) >> 6;
  for (int j = wave; j < n64; j += nwaves) {
    const int o = j * 64 + lane;
    const bool valid = o < OUT;
    FcParams<KM> P;
    load_params<KC, KM, true>(P, min(o, OUT - 1), K, pv);
    uint32_t ia[KM], ib[KM];
#pragma unroll
    for (int k = 0; k < KM; ++k) {
      ia[k] = min((uint32_t)P.ia[k], lim);
      ib[k] = min((uint32_t)P.ib[k], lim);
    }
    vt A = zero_vec<vt>(), Bv = zero_vec<vt>();
#pragma unroll
    for (int k = 0; k < KM; ++k) {
      if (KC > 0 || k < K) {
        fma_acc(A, P.fa[k], xs[ia[k]]);
        fma_acc(Bv, P.fb[k], xs[ib[k]]);
      }
    }
    float ga[S], gb[S];
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const float g = (valid && b0 + s < B) ? gy[(int64_t)(b0 + s) * OUT + o] : 0.0f;
      float gp[4];
      node_grad<NODE>(lanev(A, s), lanev(Bv, s), g, P.p, inv_tau, ga[s], gb[s], gp);
    }
#pragma unroll
    for (int k = 0; k < KM; ++k) {
      if (KC > 0 || k < K) {
#pragma unroll
        for (int s = 0; s < S; ++s) {
          atomicAdd(&gs[ia[k] * S + s], ga[s] * P.fa[k]);
          atomicAdd(&gs[ib[k] * S + s], gb[s] * P.fb[k]);
        }
      }
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < IN; i += blockDim.x) {
#pragma unroll
    for (int s = 0; s < S; ++s)
      if (b0 + s < B) gx[(int64_t)(b0 + s) * IN + i] = gs[i * S + s];
  }
}

// Weight / node-parameter gradient partials of one output per thread over a
// range of sample tiles: part [NR][2K+4][OUT] (components w_a[0..K),
// w_b[0..K), param[0..4)).
template <int NODE, int KC, int S>
__global__ void __launch_bounds__((bwd_threads<KC>()))
fc_soft_bwd_w_kernel(const float* __restrict__ x, int B, int IN, int OUT, int Kr, ParamView pv,
                     float inv_tau, const float* __restrict__ gy, int n_orange, int tiles_per_range,
                     float* __restrict__ part) {
  constexpr int KM = KC > 0 ? KC : 16;
  using vt = typename vecf<S>::t;
  extern __shared__ __align__(16) unsigned char smem[];
  vt* xs = reinterpret_cast<vt*>(smem);
  const int K = KC > 0 ? KC : Kr;
  const int r_o = (int)(blockIdx.x % (uint32_t)n_orange);
  const int r_b = (int)(blockIdx.x / (uint32_t)n_orange);
  const int o = r_o * blockDim.x + threadIdx.x;
  const bool valid = o < OUT;
  FcParams<KM> P;
  load_params<KC, KM, true>(P, min(o, OUT - 1), K, pv);
  const uint32_t lim = (uint32_t)IN - 1u;
#pragma unroll
  for (int k = 0; k < KM; ++k) {  // clamp in place: one copy of the indices
    P.ia[k] = (int)min((uint32_t)P.ia[k], lim);
    P.ib[k] = (int)min((uint32_t)P.ib[k], lim);
  }
  const int* ia = P.ia;
  const int* ib = P.ib;
  float swa[KM], swb[KM], sp[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int k = 0; k < KM; ++k) swa[k] = swb[k] = 0.0f;

  const int n_tiles = (B + S - 1) / S;
  const int t_end = min(n_tiles, (r_b + 1) * tiles_per_range);
  for (int t = r_b * tiles_per_range; t < t_end; ++t) {
    const int b0 = t * S;
    __syncthreads();  // the previous tile's reads are done
    for (int i = threadIdx.x; i < IN; i += blockDim.x) {
      float e[S];
#pragma unroll
      for (int s = 0; s < S; ++s) e[s] = (b0 + s < B) ? x[(int64_t)(b0 + s) * IN + i] : 0.0f;
      xs[i] = make_vec<S>(e);
    }
    __syncthreads();
    vt A = zero_vec<vt>(), Bv = zero_vec<vt>();
#pragma unroll
    for (int k = 0; k < KM; ++k) {
      if (KC > 0 || k < K) {
        fma_acc(A, P.fa[k], xs[ia[k]]);
        fma_acc(Bv, P.fb[k], xs[ib[k]]);
      }
    }
    float ga[S], gb[S];
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const float g = (valid && b0 + s < B) ? gy[(int64_t)(b0 + s) * OUT + o] : 0.0f;
      float gp[4];
      node_grad<NODE>(lanev(A, s), lanev(Bv, s), g, P.p, inv_tau, ga[s], gb[s], gp);
#pragma unroll
      for (int q = 0; q < 4; ++q) sp[q] += gp[q];
    }
    // second pass over the candidates: sum_s ga[s] * x[s][cand]
#pragma unroll
    for (int k = 0; k < KM; ++k) {
      if (KC > 0 || k < K) {
        const vt va = xs[ia[k]], vb = xs[ib[k]];
#pragma unroll
        for (int s = 0; s < S; ++s) {
          swa[k] = fmaf(ga[s], lanev(va, s), swa[k]);
          swb[k] = fmaf(gb[s], lanev(vb, s), swb[k]);
        }
      }
    }
  }
  if (valid) {
    float* base = part + (int64_t)r_b * (2 * K + 4) * OUT + o;
#pragma unroll
    for (int k = 0; k < KM; ++k) {
      if (KC > 0 || k < K) {
        base[(int64_t)k * OUT] = swa[k];
        base[(int64_t)(K + k) * OUT] = swb[k];
      }
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) base[(int64_t)(2 * K + q) * OUT] = sp[q];
  }
}

// gw [OUT,2,K], gnp [OUT,4] = sum over r of part[r] (r ascending).
__global__ void __launch_bounds__(256) fc_soft_bwd_reduce_kernel(const float* __restrict__ part,
                                                                 int NR, int OUT, int K,
                                                                 float* __restrict__ gw,
                                                                 float* __restrict__ gnp) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int NC = 2 * K + 4;
  if (t >= (int64_t)NC * OUT) return;
  const int c = (int)(t / OUT), o = (int)(t - (int64_t)c * OUT);
  float s = 0.0f;
  for (int r = 0; r < NR; ++r) s += part[((int64_t)r * NC + c) * OUT + o];
  if (c < 2 * K) {
    if (gw) gw[(int64_t)o * 2 * K + c] = s;  // c = side * K + k
  } else if (gnp) {
    gnp[(int64_t)o * 4 + (c - 2 * K)] = s;
  }
}

// ---------------------------------------------------------------------------
// launch helpers
// ---------------------------------------------------------------------------
static int bwd_tile(int64_t IN, int64_t per_float_bytes_per_sample) {
  const int64_t cap = std::min<int64_t>(device_lds_bytes(), 160 * 1024);
  for (int s : {4, 2, 1})
    if (IN * s * per_float_bytes_per_sample <= cap) return s;
  return 0;
}

struct BwdPlan {
  int Sx, Sw;          // samples per LDS tile of the two kernels (0 = unsupported)
  int n_orange, NR, tiles_per_range;
  int64_t rec_floats, part_floats;
};

static BwdPlan bwd_plan(int64_t B, int64_t IN, int64_t OUT, int K) {
  BwdPlan p{};
  p.Sx = bwd_tile(IN, 8);   // x tile + gradient accumulator
  p.Sw = bwd_tile(IN, 4);   // x tile
  if (K == 8) p.Sw = std::min(p.Sw, 2);  // 4-sample tiles overflow 128 VGPRs at 1024 threads
  const int threads = K == 8 || K == 4 ? 1024 : 512;
  p.n_orange = (int)cdiv(OUT, threads);
  const int64_t n_tiles = p.Sw ? cdiv(std::max<int64_t>(B, 1), p.Sw) : 1;
  p.NR = (int)std::max<int64_t>(1, std::min<int64_t>(n_tiles, cdiv(2 * device_cus(), p.n_orange)));
  p.tiles_per_range = (int)cdiv(n_tiles, p.NR);
  p.NR = (int)cdiv(n_tiles, p.tiles_per_range);
  p.rec_floats = cdiv(OUT, 64) * 64 * (int64_t)(K + 1) * 4;
  p.part_floats = (int64_t)p.NR * (2 * K + 4) * OUT;
  return p;
}

template <int NODE, int KC, int S>
static int launch_bwd_x(const float* x, int64_t B, int64_t IN, int64_t OUT, int K,
                        const ParamView& pv, float inv_tau, const float* gy, float* gx,
                        hipStream_t st) {
  auto kern = fc_soft_bwd_x_kernel<NODE, KC, S>;
  const size_t lds = (size_t)IN * S * 8;
  if (lds > 65536) {
    hipError_t e = hipFuncSetAttribute((const void*)kern,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) {
      set_error("fc_soft_bwd: LDS %zu: %s", lds, hipGetErrorString(e));
      return (int)e;
    }
  }
  hipLaunchKernelGGL(kern, dim3((unsigned)cdiv(B, S)), dim3(bwd_threads<KC>()), lds, st, x,
                     (int)B, (int)IN, (int)OUT, K, pv, inv_tau, gy, gx);
  SLG_LAUNCH_CHECK("fc_soft_bwd_x");
  return 0;
}

template <int NODE, int KC, int S>
static int launch_bwd_w(const float* x, int64_t B, int64_t IN, int64_t OUT, int K,
                        const ParamView& pv, float inv_tau, const float* gy, const BwdPlan& p,
                        float* part, hipStream_t st) {
  auto kern = fc_soft_bwd_w_kernel<NODE, KC, S>;
  const size_t lds = (size_t)IN * S * 4;
  if (lds > 65536) {
    hipError_t e = hipFuncSetAttribute((const void*)kern,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) {
      set_error("fc_soft_bwd: LDS %zu: %s", lds, hipGetErrorString(e));
      return (int)e;
    }
  }
  hipLaunchKernelGGL(kern, dim3((unsigned)(p.n_orange * p.NR)), dim3(bwd_threads<KC>()), lds, st,
                     x, (int)B, (int)IN, (int)OUT, K, pv, inv_tau, gy, p.n_orange,
                     p.tiles_per_range, part);
  SLG_LAUNCH_CHECK("fc_soft_bwd_w");
  return 0;
}

template <int NODE, int KC>
static int bwd_node_k(const float* x, int64_t B, int64_t IN, int64_t OUT, int K,
                      const ParamView& pv, float inv_tau, const float* gy, float* gx,
                      float* part, const BwdPlan& p, hipStream_t st) {
  if (gx) {
    int rc = p.Sx == 4 ? launch_bwd_x<NODE, KC, 4>(x, B, IN, OUT, K, pv, inv_tau, gy, gx, st)
           : p.Sx == 2 ? launch_bwd_x<NODE, KC, 2>(x, B, IN, OUT, K, pv, inv_tau, gy, gx, st)
                       : launch_bwd_x<NODE, KC, 1>(x, B, IN, OUT, K, pv, inv_tau, gy, gx, st);
    if (rc) return rc;
  }
  if (part) {
    return p.Sw == 4 ? launch_bwd_w<NODE, KC, 4>(x, B, IN, OUT, K, pv, inv_tau, gy, p, part, st)
         : p.Sw == 2 ? launch_bwd_w<NODE, KC, 2>(x, B, IN, OUT, K, pv, inv_tau, gy, p, part, st)
                     : launch_bwd_w<NODE, KC, 1>(x, B, IN, OUT, K, pv, inv_tau, gy, p, part, st);
  }
  return 0;
}

template <int NODE>
static int bwd_node(const float* x, int64_t B, int64_t IN, int64_t OUT, int K, const ParamView& pv,
                    float inv_tau, const float* gy, float* gx, float* part, const BwdPlan& p,
                    hipStream_t st) {
  if (K == 8) return bwd_node_k<NODE, 8>(x, B, IN, OUT, K, pv, inv_tau, gy, gx, part, p, st);
  if (K == 4) return bwd_node_k<NODE, 4>(x, B, IN, OUT, K, pv, inv_tau, gy, gx, part, p, st);
  return bwd_node_k<NODE, 0>(x, B, IN, OUT, K, pv, inv_tau, gy, gx, part, p, st);
}

}  // namespace slg

using namespace slg;

extern "C" {

int64_t slg_fc_soft_bwd_workspace(int64_t B, int64_t IN, int64_t OUT, int32_t K) {
  if (B < 0 || IN <= 0 || OUT <= 0 || K < 1 || K > 16) return -1;
  const BwdPlan p = bwd_plan(B, IN, OUT, K);
  if (!p.Sx || !p.Sw) return -1;
  return p.rec_floats + p.part_floats;
}

int slg_fc_soft_bwd(const float* x, int64_t B, int64_t IN, int64_t OUT, int32_t K,
                    const int32_t* cand, const float* w, int32_t node_kind,
                    const float* node_param, float inv_tau, const float* gy, float* gx,
                    float* gw, float* gnp, float* workspace, int64_t workspace_floats,
                    slg_stream_t stream) {
  SLG_REQUIRE(cand && w && node_param && workspace && ((x && gy) || B == 0), SLG_E_ARG,
              "fc_soft_bwd: null pointer");
  SLG_REQUIRE(node_kind == SLG_NODE_GATE16 || node_kind == SLG_NODE_WALSH ||
                  node_kind == SLG_NODE_MULTILINEAR2,
              SLG_E_ARG, "fc_soft_bwd: node_kind %d", node_kind);
  SLG_REQUIRE(B >= 0 && IN > 0 && OUT > 0 && K >= 1 && K <= 16 && B < (1LL << 31) &&
                  IN < (1LL << 28) && OUT < (1LL << 28) && (int64_t)B * IN < (1LL << 40),
              SLG_E_SHAPE, "fc_soft_bwd: bad sizes");
  const BwdPlan p = bwd_plan(B, IN, OUT, K);
  SLG_REQUIRE(p.Sx && p.Sw, SLG_E_UNSUPPORTED, "fc_soft_bwd: IN=%lld does not fit LDS",
              (long long)IN);
  SLG_REQUIRE(workspace_floats >= p.rec_floats + p.part_floats, SLG_E_ARG,
              "fc_soft_bwd: workspace of %lld floats, %lld needed", (long long)workspace_floats,
              (long long)(p.rec_floats + p.part_floats));
  hipStream_t st = as_stream(stream);
  float* rec = workspace;
  float* part = workspace + p.rec_floats;
  hipLaunchKernelGGL(fc_soft_pack_records_kernel, dim3((unsigned)cdiv(p.rec_floats, 256)),
                     dim3(256), 0, st, cand, w, node_param, (int)OUT, K, (int)IN, rec);
  SLG_LAUNCH_CHECK("fc_soft_pack_records");
  const bool want_w = gw || gnp;
  if (B > 0) {
    ParamView pv{};
    pv.rec = rec;
    float* pp = want_w ? part : nullptr;
    int rc = 0;
    switch (node_kind) {
      case SLG_NODE_GATE16:
        rc = bwd_node<SLG_NODE_GATE16>(x, B, IN, OUT, K, pv, inv_tau, gy, gx, pp, p, st); break;
      case SLG_NODE_WALSH:
        rc = bwd_node<SLG_NODE_WALSH>(x, B, IN, OUT, K, pv, inv_tau, gy, gx, pp, p, st); break;
      default:
        rc = bwd_node<SLG_NODE_MULTILINEAR2>(x, B, IN, OUT, K, pv, inv_tau, gy, gx, pp, p, st);
        break;
    }
    if (rc) return rc;
  }
  if (want_w) {
    const int NR = B > 0 ? p.NR : 0;  // no samples: zero gradients
    const int64_t n = (int64_t)(2 * K + 4) * OUT;
    hipLaunchKernelGGL(fc_soft_bwd_reduce_kernel, dim3((unsigned)cdiv(n, 256)), dim3(256), 0, st,
                       part, NR, (int)OUT, K, gw, gnp);
    SLG_LAUNCH_CHECK("fc_soft_bwd_reduce");
  }
  return 0;
}

}  // extern "C"
