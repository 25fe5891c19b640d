// Pieces shared by the FC soft forward (fc_soft.hip) and backward
// (fc_soft_bwd.hip): vector types, the parameter views and record loads,
// and the node evaluation.
#pragma once
#include "slg_common.h"

namespace slg {

// Native vector types: one ds_read_b64 / ds_read_b128 per gather (HIP's
// float2/float4 structs are split into scalar LDS reads by the compiler).
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
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
// The per-(sample, output) sigmoid of the walsh node: 1 / (1 + 2^(-z log2 e))
// with the hardware exp2 and reciprocal (v_exp_f32, v_rcp_f32: about 1 ulp
// each, against some twenty instructions for expf and an IEEE divide). Large
// |z| saturates to exactly 0 or 1 as the divide form does.
__device__ inline float sigmoid_hw(float z) {
  const float e = __builtin_amdgcn_exp2f(z * -1.4426950408889634f);
  return __builtin_amdgcn_rcpf(1.0f + e);
}

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

// Stage V rows of x (samples b0 .. b0+V-1, zeros past B) into LDS
// transposed: dst[i] holds the V samples of input i. Threads load float4 runs
// of 4 inputs from each row (NBAT batches in flight per thread), then scatter
// them to 4 input slots; rows whose length is not a multiple of 4 go one
// input at a time. STREAM: non-temporal loads (rows read once).
template <int V, bool STREAM, int NBAT = (V == 4 ? 2 : 4)>
__device__ inline void stage_rows(typename vecf<V>::t* __restrict__ dst,
                                  const float* __restrict__ x, int B, int IN, int b0) {
  using vt = typename vecf<V>::t;
  if ((IN & 3) == 0) {
    const int n4 = IN >> 2;
    for (int q0 = threadIdx.x; q0 < n4; q0 += NBAT * blockDim.x) {
      float4 t[NBAT][V];
#pragma unroll
      for (int u = 0; u < NBAT; ++u) {
        const int q = q0 + u * blockDim.x;
#pragma unroll
        for (int v = 0; v < V; ++v) {
          const int b = b0 + v;
          const float* p = x + (int64_t)b * IN + 4 * q;
          t[u][v] = (b < B && q < n4)
                        ? (STREAM ? ld_stream4(p) : *reinterpret_cast<const float4*>(p))
                        : make_float4(0.f, 0.f, 0.f, 0.f);
        }
      }
#pragma unroll
      for (int u = 0; u < NBAT; ++u) {
        const int q = q0 + u * blockDim.x;
        if (q < n4) {
#pragma unroll
          for (int cc = 0; cc < 4; ++cc) {
            float e[V];
#pragma unroll
            for (int v = 0; v < V; ++v) e[v] = lanev(t[u][v], cc);
            dst[4 * q + cc] = make_vec<V>(e);
          }
        }
      }
    }
  } else {
    for (int i = threadIdx.x; i < IN; i += blockDim.x) {
      float e[V];
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const int b = b0 + v;
        const float* p = x + (int64_t)b * IN + i;
        e[v] = (b < B) ? (STREAM ? __builtin_nontemporal_load(p) : *p) : 0.0f;
      }
      dst[i] = make_vec<V>(e);
    }
  }
}

// Node evaluation on the two gathered operands (silogic/nodes.py:86-91 for
// gate16, the warp_logic form of kernels/warp.py:14-31 for walsh,
// nodes.py:174-178 with n = 2 for multilinear). Written as explicit fmaf
// chains, so every kernel that evaluates a node (per layer, whole network,
// wide rows, backward recompute) rounds it the same way whatever the
// compiler would contract.
__device__ inline float bilinear(float a, float b, const float4& p) {
  return fmaf(p.w, a * b, fmaf(p.z, b, fmaf(p.y, a, p.x)));
}
template <int NODE>
__device__ inline float node_eval(float a, float b, const float4& p, float inv_tau) {
  if constexpr (NODE == SLG_NODE_GATE16) {
    return bilinear(a, b, p);
  } else if constexpr (NODE == SLG_NODE_WALSH) {
    return sigmoid_hw(bilinear(a, b, p) * inv_tau);
  } else {
    // corners P = 0:(0,0) 1:(1,0) 2:(0,1) 3:(1,1) (bit j of P = slot j)
    const float ua = 1.0f - a, ub = 1.0f - b;
    return fmaf(a * b, p.w, fmaf(ua * b, p.z, fmaf(a * ub, p.y, (ua * ub) * p.x)));
  }
}

// Where one layer's parameters live: separate arrays (cand [OUT,2,K], w
// [OUT,2,K], node_param [OUT,4]) or one record per output (strides in 32-bit
// words; see slg_fc_soft_records).
struct ParamView {
  const int* ca;
  const int* cb;
  const float* wa;
  const float* wb;
  const float* np;
  int cstride, wstride, npstride;
  const float* rec;  // records (REC kernels): [ceil(OUT/64)][rec_quads(K)][64][4] words
};

// Quads per output record: K index words (idx_a | idx_b << 16, inputs below
// 65536), K words w_a, K words w_b, zero padding to a whole quad, then one
// quad of node parameters.
__host__ __device__ constexpr int rec_quads(int K) { return (3 * K + 3) / 4 + 1; }

// Per-output parameters held in registers: 2K candidate indices, 2K weights,
// 4 node coefficients.
template <int KM>
struct FcParams {
  int ia[KM], ib[KM];
  float fa[KM], fb[KM];
  float4 p;
};

// KC = compile-time candidate count (0 = runtime K <= 16, scalar loads).
// The loads are unconditional straight-line code, so the compiler's wait
// counts stay exact across loop iterations.
//
// Records (REC): output o's rec_quads(K) quads of 4 words live at quad index
// ((o / 64) * rec_quads(K) + q) * 64 + o % 64, so one 16-byte load per quad
// moves 1 KB of contiguous memory for the 64 outputs of a wave. Words 0..K-1
// hold idx_a | idx_b << 16, K..2K-1 w_a, 2K..3K-1 w_b, and the last quad the
// node parameters. The soft kernels re-read every record once per sample
// tile, so the 16-bit index pairs cut their record traffic by two quads of
// nine at K = 8.
template <int KC, int KM, bool REC>
__device__ inline void load_params(FcParams<KM>& P, int o, int K, const ParamView& pv) {
  if constexpr (REC) {
    const int RQ = rec_quads(K);
    const f32x4* r = reinterpret_cast<const f32x4*>(pv.rec) +
                     ((int64_t)(o >> 6) * RQ) * 64 + (o & 63);
    if constexpr (KC > 0 && (KC % 4) == 0) {
      constexpr int Q = KC / 4;
#pragma unroll
      for (int q = 0; q < Q; ++q) {
        const i32x4 c4 = __builtin_bit_cast(i32x4, r[(0 * Q + q) * 64]);
        const f32x4 u4 = r[(1 * Q + q) * 64];
        const f32x4 v4 = r[(2 * Q + q) * 64];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          P.ia[4 * q + e] = (int)((uint32_t)c4[e] & 0xFFFFu);
          P.ib[4 * q + e] = (int)((uint32_t)c4[e] >> 16);
          P.fa[4 * q + e] = u4[e];
          P.fb[4 * q + e] = v4[e];
        }
      }
    } else {
      const float* rw = reinterpret_cast<const float*>(r - (o & 63));  // quad 0 of lane 0
      const int l = o & 63;
      auto word = [&](int w) { return rw[((w >> 2) * 64 + l) * 4 + (w & 3)]; };
#pragma unroll
      for (int k = 0; k < KM; ++k) {
        if (k < K) {
          const uint32_t c = __float_as_uint(word(k));
          P.ia[k] = (int)(c & 0xFFFFu);
          P.ib[k] = (int)(c >> 16);
          P.fa[k] = word(K + k);
          P.fb[k] = word(2 * K + k);
        } else {
          P.ia[k] = 0; P.ib[k] = 0; P.fa[k] = 0.f; P.fb[k] = 0.f;
        }
      }
    }
    const f32x4 p4 = r[(RQ - 1) * 64];
    P.p = make_float4(p4[0], p4[1], p4[2], p4[3]);
    return;
  }
  if constexpr (KC > 0 && (KC % 4) == 0) {
    const int* ca = pv.ca + (int64_t)o * pv.cstride;
    const int* cb = pv.cb + (int64_t)o * pv.cstride;
    const float* wa = pv.wa + (int64_t)o * pv.wstride;
    const float* wb = pv.wb + (int64_t)o * pv.wstride;
#pragma unroll
    for (int q = 0; q < KC / 4; ++q) {
      const i32x4 a4 = *reinterpret_cast<const i32x4*>(ca + 4 * q);
      const i32x4 b4 = *reinterpret_cast<const i32x4*>(cb + 4 * q);
      const f32x4 u4 = *reinterpret_cast<const f32x4*>(wa + 4 * q);
      const f32x4 v4 = *reinterpret_cast<const f32x4*>(wb + 4 * q);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        P.ia[4 * q + e] = a4[e];
        P.ib[4 * q + e] = b4[e];
        P.fa[4 * q + e] = u4[e];
        P.fb[4 * q + e] = v4[e];
      }
    }
  } else {
#pragma unroll
    for (int k = 0; k < KM; ++k) {
      if (k < K) {
        P.ia[k] = pv.ca[(int64_t)o * pv.cstride + k];
        P.ib[k] = pv.cb[(int64_t)o * pv.cstride + k];
        P.fa[k] = pv.wa[(int64_t)o * pv.wstride + k];
        P.fb[k] = pv.wb[(int64_t)o * pv.wstride + k];
      } else {
        P.ia[k] = 0; P.ib[k] = 0; P.fa[k] = 0.f; P.fb[k] = 0.f;
      }
    }
  }
  const f32x4 p4 = *reinterpret_cast<const f32x4*>(pv.np + (int64_t)o * pv.npstride);
  P.p = make_float4(p4[0], p4[1], p4[2], p4[3]);
}

}  // namespace slg
