// FC soft backward for gfx950 (the gradients DenseLogicFn / WarpLogicFn
// return: kernels/dense.py:46-75, 107-120; warp.py:33-64): given x [B,IN],
// the layer's candidates / weights / node parameters and gy [B,OUT], write
//   gx  [B,IN]      = sum over (o, k) of ga[b,o] * w_a[o,k] at x[b, cand_a[o,k]]
//                     (and the b side),
//   gw  [OUT,2,K]   = sum over b of ga[b,o] * x[b, cand_a[o,k]] (and b),
//   gnp [OUT,4]     = sum over b of dL/dparam,
// where ga, gb are the node's operand gradients at the recomputed operands.
//
// No atomics on values, and every sum runs in a fixed order (the gradients
// are the same bits on every call):
//   * records: the parameters repacked into the forward's chunk-major
//     records, so every parameter load of a wave is one 16-byte load per lane.
//   * fc_soft_bwd_w_kernel: a workgroup owns 1024 outputs (one per thread)
//     and a range of samples; it streams that range through LDS in S-sample
//     tiles, keeps its outputs' 2K + 4 weight / parameter gradient sums in
//     registers (one partial per sample range), and writes every (sample,
//     output) operand gradient ga, gb to gbr [B][2*OUT] (coalesced rows).
//   * fc_soft_bwd_reduce_kernel: sums the partials over sample ranges in
//     ascending order.
//   * the input gradient is the transposed problem: a table lists, for every
//     input, the (row = side*OUT + o, weight) of the references to it in
//     ascending reference order (count, scan, place, rank kernels); gbr is
//     transposed to sample-minor rows gab [2*OUT][LB]; the gather kernel
//     walks each input's entries with its lanes along samples.
#include "fc_soft_common.h"
#include "fc_bwd_input.h"
#include "ref_table.h"

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
      const float y = sigmoid_hw(bilinear(a, b, p) * inv_tau);
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
// (quad q of output o at ((o/64)*rec_quads(K)+q)*64 + o%64; words
// idx_a | idx_b << 16, w_a, w_b, zero padding, params). One thread per
// record word.
__global__ void __launch_bounds__(256) fc_soft_pack_records_kernel(const int* __restrict__ cand,
                                                                   const float* __restrict__ w,
                                                                   const float* __restrict__ np,
                                                                   int OUT, int K, int IN,
                                                                   uint32_t* __restrict__ rec) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int RQ = rec_quads(K);
  const int64_t nq = (int64_t)((OUT + 63) / 64) * RQ * 64;
  if (t >= nq * 4) return;
  const int e = (int)(t & 3);
  const int64_t Q = t >> 2;
  const int lane = (int)(Q % 64);
  const int q = (int)((Q / 64) % RQ);
  const int c = (int)(Q / (64 * (int64_t)RQ));
  const int o = min(c * 64 + lane, OUT - 1);
  const int word = q * 4 + e;
  // words are written as integers: an index pair with idx_b >= 32640 is a
  // NaN bit pattern, which a float move could quieten
  uint32_t v = 0u;
  if (word < K) {
    const uint32_t ia = (uint32_t)min(max(cand[(int64_t)o * 2 * K + word], 0), IN - 1);
    const uint32_t ib = (uint32_t)min(max(cand[(int64_t)o * 2 * K + K + word], 0), IN - 1);
    v = ia | (ib << 16);
  } else if (word < 3 * K) {
    v = __float_as_uint(w[(int64_t)o * 2 * K + (word - K)]);  // w_a then w_b
  } else if (word >= 4 * (RQ - 1)) {
    v = __float_as_uint(np[(int64_t)o * 4 + (word - 4 * (RQ - 1))]);
  }
  rec[t] = v;
}

template <int KC>
constexpr int bwd_threads() { return KC > 0 && KC <= 8 ? 1024 : 512; }

// ---------------------------------------------------------------------------
// Transposed reference table: for every input i, the references (o, side, k)
// whose candidate is i, in ascending r = o*2K + side*K + k (a fixed order, so
// the input gradient sums in the same order on every call), as entries
// (row, weight) with row = side*OUT + o indexing the operand-gradient rows.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256) fc_soft_bwd_keys_kernel(const int* __restrict__ cand, int R,
                                                               int IN, int* __restrict__ keys) {
  const int r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r < R) keys[r] = min(max(cand[r], 0), IN - 1);
}

__global__ void __launch_bounds__(256) fc_soft_bwd_entries_kernel(const int* __restrict__ sorted,
                                                                  int R, int OUT, int NS, int K,
                                                                  const float* __restrict__ w,
                                                                  int2* __restrict__ ent) {
  const int j = blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= R) return;
  const int r = sorted[j], SK = NS * K;  // r = (o * NS + side) * K + k
  const int o = r / SK, side = (r - o * SK) / K;
  ent[j] = make_int2(side * OUT + o, __float_as_int(w[r]));
}

// gab [R2][LB] = transpose of gbr [B][R2] (rows b >= B of gab's columns are
// zero), through a 64 x 64 LDS tile; float4 loads along gbr rows when R2 is
// a multiple of 4, float4 stores along gab rows (LB is a multiple of 64).
__global__ void __launch_bounds__(256) fc_soft_bwd_transpose_kernel(const float* __restrict__ gbr,
                                                                    int B, int R2, int64_t LB,
                                                                    int n_rtiles,
                                                                    float* __restrict__ gab) {
  __shared__ float t[64][65];  // [b][r]
  const int rt = blockIdx.x % n_rtiles, bt = blockIdx.x / n_rtiles;
  const int r0 = rt * 64, b0 = bt * 64;
  const int c4 = threadIdx.x & 15, q = threadIdx.x >> 4;  // 16 float4 columns x 16 rows
  if ((R2 & 3) == 0) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int bl = q + 16 * k, b = b0 + bl, r = r0 + 4 * c4;
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (b < B && r < R2) v = *reinterpret_cast<const float4*>(gbr + (int64_t)b * R2 + r);
      t[bl][4 * c4] = v.x;
      t[bl][4 * c4 + 1] = v.y;
      t[bl][4 * c4 + 2] = v.z;
      t[bl][4 * c4 + 3] = v.w;
    }
  } else {
    const int c = threadIdx.x & 63, qq = threadIdx.x >> 6;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const int bl = qq + 4 * k, b = b0 + bl, r = r0 + c;
      t[bl][c] = (b < B && r < R2) ? gbr[(int64_t)b * R2 + r] : 0.0f;
    }
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int rl = q + 16 * k, r = r0 + rl;
    if (r < R2) {
      const float4 v = make_float4(t[4 * c4][rl], t[4 * c4 + 1][rl], t[4 * c4 + 2][rl],
                                   t[4 * c4 + 3][rl]);
      *reinterpret_cast<float4*>(gab + (int64_t)r * LB + b0 + 4 * c4) = v;
    }
  }
}

// Input gradient from the node-gradient rows gab [2*OUT][LB] (row side*OUT+o,
// sample-minor): gx[b][i] = sum over the entries e of input i, in table
// order, of weight(e) * gab[row(e)][b]. A workgroup owns 4*IW inputs x 64*V
// samples. Each wave walks the entries of its IW consecutive inputs as one
// flat range (contiguous in the table) with its lanes along samples: the
// entries are wave-uniform (scalar loads, the next 8 prefetched), each costs
// one coalesced 64V-sample row-segment load, and 8 such loads are in flight.
// An input's sum is complete when the walk reaches the next input's start.
// The results go through LDS so gx rows are written contiguously.
template <int V, int IW>
__global__ void __launch_bounds__(256) fc_soft_bwd_gather_kernel(const float* __restrict__ gab,
                                                                 int64_t LB, int B, int IN,
                                                                 const int* __restrict__ start,
                                                                 const int2* __restrict__ ent,
                                                                 int n_itiles, int n_blocks,
                                                                 float* __restrict__ gx) {
  using vt = typename vecf<V>::t;
  constexpr int NI = 4 * IW;       // inputs per workgroup
  constexpr int NS = 64 * V;       // samples per workgroup
  constexpr int G = 8;             // entries per step
  __shared__ float T[NI][NS + 1];  // [input][sample]
  const int L = (int)xcd_logical_id(blockIdx.x, gridDim.x);
  if (L >= n_blocks) return;
  const int it = L % n_itiles, sc = L / n_itiles;
  const int i0 = it * NI;
  const int b0 = sc * NS;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const float* col = gab + b0 + lane * V;
  const int ia = i0 + wave * IW;
  const int iend = min(ia + IW, IN);
  int cur = ia;  // input whose sum is being accumulated
  float acc[V];
#pragma unroll
  for (int v = 0; v < V; ++v) acc[v] = 0.0f;
  if (ia < iend) {
    int e = start[ia];
    const int e_end = start[iend];
    int nb = start[ia + 1];  // first entry of input cur + 1
    int2 qn[G];
#pragma unroll
    for (int u = 0; u < G; ++u) qn[u] = ent[min(e + u, max(e_end - 1, 0))];
    while (e < e_end) {
      int2 q[G];
#pragma unroll
      for (int u = 0; u < G; ++u) q[u] = qn[u];
      vt g[G];
#pragma unroll
      for (int u = 0; u < G; ++u) g[u] = *reinterpret_cast<const vt*>(col + (int64_t)q[u].x * LB);
      const int en = e + G;
#pragma unroll
      for (int u = 0; u < G; ++u) qn[u] = ent[min(en + u, e_end - 1)];
#pragma unroll
      for (int u = 0; u < G; ++u) {
        if (e + u < e_end) {
          while (e + u == nb) {  // input cur is complete (inputs without entries: zero)
#pragma unroll
            for (int v = 0; v < V; ++v) {
              T[cur - i0][lane * V + v] = acc[v];
              acc[v] = 0.0f;
            }
            ++cur;
            nb = start[cur + 1];
          }
#pragma unroll
          for (int v = 0; v < V; ++v) acc[v] = fmaf(__int_as_float(q[u].y), lanev(g[u], v), acc[v]);
        }
      }
      e = en;
    }
  }
  for (; cur < ia + IW; ++cur) {  // the last input with entries, then empty ones
#pragma unroll
    for (int v = 0; v < V; ++v) {
      T[cur - i0][lane * V + v] = acc[v];
      acc[v] = 0.0f;
    }
  }
  __syncthreads();
  const int c = threadIdx.x % NI;
#pragma unroll 4
  for (int s = threadIdx.x / NI; s < NS; s += 256 / NI) {
    if (b0 + s < B && i0 + c < IN) gx[(int64_t)(b0 + s) * IN + i0 + c] = T[c][s];
  }
}

// Weight / node-parameter gradient partials of one output per thread over a
// range of sample tiles: part [NR][2K+4][OUT] (components w_a[0..K),
// w_b[0..K), param[0..4)); with gbr, also the node's operand gradients
// ga, gb of every (sample, output) at gbr[b][o], gbr[b][OUT+o] (rows of
// 2*OUT, coalesced along the outputs), transposed for the gather kernel.
//
// WIDE (rows wider than LDS): one sample per tile, staged slab by slab (SL
// inputs at a time); each thread keeps its output's 2K gathered operands in
// registers, filling those in the current slab, then runs the same math.
// Parameters come from the separate arrays (32-bit indices).
template <int NODE, int KC, int S, bool WIDE>
__global__ void __launch_bounds__((bwd_threads<KC>()))
fc_soft_bwd_w_kernel(const float* __restrict__ x, int B, int IN, int OUT, int Kr, ParamView pv,
                     float inv_tau, const float* __restrict__ gy, int n_orange, int tiles_per_range,
                     float* __restrict__ part, float* __restrict__ gbr, int SL) {
  static_assert(!WIDE || S == 1, "slab staging takes one sample per tile");
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
  load_params<KC, KM, !WIDE>(P, min(o, OUT - 1), K, pv);
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
    vt xa[WIDE ? KM : 1], xb[WIDE ? KM : 1];  // wide: the gathered operands
    if constexpr (WIDE) {
#pragma unroll
      for (int k = 0; k < KM; ++k) xa[k] = xb[k] = 0.0f;
      for (int s0 = 0; s0 < IN; s0 += SL) {
        const int sl = min(SL, IN - s0);
        __syncthreads();  // the previous slab's reads are done
        for (int i = threadIdx.x; i < sl; i += blockDim.x)
          xs[i] = b0 < B ? x[(int64_t)b0 * IN + s0 + i] : 0.0f;
        __syncthreads();
#pragma unroll
        for (int k = 0; k < KM; ++k) {
          if (KC > 0 || k < K) {
            const uint32_t ra = (uint32_t)ia[k] - (uint32_t)s0, rb = (uint32_t)ib[k] - (uint32_t)s0;
            if (ra < (uint32_t)sl) xa[k] = xs[ra];
            if (rb < (uint32_t)sl) xb[k] = xs[rb];
          }
        }
      }
    } else {
      __syncthreads();  // the previous tile's reads are done
      stage_rows<S, false>(xs, x, B, IN, b0);  // the other output ranges re-read these rows
      __syncthreads();
    }
    auto opa = [&](int k) -> vt {
      if constexpr (WIDE) return xa[k]; else return xs[ia[k]];
    };
    auto opb = [&](int k) -> vt {
      if constexpr (WIDE) return xb[k]; else return xs[ib[k]];
    };
    vt A = zero_vec<vt>(), Bv = zero_vec<vt>();
#pragma unroll
    for (int k = 0; k < KM; ++k) {
      if (KC > 0 || k < K) {
        fma_acc(A, P.fa[k], opa(k));
        fma_acc(Bv, P.fb[k], opb(k));
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
    if (gbr != nullptr && valid) {  // sample rows of 2*OUT; tiles end at or before LB
#pragma unroll
      for (int s = 0; s < S; ++s) {
        gbr[(int64_t)(b0 + s) * (2 * OUT) + o] = ga[s];
        gbr[(int64_t)(b0 + s) * (2 * OUT) + OUT + o] = gb[s];
      }
    }
    // second pass over the candidates: sum_s ga[s] * x[s][cand]
#pragma unroll
    for (int k = 0; k < KM; ++k) {
      if (KC > 0 || k < K) {
        const vt va = opa(k), vb = opb(k);
#pragma unroll
        for (int s = 0; s < S; ++s) {
          swa[k] = fmaf(ga[s], lanev(va, s), swa[k]);
          swb[k] = fmaf(gb[s], lanev(vb, s), swb[k]);
        }
      }
    }
  }
  if (part != nullptr && valid) {
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

// gw [OUT,2,K], gnp [OUT,4] = sum over ranges r of part[r]: a workgroup
// takes 16 columns (component, output); its 16 thread rows sum the ranges
// r = row (mod 16) in ascending order, and the 16 row sums are added in row
// order (a fixed order on every call).
__global__ void __launch_bounds__(256) fc_soft_bwd_reduce_kernel(const float* __restrict__ part,
                                                                 int NR, int OUT, int K,
                                                                 float* __restrict__ gw,
                                                                 float* __restrict__ gnp) {
  __shared__ float rs[16][17];
  const int col = threadIdx.x & 15, row = threadIdx.x >> 4;
  const int64_t t = (int64_t)blockIdx.x * 16 + col;
  const int NC = 2 * K + 4;
  const int64_t n = (int64_t)NC * OUT;
  float s = 0.0f;
  if (t < n)
    for (int r = row; r < NR; r += 16) s += part[(int64_t)r * n + t];
  rs[row][col] = s;
  __syncthreads();
  if (row != 0 || t >= n) return;
  float sum = 0.0f;
  for (int q = 0; q < 16; ++q) sum += rs[q][col];
  const int c = (int)(t / OUT), o = (int)(t - (int64_t)c * OUT);
  if (c < 2 * K) {
    if (gw) gw[(int64_t)o * 2 * K + c] = sum;  // c = side * K + k
  } else if (gnp) {
    gnp[(int64_t)o * 4 + (c - 2 * K)] = sum;
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

constexpr int kGatherV = 4;              // samples per lane in the gather kernel
constexpr int kGatherIW = 8;             // inputs per wave in the gather kernel
constexpr int kGatherSamples = 64 * kGatherV;
constexpr int kGatherInputs = 4 * kGatherIW;

inline int64_t round4(int64_t n) { return (n + 3) & ~int64_t(3); }

// Workspace (in 4-byte words): records | partials | gbr | input-gradient part.
struct BwdPlan {
  int Sw;              // samples per LDS tile of the weight kernel (0 = unsupported)
  int SL;              // > 0: rows wider than LDS, staged SL inputs at a time (Sw = 1)
  int n_orange, NR, tiles_per_range;
  int64_t rec_floats, part_floats, gbr_floats, in_floats;
  int64_t total() const { return rec_floats + part_floats + gbr_floats + in_floats; }
};

// Input-gradient workspace: gab [nsides*OUT][LB] | keys | table | entries.
struct InPlan {
  int64_t LB, R, gab_floats, keys_ints, table_ints, ent_ints;
  int64_t total() const { return gab_floats + keys_ints + table_ints + ent_ints; }
};

static InPlan in_plan(int64_t B, int64_t IN, int64_t OUT, int nsides, int K) {
  InPlan q{};
  q.LB = cdiv(std::max<int64_t>(B, 1), kGatherSamples) * kGatherSamples;
  q.R = nsides * OUT * (int64_t)K;
  q.gab_floats = nsides * OUT * q.LB;
  q.keys_ints = round4(q.R);
  q.table_ints = ref_table_ints(q.R, IN);
  q.ent_ints = 2 * q.R;
  return q;
}

int64_t fc_input_grad_floats(int64_t B, int64_t IN, int64_t OUT, int nsides, int K) {
  return in_plan(B, IN, OUT, nsides, K).total();
}

int fc_input_grad(const float* gbr, int64_t B, int64_t IN, int64_t OUT, int nsides, int K,
                  const int32_t* cand, const float* w, float* ws, float* gx, hipStream_t st) {
  const InPlan q = in_plan(B, IN, OUT, nsides, K);
  SLG_REQUIRE(q.R < (1LL << 31) && nsides * OUT < (1LL << 31), SLG_E_SHAPE,
              "fc input gradient: too many references");
  float* gab = ws;
  int* keys = reinterpret_cast<int*>(gab + q.gab_floats);
  int* table = keys + q.keys_ints;
  int2* ent = reinterpret_cast<int2*>(table + q.table_ints);  // 8-byte aligned: offsets are even
  const int R = (int)q.R;
  hipLaunchKernelGGL(fc_soft_bwd_keys_kernel, dim3((unsigned)cdiv(R, 256)), dim3(256), 0, st,
                     cand, R, (int)IN, keys);
  RefTable tb{};
  int rc = build_ref_table(keys, R, IN, table, st, &tb);
  if (rc) return rc;
  hipLaunchKernelGGL(fc_soft_bwd_entries_kernel, dim3((unsigned)cdiv(R, 256)), dim3(256), 0, st,
                     tb.sorted, R, (int)OUT, nsides, K, w, ent);
  SLG_LAUNCH_CHECK("fc input gradient entries");
  const int R2 = (int)(nsides * OUT);
  const int n_rtiles = (int)cdiv(R2, 64);
  const int64_t n_tr = n_rtiles * (q.LB / 64);
  SLG_REQUIRE(n_tr < (1LL << 31), SLG_E_SHAPE, "fc input gradient: grid too large");
  hipLaunchKernelGGL(fc_soft_bwd_transpose_kernel, dim3((unsigned)n_tr), dim3(256), 0, st, gbr,
                     (int)B, R2, q.LB, n_rtiles, gab);
  SLG_LAUNCH_CHECK("fc input gradient transpose");
  const int n_itiles = (int)cdiv(IN, kGatherInputs);
  const int64_t n_blocks = n_itiles * (q.LB / kGatherSamples);
  SLG_REQUIRE(n_blocks < (1LL << 31) - 8, SLG_E_SHAPE, "fc input gradient: grid too large");
  const int64_t grid = cdiv(n_blocks, 8) * 8;  // a multiple of 8 for the XCD remap
  auto gather = fc_soft_bwd_gather_kernel<kGatherV, kGatherIW>;
  hipLaunchKernelGGL(gather, dim3((unsigned)grid), dim3(256), 0, st, gab, q.LB, (int)B, (int)IN,
                     tb.start, ent, n_itiles, (int)n_blocks, gx);
  SLG_LAUNCH_CHECK("fc input gradient gather");
  return 0;
}

static BwdPlan bwd_plan(int64_t B, int64_t IN, int64_t OUT, int K) {
  BwdPlan p{};
  p.Sw = bwd_tile(IN, 4);   // x tile
  if (K == 8) p.Sw = std::min(p.Sw, 2);  // 4-sample tiles overflow 128 VGPRs at 1024 threads
  if (p.Sw == 0) {  // slab staging, one sample per tile
    p.Sw = 1;
    p.SL = (int)(std::min<int64_t>(device_lds_bytes(), 160 * 1024) / 4);
  }
  const int threads = K == 8 || K == 4 ? 1024 : 512;
  p.n_orange = (int)cdiv(OUT, threads);
  const int64_t n_tiles = p.Sw ? cdiv(std::max<int64_t>(B, 1), p.Sw) : 1;
  // one round of workgroups: as many sample ranges as resident slots allow
  // (2048 threads and 160 KB of LDS per CU); a partial second round would
  // double the kernel's time
  const int64_t lds = p.SL ? (int64_t)p.SL * 4 : std::max<int64_t>(IN * std::max(p.Sw, 1) * 4, 1);
  const int64_t per_cu = std::max<int64_t>(1, std::min<int64_t>(2048 / threads, (160 * 1024) / lds));
  const int64_t slots = per_cu * device_cus();
  p.NR = (int)std::max<int64_t>(1, std::min<int64_t>(n_tiles, slots / p.n_orange));
  p.tiles_per_range = (int)cdiv(n_tiles, p.NR);
  p.NR = (int)cdiv(n_tiles, p.tiles_per_range);
  const int64_t LB = cdiv(std::max<int64_t>(B, 1), kGatherSamples) * kGatherSamples;
  p.rec_floats = p.SL ? 0 : cdiv(OUT, 64) * 64 * (int64_t)rec_quads(K) * 4;
  p.part_floats = round4((int64_t)p.NR * (2 * K + 4) * OUT);
  p.gbr_floats = 2 * OUT * LB;  // rows b < n_tiles * Sw <= LB
  p.in_floats = fc_input_grad_floats(B, IN, OUT, 2, K);
  return p;
}

template <int NODE, int KC, int S, bool WIDE = false>
static int launch_bwd_w(const float* x, int64_t B, int64_t IN, int64_t OUT, int K,
                        const ParamView& pv, float inv_tau, const float* gy, const BwdPlan& p,
                        float* part, float* gbr, hipStream_t st) {
  auto kern = fc_soft_bwd_w_kernel<NODE, KC, S, WIDE>;
  const size_t lds = WIDE ? (size_t)p.SL * 4 : (size_t)IN * S * 4;
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
                     p.tiles_per_range, part, gbr, p.SL);
  SLG_LAUNCH_CHECK("fc_soft_bwd_w");
  return 0;
}

template <int NODE, int KC>
static int bwd_node_k(const float* x, int64_t B, int64_t IN, int64_t OUT, int K,
                      const ParamView& pv, float inv_tau, const float* gy, float* part, float* gbr,
                      const BwdPlan& p, hipStream_t st) {
  if (p.SL) return launch_bwd_w<NODE, KC, 1, true>(x, B, IN, OUT, K, pv, inv_tau, gy, p, part, gbr, st);
  if constexpr (KC != 8) {  // K = 8 tiles stop at 2 samples (the plan caps them)
    if (p.Sw == 4)
      return launch_bwd_w<NODE, KC, 4>(x, B, IN, OUT, K, pv, inv_tau, gy, p, part, gbr, st);
  }
  return p.Sw >= 2 ? launch_bwd_w<NODE, KC, 2>(x, B, IN, OUT, K, pv, inv_tau, gy, p, part, gbr, st)
                   : launch_bwd_w<NODE, KC, 1>(x, B, IN, OUT, K, pv, inv_tau, gy, p, part, gbr, st);
}

template <int NODE>
static int bwd_node(const float* x, int64_t B, int64_t IN, int64_t OUT, int K, const ParamView& pv,
                    float inv_tau, const float* gy, float* part, float* gbr, const BwdPlan& p,
                    hipStream_t st) {
  if (K == 8) return bwd_node_k<NODE, 8>(x, B, IN, OUT, K, pv, inv_tau, gy, part, gbr, p, st);
  if (K == 4) return bwd_node_k<NODE, 4>(x, B, IN, OUT, K, pv, inv_tau, gy, part, gbr, p, st);
  return bwd_node_k<NODE, 0>(x, B, IN, OUT, K, pv, inv_tau, gy, part, gbr, p, st);
}

}  // namespace slg

using namespace slg;

extern "C" {

int64_t slg_fc_soft_bwd_workspace(int64_t B, int64_t IN, int64_t OUT, int32_t K) {
  if (B < 0 || IN <= 0 || OUT <= 0 || K < 1 || K > 16 || 2 * OUT * K >= (1LL << 31)) return -1;
  const BwdPlan p = bwd_plan(B, IN, OUT, K);
  // records hold 16-bit input indices; wider rows take the slab kernel,
  // which reads the separate arrays
  if (!p.Sw || (IN > 65536 && !p.SL)) return -1;
  return p.total();
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
                  IN < (1LL << 28) && OUT < (1LL << 28) && 2 * OUT * K < (1LL << 31) &&
                  (int64_t)B * IN < (1LL << 40),
              SLG_E_SHAPE, "fc_soft_bwd: bad sizes");
  const BwdPlan p = bwd_plan(B, IN, OUT, K);
  SLG_REQUIRE(p.Sw && (IN <= 65536 || p.SL), SLG_E_UNSUPPORTED,
              "fc_soft_bwd: IN=%lld does not fit LDS", (long long)IN);
  SLG_REQUIRE(workspace_floats >= p.total(), SLG_E_ARG,
              "fc_soft_bwd: workspace of %lld floats, %lld needed", (long long)workspace_floats,
              (long long)p.total());
  hipStream_t st = as_stream(stream);
  float* rec = workspace;
  float* part = rec + p.rec_floats;
  float* gbr = part + p.part_floats;
  float* in_ws = gbr + p.gbr_floats;
  if (!p.SL) {
    hipLaunchKernelGGL(fc_soft_pack_records_kernel, dim3((unsigned)cdiv(p.rec_floats, 256)),
                       dim3(256), 0, st, cand, w, node_param, (int)OUT, K, (int)IN,
                       reinterpret_cast<uint32_t*>(rec));
    SLG_LAUNCH_CHECK("fc_soft_pack_records");
  }
  const bool want_w = gw || gnp;
  const bool want_x = gx != nullptr && B > 0;
  if (B > 0 && (want_w || want_x)) {
    ParamView pv{};
    if (p.SL) {  // the slab kernel reads the separate arrays
      pv.ca = cand;
      pv.cb = cand + K;
      pv.wa = w;
      pv.wb = w + K;
      pv.np = node_param;
      pv.cstride = 2 * K;
      pv.wstride = 2 * K;
      pv.npstride = 4;
    } else {
      pv.rec = rec;
    }
    float* pp = want_w ? part : nullptr;
    float* pg = want_x ? gbr : nullptr;
    int rc = 0;
    switch (node_kind) {
      case SLG_NODE_GATE16:
        rc = bwd_node<SLG_NODE_GATE16>(x, B, IN, OUT, K, pv, inv_tau, gy, pp, pg, p, st); break;
      case SLG_NODE_WALSH:
        rc = bwd_node<SLG_NODE_WALSH>(x, B, IN, OUT, K, pv, inv_tau, gy, pp, pg, p, st); break;
      default:
        rc = bwd_node<SLG_NODE_MULTILINEAR2>(x, B, IN, OUT, K, pv, inv_tau, gy, pp, pg, p, st);
        break;
    }
    if (rc) return rc;
  }
  if (want_x) {
    int rc = fc_input_grad(gbr, B, IN, OUT, 2, K, cand, w, in_ws, gx, st);
    if (rc) return rc;
  }
  if (want_w) {
    const int NR = B > 0 ? p.NR : 0;  // no samples: zero gradients
    const int64_t n = (int64_t)(2 * K + 4) * OUT;
    hipLaunchKernelGGL(fc_soft_bwd_reduce_kernel, dim3((unsigned)cdiv(n, 16)), dim3(256), 0, st,
                       part, NR, (int)OUT, K, gw, gnp);
    SLG_LAUNCH_CHECK("fc_soft_bwd_reduce");
  }
  return 0;
}

}  // extern "C"
