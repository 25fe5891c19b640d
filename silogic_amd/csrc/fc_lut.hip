// FC layers of n-input LUT nodes (arity 2..6) for gfx950: the multilinear
// node (silogic/nodes.py:165-189) and the DWN-style hybrid node (nodes.py:
// 198-206; the reference's fused op kernels/multilinear.py:1-176). Output o
// of a layer with Top-K (or fixed, K = 1) wiring reads operands
//   a_j = sum_k w[o,j,k] * x[cand[o,j,k]],   j < n,
// and, with s = sigmoid(logits) [OUT, 2^n] and address bit j = leaf j,
//   multilinear: y = sum_p s[o,p] * prod_j (bit_j(p) ? a_j : 1 - a_j)
//   hybrid:      y = s[o, sum_j (a_j >= 0.5) << j]  (gradient of the former).
// Hard: y = (logits[o, addr] > 0) at the address of the hard operands.
//
// Soft forward: a workgroup owns S samples (staged in LDS, transposed) and
// 1024 outputs (four waves of four 64-output chunks); lane = output. Each
// chunk's parameters are read from chunk-major records (one coalesced load
// per slot: candidates, weights, LUT values), so the multilinear LUT sits in
// registers for all S samples; the hybrid lane reads its one entry per sample.
//
// Backward (both nodes: the gradient of the multilinear form, which the
// hybrid node uses as its surrogate, multilinear.py:141-160). No value
// atomics; every sum has a fixed order:
//   A. per sample tile and 1024 outputs (the forward's shape): the operand
//      gradients ga_j = g * dy/da_j (interpolation of the LUT differences
//      over the other leaves) to gbr [B][n*OUT] and the operand values to
//      arows [B][n*OUT], both coalesced along the outputs;
//   W. one output per thread over a range of samples, x tiles in LDS: the
//      weight sums ga_j * x[cand] in registers, one partial per range;
//   C. one (output, low corner c1) per thread over a range of samples: the
//      corner sums g * prod_j (a_j or 1 - a_j) as A(c1) * B(c2) for all
//      high corners c2, one partial per range;
//   then the partials are added over ranges in order, and the input gradient
//   is the shared gather over the reference table (fc_bwd_input.h).
#include "fc_bwd_input.h"
#include "fc_soft_common.h"

#include <mutex>

extern "C" int64_t slg_fc_lut_soft_workspace(int64_t OUT, int32_t arity, int32_t K);

namespace slg {

// Record slots of a 64-output chunk: NA*KM candidate indices, NA*KM weights,
// 2^NA LUT values; word (chunk, slot, lane) at (chunk * nslot + slot) * 64 + lane.
__host__ __device__ constexpr int lut_nslot(int na, int km) { return 2 * na * km + (1 << na); }

// Records from cand [OUT,n,K] int32 (clamped to IN), w [OUT,n,K] and s
// [OUT,2^n]; K padded to KM with weight 0. One thread per record word; the
// words are written as integers (index words are not float values).
__global__ void __launch_bounds__(256) fc_lut_pack_kernel(const int* __restrict__ cand,
                                                          const float* __restrict__ w,
                                                          const float* __restrict__ s, int OUT,
                                                          int NA, int K, int KM, int IN,
                                                          uint32_t* __restrict__ rec) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int nslot = lut_nslot(NA, KM);
  const int64_t n = (int64_t)((OUT + 63) / 64) * nslot * 64;
  if (t >= n) return;
  const int lane = (int)(t & 63);
  const int64_t q = t >> 6;
  const int slot = (int)(q % nslot);
  const int chunk = (int)(q / nslot);
  const int o = min(chunk * 64 + lane, OUT - 1);
  const int NK = NA * KM;
  uint32_t v;
  if (slot < 2 * NK) {
    const int jk = slot < NK ? slot : slot - NK;
    const int j = jk / KM, k = jk - j * KM;
    if (k >= K) {
      v = 0u;  // index 0 / weight +0.0f
    } else {
      const int64_t idx = ((int64_t)o * NA + j) * K + k;
      v = slot < NK ? (uint32_t)min(max(cand[idx], 0), IN - 1) : __float_as_uint(w[idx]);
    }
  } else {
    v = __float_as_uint(s[(int64_t)o * (1 << NA) + (slot - 2 * NK)]);
  }
  rec[t] = v;
}

// Multilinear interpolation of the 2^NA values t (overwritten) at leaves a:
// leaf 0 pairs entries 2m, 2m+1 (address bit 0), then leaf 1, ...
template <int NA>
__device__ inline float lut_lerp(float (&t)[1 << NA], const float (&a)[NA]) {
#pragma unroll
  for (int j = 0; j < NA; ++j) {
#pragma unroll
    for (int m = 0; m < (1 << (NA - 1 - j)); ++m) t[m] = fmaf(a[j], t[2 * m + 1] - t[2 * m], t[2 * m]);
  }
  return t[0];
}

template <bool HYB, int NA, int KM, int S>
__global__ void __launch_bounds__(256) fc_lut_soft_kernel(const float* __restrict__ x, int B,
                                                          int IN, int OUT,
                                                          const float* __restrict__ rec,
                                                          int n_og, float* __restrict__ y) {
  constexpr int NP = 1 << NA;
  constexpr int NK = NA * KM;
  constexpr int NSLOT = lut_nslot(NA, KM);
  using vt = typename vecf<S>::t;
  extern __shared__ __align__(16) unsigned char smem[];
  vt* xs = reinterpret_cast<vt*>(smem);
  const int tile = (int)(blockIdx.x / (unsigned)n_og), og = (int)(blockIdx.x % (unsigned)n_og);
  const int b0 = tile * S;
  stage_rows<S, true>(xs, x, B, IN, b0);
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n64 = (OUT + 63) >> 6;
  for (int c = og * 16 + wave; c < min(n64, og * 16 + 16); c += 4) {
    const float* rc = rec + (int64_t)c * NSLOT * 64 + lane;
    int idx[NK];
    float wt[NK];
#pragma unroll
    for (int i = 0; i < NK; ++i) {
      idx[i] = __float_as_int(rc[i * 64]);
      wt[i] = rc[(NK + i) * 64];
    }
    float acc[S][NA];
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
      for (int j = 0; j < NA; ++j) acc[s][j] = 0.0f;
#pragma unroll
    for (int k = 0; k < KM; ++k) {
#pragma unroll
      for (int j = 0; j < NA; ++j) {
        const vt v = xs[idx[j * KM + k]];
#pragma unroll
        for (int s = 0; s < S; ++s) acc[s][j] = fmaf(wt[j * KM + k], lanev(v, s), acc[s][j]);
      }
    }
    const int o = c * 64 + lane;
    if constexpr (HYB) {
#pragma unroll
      for (int s = 0; s < S; ++s) {
        int addr = 0;
#pragma unroll
        for (int j = 0; j < NA; ++j) addr |= (acc[s][j] >= 0.5f ? 1 : 0) << j;
        const float val = rc[(2 * NK + addr) * 64];
        if (o < OUT && b0 + s < B) y[(int64_t)(b0 + s) * OUT + o] = val;
      }
    } else {
      float lut[NP];
#pragma unroll
      for (int p = 0; p < NP; ++p) lut[p] = rc[(2 * NK + p) * 64];
#pragma unroll
      for (int s = 0; s < S; ++s) {
        float t[NP];
#pragma unroll
        for (int p = 0; p < NP; ++p) t[p] = lut[p];
        const float val = lut_lerp<NA>(t, acc[s]);
        if (o < OUT && b0 + s < B) y[(int64_t)(b0 + s) * OUT + o] = val;
      }
    }
  }
}

// Hard LUT codes: idx[o][j] = the first candidate of slot j with the largest
// connection logit (TopK, connectomes.py:118-123; conn == NULL: K = 1) and
// tt[o] bit p = (logits[o][p] > 0) (nodes.py:180-187).
__global__ void __launch_bounds__(256) fc_lut_hard_prep_kernel(const int* __restrict__ cand,
                                                               const float* __restrict__ conn,
                                                               int OUT, int NA, int K, int IN,
                                                               const float* __restrict__ logits,
                                                               int* __restrict__ idx,
                                                               uint64_t* __restrict__ tt) {
  const int o = blockIdx.x * blockDim.x + threadIdx.x;
  if (o >= OUT) return;
  for (int j = 0; j < NA; ++j) {
    const int64_t base = ((int64_t)o * NA + j) * K;
    int best = 0;
    if (conn) {
      float bv = conn[base];
      for (int k = 1; k < K; ++k)
        if (conn[base + k] > bv) {  // first maximum (torch.argmax)
          bv = conn[base + k];
          best = k;
        }
    }
    idx[(int64_t)o * NA + j] = min(max(cand[base + best], 0), IN - 1);
  }
  uint64_t bits = 0;
  for (int p = 0; p < (1 << NA); ++p)
    if (logits[(int64_t)o * (1 << NA) + p] > 0.0f) bits |= 1ull << p;
  tt[o] = bits;
}


// ---------------------------------------------------------------------------
// backward kernels
// ---------------------------------------------------------------------------
// g * dy/da_j for every leaf j: interpolation over the other leaves (in
// increasing order) of the differences lut[p | bit j] - lut[p], reduced as a
// stream (entry q is combined with the pending left siblings of the levels
// where q has a 1 bit), so every index is a compile-time constant.
template <int NA>
__device__ inline void lut_leaf_grads(const float (&lut)[1 << NA], const float (&a)[NA], float g,
                                      float (&ga)[NA]) {
  constexpr int H2 = 1 << (NA - 1);
#pragma unroll
  for (int j = 0; j < NA; ++j) {
    float vo[NA];  // the other leaves, in increasing order
#pragma unroll
    for (int i = 0, m = 0; i < NA; ++i)
      if (i != j) vo[m++] = a[i];
    float st[NA];
#pragma unroll
    for (int q = 0; q < H2; ++q) {
      const int p0 = ((q >> j) << (j + 1)) | (q & ((1 << j) - 1));
      float val = lut[p0 | (1 << j)] - lut[p0];
      int lvl = 0;
#pragma unroll
      for (; lvl < NA - 1 && ((q >> lvl) & 1); ++lvl) val = fmaf(vo[lvl], val - st[lvl], st[lvl]);
      st[lvl] = val;
    }
    ga[j] = g * st[NA - 1];
  }
}

template <int NA, int KM, int S>
__global__ void __launch_bounds__(256) fc_lut_bwd_a_kernel(const float* __restrict__ x, int B,
                                                           int IN, int OUT,
                                                           const float* __restrict__ rec,
                                                           int n_og, const float* __restrict__ gy,
                                                           float* __restrict__ gbr,
                                                           float* __restrict__ arows) {
  constexpr int NP = 1 << NA;
  constexpr int NK = NA * KM;
  constexpr int NSLOT = lut_nslot(NA, KM);
  using vt = typename vecf<S>::t;
  extern __shared__ __align__(16) unsigned char smem[];
  vt* xs = reinterpret_cast<vt*>(smem);
  const int tile = (int)(blockIdx.x / (unsigned)n_og), og = (int)(blockIdx.x % (unsigned)n_og);
  const int b0 = tile * S;
  stage_rows<S, true>(xs, x, B, IN, b0);
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n64 = (OUT + 63) >> 6;
  const int64_t row = (int64_t)NA * OUT;
  for (int c = og * 16 + wave; c < min(n64, og * 16 + 16); c += 4) {
    const float* rc = rec + (int64_t)c * NSLOT * 64 + lane;
    int idx[NK];
    float wt[NK];
#pragma unroll
    for (int i = 0; i < NK; ++i) {
      idx[i] = __float_as_int(rc[i * 64]);
      wt[i] = rc[(NK + i) * 64];
    }
    float lut[NP];
#pragma unroll
    for (int p = 0; p < NP; ++p) lut[p] = rc[(2 * NK + p) * 64];
    float acc[S][NA];
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
      for (int j = 0; j < NA; ++j) acc[s][j] = 0.0f;
#pragma unroll
    for (int k = 0; k < KM; ++k) {
#pragma unroll
      for (int j = 0; j < NA; ++j) {
        const vt v = xs[idx[j * KM + k]];
#pragma unroll
        for (int s = 0; s < S; ++s) acc[s][j] = fmaf(wt[j * KM + k], lanev(v, s), acc[s][j]);
      }
    }
    const int o = c * 64 + lane;
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const int b = b0 + s;
      if (o < OUT && b < B) {
        const float g = gy[(int64_t)b * OUT + o];
        float ga[NA];
        lut_leaf_grads<NA>(lut, acc[s], g, ga);
#pragma unroll
        for (int j = 0; j < NA; ++j) {
          gbr[(int64_t)b * row + (int64_t)j * OUT + o] = ga[j];
          if (arows) arows[(int64_t)b * row + (int64_t)j * OUT + o] = acc[s][j];
        }
      }
    }
  }
}

// Weight sums of one output per thread over sample tiles [t0, t1):
// part [NR][NK][OUT] (slot j*KM + k).
template <int NA, int KM, int S>
__global__ void __launch_bounds__(512) fc_lut_bwd_w_kernel(const float* __restrict__ x, int B,
                                                           int IN, int OUT,
                                                           const float* __restrict__ rec,
                                                           const float* __restrict__ gbr,
                                                           int n_orange, int tiles_per_range,
                                                           float* __restrict__ part) {
  constexpr int NK = NA * KM;
  constexpr int NSLOT = lut_nslot(NA, KM);
  using vt = typename vecf<S>::t;
  extern __shared__ __align__(16) unsigned char smem[];
  vt* xs = reinterpret_cast<vt*>(smem);
  const int r_o = (int)(blockIdx.x % (unsigned)n_orange);
  const int r_b = (int)(blockIdx.x / (unsigned)n_orange);
  const int o = r_o * blockDim.x + threadIdx.x;
  const bool valid = o < OUT;
  const int oc = min(o, OUT - 1);
  const float* rc = rec + (int64_t)(oc >> 6) * NSLOT * 64 + (oc & 63);
  int idx[NK];
#pragma unroll
  for (int i = 0; i < NK; ++i) idx[i] = __float_as_int(rc[i * 64]);
  float sw[NK];
#pragma unroll
  for (int i = 0; i < NK; ++i) sw[i] = 0.0f;
  const int64_t row = (int64_t)NA * OUT;
  const int n_tiles = (B + S - 1) / S;
  const int t_end = min(n_tiles, (r_b + 1) * tiles_per_range);
  for (int t = r_b * tiles_per_range; t < t_end; ++t) {
    const int b0 = t * S;
    __syncthreads();  // the previous tile's reads are done
    stage_rows<S, false>(xs, x, B, IN, b0);
    __syncthreads();
#pragma unroll
    for (int j = 0; j < NA; ++j) {
      float ga[S];
#pragma unroll
      for (int s = 0; s < S; ++s)
        ga[s] = (valid && b0 + s < B) ? gbr[(int64_t)(b0 + s) * row + (int64_t)j * OUT + o] : 0.0f;
#pragma unroll
      for (int k = 0; k < KM; ++k) {
        const vt v = xs[idx[j * KM + k]];
#pragma unroll
        for (int s = 0; s < S; ++s) sw[j * KM + k] = fmaf(ga[s], lanev(v, s), sw[j * KM + k]);
      }
    }
  }
  if (valid) {
    float* base = part + (int64_t)r_b * NK * OUT + o;
#pragma unroll
    for (int i = 0; i < NK; ++i) base[(int64_t)i * OUT] = sw[i];
  }
}

// Corner sums: thread (output o, low corner c1) over samples [r*spr,
// (r+1)*spr): for every high corner c2, sum of g * A(c1) * B(c2); part
// [NR][2^NA][OUT] (corner c1 + (c2 << H1)). The NC1 threads of an output are
// adjacent lanes, so one wave load of an operand row serves all of them.
template <int NA>
__global__ void __launch_bounds__(256) fc_lut_bwd_c_kernel(const float* __restrict__ arows,
                                                           const float* __restrict__ gy, int B,
                                                           int OUT, int spr,
                                                           float* __restrict__ part) {
  constexpr int H1 = NA / 2, NC1 = 1 << H1, NC2 = 1 << (NA - H1), NP = 1 << NA;
  const int o = blockIdx.x * (256 / NC1) + threadIdx.x / NC1;
  const int c1 = threadIdx.x % NC1, r = blockIdx.y;
  if (o >= OUT) return;
  float acc[NC2];
#pragma unroll
  for (int i = 0; i < NC2; ++i) acc[i] = 0.0f;
  const int64_t row = (int64_t)NA * OUT;
  const int b_end = min(B, (r + 1) * spr);
  for (int b = r * spr; b < b_end; ++b) {
    float a[NA];
#pragma unroll
    for (int j = 0; j < NA; ++j) a[j] = arows[(int64_t)b * row + (int64_t)j * OUT + o];
    float A = gy[(int64_t)b * OUT + o];
#pragma unroll
    for (int j = 0; j < H1; ++j) A *= ((c1 >> j) & 1) ? a[j] : 1.0f - a[j];
    float bw[NC2];
    bw[0] = A;
#pragma unroll
    for (int j = H1; j < NA; ++j) {
      const int sz = 1 << (j - H1);
#pragma unroll
      for (int i = 0; i < sz; ++i) {
        bw[i + sz] = bw[i] * a[j];
        bw[i] = bw[i] * (1.0f - a[j]);
      }
    }
#pragma unroll
    for (int c2 = 0; c2 < NC2; ++c2) acc[c2] += bw[c2];
  }
  float* base = part + (int64_t)r * NP * OUT + o;
#pragma unroll
  for (int c2 = 0; c2 < NC2; ++c2) base[(int64_t)(c1 + (c2 << H1)) * OUT] = acc[c2];
}

// out = sum over ranges of part [NR][NC][OUT] in fixed order (16 columns per
// workgroup, 16 thread rows over the ranges), scattered as
//   weights (mode 0): column (slot j*KM + k, o) -> gw[(o*NA + j)*K + k] for k < K
//   corners (mode 1): column (p, o) -> gs[o*NC + p].
__global__ void __launch_bounds__(256) fc_lut_bwd_reduce_kernel(const float* __restrict__ part,
                                                                int NR, int NC, int OUT, int mode,
                                                                int NA, int KM, int K,
                                                                float* __restrict__ out) {
  __shared__ float rs[16][17];
  const int col = threadIdx.x & 15, rw = threadIdx.x >> 4;
  const int64_t t = (int64_t)blockIdx.x * 16 + col;
  const int64_t n = (int64_t)NC * OUT;
  float s = 0.0f;
  if (t < n)
    for (int r = rw; r < NR; r += 16) s += part[(int64_t)r * n + t];
  rs[rw][col] = s;
  __syncthreads();
  if (rw != 0 || t >= n) return;
  float sum = 0.0f;
  for (int q = 0; q < 16; ++q) sum += rs[q][col];
  const int c = (int)(t / OUT), o = (int)(t - (int64_t)c * OUT);
  if (mode == 0) {
    const int j = c / KM, k = c - j * KM;
    if (k < K) out[((int64_t)o * NA + j) * K + k] = sum;
  } else {
    out[(int64_t)o * NC + c] = sum;
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
static int lut_km(int K) { return K <= 1 ? 1 : (K <= 4 ? 4 : 8); }

static inline int64_t round4i(int64_t n) { return (n + 3) & ~int64_t(3); }

static int lut_tile(int64_t IN) {
  const int64_t cap = std::min<int64_t>(device_lds_bytes(), 160 * 1024);
  for (int s : {4, 2, 1})
    if (IN * s * 4 <= cap) return s;
  return 0;
}

template <bool HYB, int NA, int KM, int S>
static int launch_lut_fwd(const float* x, int64_t B, int64_t IN, int64_t OUT, const float* rec,
                          float* y, hipStream_t st) {
  auto kern = fc_lut_soft_kernel<HYB, NA, KM, S>;
  const size_t lds = (size_t)IN * S * 4;
  if (lds > 65536) {
    hipError_t e = hipFuncSetAttribute((const void*)kern,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) {
      set_error("fc_lut_soft: LDS %zu: %s", lds, hipGetErrorString(e));
      return (int)e;
    }
  }
  const int64_t n_og = cdiv(OUT, 1024), n_tiles = cdiv(B, S);
  SLG_REQUIRE(n_og * n_tiles < (1LL << 31), SLG_E_SHAPE, "fc_lut_soft: grid too large");
  hipLaunchKernelGGL(kern, dim3((unsigned)(n_og * n_tiles)), dim3(256), lds, st, x, (int)B,
                     (int)IN, (int)OUT, rec, (int)n_og, y);
  SLG_LAUNCH_CHECK("fc_lut_soft");
  return 0;
}

template <bool HYB, int NA, int KM>
static int lut_fwd_s(int S, const float* x, int64_t B, int64_t IN, int64_t OUT, const float* rec,
                     float* y, hipStream_t st) {
  if (S == 4) return launch_lut_fwd<HYB, NA, KM, 4>(x, B, IN, OUT, rec, y, st);
  if (S == 2) return launch_lut_fwd<HYB, NA, KM, 2>(x, B, IN, OUT, rec, y, st);
  return launch_lut_fwd<HYB, NA, KM, 1>(x, B, IN, OUT, rec, y, st);
}

template <bool HYB, int NA>
static int lut_fwd_k(int KM, int S, const float* x, int64_t B, int64_t IN, int64_t OUT,
                     const float* rec, float* y, hipStream_t st) {
  if (KM == 1) return lut_fwd_s<HYB, NA, 1>(S, x, B, IN, OUT, rec, y, st);
  if (KM == 4) return lut_fwd_s<HYB, NA, 4>(S, x, B, IN, OUT, rec, y, st);
  return lut_fwd_s<HYB, NA, 8>(S, x, B, IN, OUT, rec, y, st);
}

template <bool HYB>
static int lut_fwd_n(int NA, int KM, int S, const float* x, int64_t B, int64_t IN, int64_t OUT,
                     const float* rec, float* y, hipStream_t st) {
  switch (NA) {
    case 2: return lut_fwd_k<HYB, 2>(KM, S, x, B, IN, OUT, rec, y, st);
    case 3: return lut_fwd_k<HYB, 3>(KM, S, x, B, IN, OUT, rec, y, st);
    case 4: return lut_fwd_k<HYB, 4>(KM, S, x, B, IN, OUT, rec, y, st);
    case 5: return lut_fwd_k<HYB, 5>(KM, S, x, B, IN, OUT, rec, y, st);
    default: return lut_fwd_k<HYB, 6>(KM, S, x, B, IN, OUT, rec, y, st);
  }
}


// Backward plan. Workspace (4-byte words): records | gbr | arows | part_w |
// part_c | input-gradient part.
struct LutBwdPlan {
  int S, Sw, KM;
  int n_orange, NRw, tiles_per_range;  // pass W
  int NRc, spr;                        // pass C
  int64_t rec, gbr, arows, partw, partc, inp;
  int64_t total() const { return rec + gbr + arows + partw + partc + inp; }
};

static LutBwdPlan lut_bwd_plan(int64_t B, int64_t IN, int64_t OUT, int NA, int K) {
  LutBwdPlan p{};
  p.S = lut_tile(IN);
  p.Sw = std::min(p.S, NA * lut_km(K) > 24 ? 1 : 2);  // pass W: registers for the sums
  p.KM = lut_km(K);
  const int NP = 1 << NA, NK = NA * p.KM;
  const int64_t Bm = std::max<int64_t>(B, 1);
  const int64_t cus = device_cus();
  // W: 512 outputs per workgroup, one round of resident workgroups
  p.n_orange = (int)cdiv(OUT, 512);
  const int64_t n_tiles = p.Sw ? cdiv(Bm, p.Sw) : 1;
  const int64_t lds = std::max<int64_t>(IN * std::max(p.Sw, 1) * 4, 1);
  const int64_t slots = std::max<int64_t>(1, std::min<int64_t>(4, (160 * 1024) / lds)) * cus;
  p.NRw = (int)std::max<int64_t>(1, std::min<int64_t>(n_tiles, slots / p.n_orange));
  p.tiles_per_range = (int)cdiv(n_tiles, p.NRw);
  p.NRw = (int)cdiv(n_tiles, p.tiles_per_range);
  // C: about 8 waves per CU
  const int64_t ctiles = cdiv(OUT, 256) * (1 << (NA / 2));
  p.NRc = (int)std::max<int64_t>(1, std::min<int64_t>(Bm, cdiv(8 * cus, ctiles)));
  p.spr = (int)cdiv(Bm, p.NRc);
  p.NRc = (int)cdiv(Bm, p.spr);
  p.rec = slg_fc_lut_soft_workspace(OUT, NA, K);
  p.gbr = round4i(Bm * NA * OUT);
  p.arows = p.gbr;
  p.partw = round4i((int64_t)p.NRw * NK * OUT);
  p.partc = round4i((int64_t)p.NRc * NP * OUT);
  p.inp = fc_input_grad_floats(B, IN, OUT, NA, K);
  return p;
}

template <int NA, int KM, int S>
static int launch_lut_bwd_a(const float* x, int64_t B, int64_t IN, int64_t OUT, const float* rec,
                            const float* gy, float* gbr, float* arows, hipStream_t st) {
  auto kern = fc_lut_bwd_a_kernel<NA, KM, S>;
  const size_t lds = (size_t)IN * S * 4;
  if (lds > 65536) {
    hipError_t e = hipFuncSetAttribute((const void*)kern,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) {
      set_error("fc_lut_bwd: LDS %zu: %s", lds, hipGetErrorString(e));
      return (int)e;
    }
  }
  const int64_t n_og = cdiv(OUT, 1024), n_tiles = cdiv(B, S);
  hipLaunchKernelGGL(kern, dim3((unsigned)(n_og * n_tiles)), dim3(256), lds, st, x, (int)B,
                     (int)IN, (int)OUT, rec, (int)n_og, gy, gbr, arows);
  SLG_LAUNCH_CHECK("fc_lut_bwd_a");
  return 0;
}

template <int NA, int KM, int S>
static int launch_lut_bwd_w(const float* x, int64_t B, int64_t IN, int64_t OUT, const float* rec,
                            const float* gbr, const LutBwdPlan& p, float* part, hipStream_t st) {
  auto kern = fc_lut_bwd_w_kernel<NA, KM, S>;
  const size_t lds = (size_t)IN * S * 4;
  if (lds > 65536) {
    hipError_t e = hipFuncSetAttribute((const void*)kern,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) {
      set_error("fc_lut_bwd: LDS %zu: %s", lds, hipGetErrorString(e));
      return (int)e;
    }
  }
  hipLaunchKernelGGL(kern, dim3((unsigned)(p.n_orange * p.NRw)), dim3(512), lds, st, x, (int)B,
                     (int)IN, (int)OUT, rec, gbr, p.n_orange, p.tiles_per_range, part);
  SLG_LAUNCH_CHECK("fc_lut_bwd_w");
  return 0;
}

template <int NA, int KM>
static int lut_bwd_t(const float* x, int64_t B, int64_t IN, int64_t OUT, const float* rec,
                     const float* gy, const LutBwdPlan& p, float* gbr, float* arows, float* partw,
                     float* partc, hipStream_t st) {
  int rc = p.S == 4 ? launch_lut_bwd_a<NA, KM, 4>(x, B, IN, OUT, rec, gy, gbr, arows, st)
         : p.S == 2 ? launch_lut_bwd_a<NA, KM, 2>(x, B, IN, OUT, rec, gy, gbr, arows, st)
                    : launch_lut_bwd_a<NA, KM, 1>(x, B, IN, OUT, rec, gy, gbr, arows, st);
  if (rc) return rc;
  if (partw) {
    rc = p.Sw == 2 ? launch_lut_bwd_w<NA, KM, 2>(x, B, IN, OUT, rec, gbr, p, partw, st)
                   : launch_lut_bwd_w<NA, KM, 1>(x, B, IN, OUT, rec, gbr, p, partw, st);
    if (rc) return rc;
  }
  if (partc) {
    hipLaunchKernelGGL(fc_lut_bwd_c_kernel<NA>,
                       dim3((unsigned)cdiv(OUT, 256 >> (NA / 2)), (unsigned)p.NRc), dim3(256), 0,
                       st, arows, gy, (int)B, (int)OUT, p.spr, partc);
    SLG_LAUNCH_CHECK("fc_lut_bwd_c");
  }
  return 0;
}

template <int NA>
static int lut_bwd_k(const float* x, int64_t B, int64_t IN, int64_t OUT, const float* rec,
                     const float* gy, const LutBwdPlan& p, float* gbr, float* arows, float* partw,
                     float* partc, hipStream_t st) {
  if (p.KM == 1) return lut_bwd_t<NA, 1>(x, B, IN, OUT, rec, gy, p, gbr, arows, partw, partc, st);
  if (p.KM == 4) return lut_bwd_t<NA, 4>(x, B, IN, OUT, rec, gy, p, gbr, arows, partw, partc, st);
  return lut_bwd_t<NA, 8>(x, B, IN, OUT, rec, gy, p, gbr, arows, partw, partc, st);
}

// The forward of both entry points: records into `rec` (rec_floats long),
// then the layer.
static int lut_soft_fwd(const float* x, int64_t B, int64_t IN, int64_t OUT, int32_t arity,
                        int32_t K, const int32_t* cand, const float* w, const float* s,
                        int32_t hybrid, float* y, float* rec, int64_t rec_floats, hipStream_t st,
                        const char* what) {
  SLG_REQUIRE(cand && w && s && ((x && y) || B == 0), SLG_E_ARG, "%s: null pointer", what);
  SLG_REQUIRE(arity >= 2 && arity <= 6 && K >= 1 && K <= 8, SLG_E_SHAPE,
              "%s: arity %d / K %d outside 2..6 / 1..8", what, arity, K);
  SLG_REQUIRE(B >= 0 && IN > 0 && OUT > 0 && B < (1LL << 31) && IN < (1LL << 28) &&
                  OUT < (1LL << 26),
              SLG_E_SHAPE, "%s: bad sizes", what);
  const int S = lut_tile(IN);
  SLG_REQUIRE(S > 0, SLG_E_UNSUPPORTED, "%s: IN=%lld does not fit LDS", what, (long long)IN);
  const int KM = lut_km(K);
  const int64_t need = slg_fc_lut_soft_workspace(OUT, arity, K);
  SLG_REQUIRE(rec_floats >= need, SLG_E_ARG, "%s: workspace of %lld floats, %lld needed", what,
              (long long)rec_floats, (long long)need);
  hipLaunchKernelGGL(fc_lut_pack_kernel, dim3((unsigned)cdiv(need, 256)), dim3(256), 0, st, cand,
                     w, s, (int)OUT, arity, K, KM, (int)IN, reinterpret_cast<uint32_t*>(rec));
  SLG_LAUNCH_CHECK("fc_lut_pack");
  if (B == 0) return 0;
  return hybrid ? lut_fwd_n<true>(arity, KM, S, x, B, IN, OUT, rec, y, st)
                : lut_fwd_n<false>(arity, KM, S, x, B, IN, OUT, rec, y, st);
}

// Static scratch of slg_fc_lut_soft_fwd_noalloc: the records of one layer,
// at most kLutScratchFloats words (16 MiB; 26 214 outputs of arity 6 with
// K = 8, 116 508 of arity 2). Every GPU the library runs on holds its own
// copy until the process ends. Host code never passes the array's name to a
// kernel: it is a host-side stand-in, and the device address comes from
// hipGetSymbolAddress, taken once per device with that device current.
constexpr int64_t kLutScratchFloats = int64_t(4) << 20;
static __device__ __align__(256) float scratch[kLutScratchFloats];

namespace {
constexpr int kScratchDevices = 64;
float* g_scratch[kScratchDevices];
hipError_t g_scratch_rc[kScratchDevices];
std::once_flag g_scratch_once[kScratchDevices];
}  // namespace

static int lut_scratch(float** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    set_error("fc_lut_soft_noalloc: hipGetDevice: %s", hipGetErrorString(e));
    return (int)e;
  }
  SLG_REQUIRE(dev >= 0 && dev < kScratchDevices, SLG_E_UNSUPPORTED,
              "fc_lut_soft_noalloc: device %d beyond %d", dev, kScratchDevices);
  std::call_once(g_scratch_once[dev], [dev] {
    void* p = nullptr;
    g_scratch_rc[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    g_scratch[dev] = g_scratch_rc[dev] == hipSuccess ? static_cast<float*>(p) : nullptr;
  });
  if (g_scratch_rc[dev] != hipSuccess || !g_scratch[dev]) {
    const hipError_t rc = g_scratch_rc[dev] != hipSuccess ? g_scratch_rc[dev] : hipErrorUnknown;
    set_error("fc_lut_soft_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", dev,
              hipGetErrorString(rc));
    return (int)rc;
  }
  *out = g_scratch[dev];
  return 0;
}

}  // namespace slg

using namespace slg;

extern "C" {

int64_t slg_fc_lut_soft_workspace(int64_t OUT, int32_t arity, int32_t K) {
  if (OUT <= 0 || arity < 2 || arity > 6 || K < 1 || K > 8) return -1;
  return cdiv(OUT, 64) * 64 * (int64_t)lut_nslot(arity, lut_km(K));
}

int slg_fc_lut_soft_fwd(const float* x, int64_t B, int64_t IN, int64_t OUT, int32_t arity,
                        int32_t K, const int32_t* cand, const float* w, const float* s,
                        int32_t hybrid, float* y, float* workspace, int64_t workspace_floats,
                        slg_stream_t stream) {
  SLG_REQUIRE(workspace, SLG_E_ARG, "fc_lut_soft: null workspace");
  return lut_soft_fwd(x, B, IN, OUT, arity, K, cand, w, s, hybrid, y, workspace,
                      workspace_floats, as_stream(stream), "fc_lut_soft");
}

int slg_fc_lut_soft_fwd_noalloc(const float* x, int64_t B, int64_t IN, int64_t OUT,
                                int32_t arity, int32_t K, const int32_t* cand, const float* w,
                                const float* s, int32_t hybrid, float* y, slg_stream_t stream) {
  const int64_t need = slg_fc_lut_soft_workspace(OUT, arity, K);
  SLG_REQUIRE(need <= kLutScratchFloats, SLG_E_SHAPE,
              "fc_lut_soft_noalloc: %lld outputs need %lld record floats, the static scratch "
              "holds %lld (use slg_fc_lut_soft_fwd with a workspace)",
              (long long)OUT, (long long)need, (long long)kLutScratchFloats);
  float* rec = nullptr;
  const int rc = lut_scratch(&rec);
  if (rc) return rc;
  return lut_soft_fwd(x, B, IN, OUT, arity, K, cand, w, s, hybrid, y, rec, kLutScratchFloats,
                      as_stream(stream), "fc_lut_soft_noalloc");
}

int64_t slg_fc_lut_soft_bwd_workspace(int64_t B, int64_t IN, int64_t OUT, int32_t arity,
                                      int32_t K) {
  if (B < 0 || IN <= 0 || OUT <= 0 || arity < 2 || arity > 6 || K < 1 || K > 8 ||
      OUT >= (1LL << 26) || (int64_t)arity * OUT * K >= (1LL << 31))
    return -1;
  if (!lut_tile(IN)) return -1;
  return lut_bwd_plan(B, IN, OUT, arity, K).total();
}

int slg_fc_lut_soft_bwd(const float* x, int64_t B, int64_t IN, int64_t OUT, int32_t arity,
                        int32_t K, const int32_t* cand, const float* w, const float* s,
                        const float* gy, float* gx, float* gw, float* gs, float* workspace,
                        int64_t workspace_floats, slg_stream_t stream) {
  SLG_REQUIRE(cand && w && s && workspace && ((x && gy) || B == 0), SLG_E_ARG,
              "fc_lut_bwd: null pointer");
  SLG_REQUIRE(arity >= 2 && arity <= 6 && K >= 1 && K <= 8, SLG_E_SHAPE,
              "fc_lut_bwd: arity %d / K %d outside 2..6 / 1..8", arity, K);
  SLG_REQUIRE(B >= 0 && IN > 0 && OUT > 0 && B < (1LL << 31) && IN < (1LL << 28) &&
                  OUT < (1LL << 26) && (int64_t)arity * OUT * K < (1LL << 31) &&
                  B * arity * OUT < (1LL << 40),
              SLG_E_SHAPE, "fc_lut_bwd: bad sizes");
  SLG_REQUIRE(lut_tile(IN) > 0, SLG_E_UNSUPPORTED, "fc_lut_bwd: IN=%lld does not fit LDS",
              (long long)IN);
  const LutBwdPlan p = lut_bwd_plan(B, IN, OUT, arity, K);
  SLG_REQUIRE(workspace_floats >= p.total(), SLG_E_ARG,
              "fc_lut_bwd: workspace of %lld floats, %lld needed", (long long)workspace_floats,
              (long long)p.total());
  hipStream_t st = as_stream(stream);
  float* rec = workspace;
  float* gbr = rec + p.rec;
  float* arows = gbr + p.gbr;
  float* partw = arows + p.arows;
  float* partc = partw + p.partw;
  float* inp = partc + p.partc;
  hipLaunchKernelGGL(fc_lut_pack_kernel, dim3((unsigned)cdiv(p.rec, 256)), dim3(256), 0, st, cand,
                     w, s, (int)OUT, arity, K, p.KM, (int)IN, reinterpret_cast<uint32_t*>(rec));
  SLG_LAUNCH_CHECK("fc_lut_pack");
  if (B > 0 && (gx || gw || gs)) {
    int rc = 0;
    float* pw = gw ? partw : nullptr;
    float* pc = gs ? partc : nullptr;
    float* ar = gs ? arows : nullptr;
    switch (arity) {
      case 2: rc = lut_bwd_k<2>(x, B, IN, OUT, rec, gy, p, gbr, ar, pw, pc, st); break;
      case 3: rc = lut_bwd_k<3>(x, B, IN, OUT, rec, gy, p, gbr, ar, pw, pc, st); break;
      case 4: rc = lut_bwd_k<4>(x, B, IN, OUT, rec, gy, p, gbr, ar, pw, pc, st); break;
      case 5: rc = lut_bwd_k<5>(x, B, IN, OUT, rec, gy, p, gbr, ar, pw, pc, st); break;
      default: rc = lut_bwd_k<6>(x, B, IN, OUT, rec, gy, p, gbr, ar, pw, pc, st); break;
    }
    if (rc) return rc;
    if (gx) {
      rc = fc_input_grad(gbr, B, IN, OUT, arity, K, cand, w, inp, gx, st);
      if (rc) return rc;
    }
  }
  const int NRw = B > 0 ? p.NRw : 0, NRc = B > 0 ? p.NRc : 0;  // no samples: zeros
  if (gw) {
    const int NK = arity * p.KM;
    hipLaunchKernelGGL(fc_lut_bwd_reduce_kernel, dim3((unsigned)cdiv((int64_t)NK * OUT, 16)),
                       dim3(256), 0, st, partw, NRw, NK, (int)OUT, 0, arity, p.KM, K, gw);
  }
  if (gs) {
    const int NP = 1 << arity;
    hipLaunchKernelGGL(fc_lut_bwd_reduce_kernel, dim3((unsigned)cdiv((int64_t)NP * OUT, 16)),
                       dim3(256), 0, st, partc, NRc, NP, (int)OUT, 1, arity, p.KM, K, gs);
  }
  SLG_LAUNCH_CHECK("fc_lut_bwd_reduce");
  return 0;
}

int slg_fc_lut_hard_prep(const int32_t* cand, const float* conn, int64_t OUT, int32_t arity,
                         int32_t K, int64_t IN, const float* logits, int32_t* idx, uint64_t* tt,
                         slg_stream_t stream) {
  SLG_REQUIRE(cand && logits && idx && tt, SLG_E_ARG, "fc_lut_hard_prep: null pointer");
  SLG_REQUIRE(arity >= 1 && arity <= 6 && K >= 1 && OUT > 0 && OUT < (1LL << 31) && IN > 0 &&
                  IN < (1LL << 31),
              SLG_E_SHAPE, "fc_lut_hard_prep: bad sizes");
  hipLaunchKernelGGL(fc_lut_hard_prep_kernel, dim3((unsigned)cdiv(OUT, 256)), dim3(256), 0,
                     as_stream(stream), cand, conn, (int)OUT, arity, K, (int)IN, logits, idx, tt);
  SLG_LAUNCH_CHECK("fc_lut_hard_prep");
  return 0;
}

}  // extern "C"
