// ConvLogicTree soft backward for gfx950, with the fused 2x2 OR-pool (the
// gradients the reference's tree-conv ops return: kernels/conv.py:94-145,
// kernels/conv_topk.py:84-121, with F.max_pool2d's routing, layers.py:558-559).
// Given x [B,C,H,W], the trees' taps (cm, ch, cw), leaf weights w and node
// parameters, and gy [B,N,Ho,Wo] on the (pooled) output, write
//   gx  [B,C,H,W]   = sum over taps of w * (leaf gradient at the tap's output),
//   gw  [N,L,K]     = sum over samples and outputs of leaf gradient * tap value,
//   gnp             = sum over samples and outputs of dL/dparam.
// With pooling, each pooled output sends its gradient to the first window
// position (row-major) holding the window's maximum, as F.max_pool2d does.
//
// One kernel does the work; no value atomics, and every sum has a fixed
// order. A workgroup owns a group of TG trees and a range of samples; per
// sample (the image staged in LDS when it is small, else read through the
// caches) it
//   A. for each (tree, routed output): recomputes the leaf values at the
//      window positions with the forward's tap order, evaluates the tree
//      (conv_tree_eval: the forward's operations, so the routing compares
//      the forward's values), routes, and back-propagates to the leaves;
//      keeps the leaf gradients and the route in LDS, and adds leaf gradient
//      * tap value (and, for gate16 trees, each node's parameter gradient)
//      to per-thread sums;
//   B. gathers the input gradient of every pixel from its channel's taps in
//      the group (a table of (tree, leaf, dh, dw, weight) per (group,
//      channel), built once per call); for LUT trees, adds
//      each corner's gradient over the sample's outputs (from the leaf
//      values and upstream gradients kept in LDS) to per-thread sums.
// At the end of its range the workgroup reduces the per-thread sums over
// each tree's threads in LDS and writes them as one partial per range; small
// kernels then add the partials over ranges and, with several groups, the
// input-gradient partials over groups.
#include <math.h>

#include <type_traits>

#include "conv_tree.h"
#include "ref_table.h"

namespace slg {

constexpr int kBwdMaxK = 8;
constexpr int kBwdThreads = 1024;  // largest workgroup (LDS reduction buffer size)
constexpr int kBwdNodeAcc = 16;    // node-parameter sums per thread

// Workgroup size cap of a variant: LUT trees (their corner sums) and gate16
// trees of depth 3 need more than the 128 VGPRs of 1024-thread workgroups.
template <int NODE, int NLEAF>
__host__ __device__ constexpr int conv_bwd_threads() {
  return (NODE == SLG_NODE_GATE16 ? NLEAF >= 8 : true) ? 512 : 1024;
}

// Per-thread node-parameter sums: gate16 trees sum every node's four
// coefficients in phase A; LUT trees take up to 16 corners in phase B.
template <int NODE, int NLEAF>
__host__ __device__ constexpr int conv_bwd_nacc() {
  return NODE == SLG_NODE_GATE16 ? 4 * (NLEAF - 1) : kBwdNodeAcc;
}

struct ConvBwdArgs {
  int C, H, W, pad, kernel;
  int Ho, Wo, P;  // routed map (pooled or the full map) and its size
  int N, K, TG, TPT, NG, SPR, B;
  int J2;  // LUT trees: position slots per (tree, low-corner) item
  int KB;  // table buckets per (group, channel): kernel^2 (by tap offset) or 1
};

// LDS layout of one workgroup (offsets in floats).
struct ConvBwdLds {
  int xs, taps, par, raw, vq, gv, gq, route, red, total;
};

// XS: the image is staged (C*H*W floats). vq / gq (leaf values and upstream
// gradients at the routed positions) exist for LUT trees only.
template <int NODE, int NLEAF, bool POOL>
__host__ __device__ inline ConvBwdLds conv_bwd_lds(bool XS, int C, int CHW, int TG, int K, int P) {
  using Nd = ConvNode<NODE, NLEAF>;
  constexpr bool LUT = NODE != SLG_NODE_GATE16;
  ConvBwdLds L{};
  int o = 0;
  L.xs = o; o += XS ? (CHW + 3) & ~3 : 0;
  L.taps = o; o += TG * NLEAF * K * 4;     // int4 per tap
  L.par = o; o += (TG * Nd::NPR + 3) & ~3;
  L.raw = o; o += LUT ? ((TG * NLEAF * (Nd::NP / 2) + 3) & ~3) : 0;
  L.vq = o; o += LUT ? ((TG * NLEAF * P + 3) & ~3) : 0;
  L.gv = o; o += (TG * NLEAF * P + 3) & ~3;
  L.gq = o; o += LUT ? ((TG * P + 3) & ~3) : 0;
  L.route = o; o += POOL ? ((TG * P + 3) / 4 + 3) & ~3 : 0;  // bytes
  L.red = o; o += kBwdThreads;
  L.total = o;
  return L;
}

// Leaf gradients g * dy/dv_l of the tree at leaf values v.
// Gate16: also adds each node's parameter gradient U * (1, a, b, ab) to
// accn[4 * node ...].
template <int NODE, int NLEAF>
__device__ inline void conv_tree_leaf_grad(const float (&v)[NLEAF], const float* par,
                                           const float* raw, float g, float (&gl)[NLEAF],
                                           float* accn) {
  if constexpr (NODE == SLG_NODE_GATE16) {
    // node outputs level by level (ids level-major), then U from the root
    constexpr int NN = NLEAF - 1;
    float nv[NN], na[NN], nb_[NN];
    {
      int nb = 0, prev = -1;  // prev: first id of the previous level (-1: leaves)
#pragma unroll
      for (int cnt = NLEAF; cnt > 1; cnt >>= 1) {
#pragma unroll
        for (int m = 0; m < cnt / 2; ++m) {
          const float a = prev < 0 ? v[2 * m] : nv[prev + 2 * m];
          const float b = prev < 0 ? v[2 * m + 1] : nv[prev + 2 * m + 1];
          const float* c = par + 4 * (nb + m);
          na[nb + m] = a;
          nb_[nb + m] = b;
          nv[nb + m] = fmaf(b, fmaf(a, c[3], c[2]), fmaf(a, c[1], c[0]));
        }
        prev = nb;
        nb += cnt / 2;
      }
    }
    float U[NN];
    U[NN - 1] = g;
    // levels from the root down: level with cnt children starts at id base
    int base = NN - 1, cnt = 2;
#pragma unroll
    for (int lvl = 0; (1 << lvl) < NLEAF; ++lvl) {
      // nodes of this level: ids base .. base + cnt/2 - 1; children at the
      // previous level (ids base - cnt .. base - 1) or the leaves
      const int nodes = cnt / 2;
#pragma unroll
      for (int m = 0; m < nodes; ++m) {
        const int id = base + m;
        const float* c = par + 4 * id;
        accn[4 * id] += U[id];
        accn[4 * id + 1] += U[id] * na[id];
        accn[4 * id + 2] += U[id] * nb_[id];
        accn[4 * id + 3] += U[id] * (na[id] * nb_[id]);
        const float ua = U[id] * (c[1] + c[3] * nb_[id]);
        const float ub = U[id] * (c[2] + c[3] * na[id]);
        if (base - cnt < 0) {  // children are leaves
          gl[2 * m] = ua;
          gl[2 * m + 1] = ub;
        } else {
          U[base - cnt + 2 * m] = ua;
          U[base - cnt + 2 * m + 1] = ub;
        }
      }
      base -= cnt;
      cnt *= 2;
    }
  } else {
    // dy/dv_j = multilinear interpolation over the other leaves (in
    // increasing order) of the differences D[j][q] = s[p | bit j] - s[p],
    // p = q with a 0 inserted at bit j (raw holds D [NLEAF][2^(NLEAF-1)]).
    // The lerp tree is reduced as a stream: leaf q is combined with the
    // pending left siblings of the levels where q has a 1 bit.
    constexpr int H2 = 1 << (NLEAF - 1);
#pragma unroll
    for (int j = 0; j < NLEAF; ++j) {
      float vo[NLEAF];  // the other leaves, in increasing order
#pragma unroll
      for (int i = 0, m = 0; i < NLEAF; ++i)
        if (i != j) vo[m++] = v[i];
      float st[NLEAF];
      const float4* d4 = reinterpret_cast<const float4*>(raw + j * H2);
#pragma unroll
      for (int q4 = 0; q4 < (H2 + 3) / 4; ++q4) {
        float dq[4];
        if constexpr (H2 >= 4) {
          const float4 t = d4[q4];
          dq[0] = t.x; dq[1] = t.y; dq[2] = t.z; dq[3] = t.w;
        } else {
#pragma unroll
          for (int u = 0; u < H2; ++u) dq[u] = raw[j * H2 + u];
        }
#pragma unroll
        for (int u = 0; u < 4 && 4 * q4 + u < H2; ++u) {
          const int q = 4 * q4 + u;
          float val = dq[u];
          int lvl = 0;
#pragma unroll
          for (; lvl < NLEAF - 1 && ((q >> lvl) & 1); ++lvl)
            val = fmaf(vo[lvl], val - st[lvl], st[lvl]);
          st[lvl] = val;
        }
      }
      gl[j] = g * st[NLEAF - 1];
    }
    (void)par;
    (void)accn;
  }
}

template <int NODE, int NLEAF, bool POOL, int KM, bool XS>
__global__ void __launch_bounds__((conv_bwd_threads<NODE, NLEAF>()))
conv_soft_bwd_kernel(const float* __restrict__ x, const float* __restrict__ gy, ConvBwdArgs a,
                     const float* __restrict__ np, const float* __restrict__ wts,
                     const int* __restrict__ cm, const int* __restrict__ ch,
                     const int* __restrict__ cw, const int* __restrict__ tstart,
                     const int4* __restrict__ tent, float* __restrict__ gx_out,
                     float* __restrict__ part_w, float* __restrict__ part_np) {
  using Nd = ConvNode<NODE, NLEAF>;
  constexpr int NPR = Nd::NPR, NP = Nd::NP;
  constexpr bool LUT = NODE != SLG_NODE_GATE16;
  constexpr int NQ = POOL ? 4 : 1;
  constexpr int NACC = conv_bwd_nacc<NODE, NLEAF>();
  extern __shared__ __align__(16) float lds[];
  const int HW = a.H * a.W, CHW = a.C * HW;
  const ConvBwdLds L = conv_bwd_lds<NODE, NLEAF, POOL>(XS, a.C, CHW, a.TG, a.K, a.P);
  float* xs = lds + L.xs;
  int4* taps = reinterpret_cast<int4*>(lds + L.taps);
  float* par = lds + L.par;
  float* raw = lds + L.raw;
  float* vq = lds + L.vq;
  float* gv = lds + L.gv;
  float* gq = lds + L.gq;
  unsigned char* route = reinterpret_cast<unsigned char*>(lds + L.route);
  float* red = lds + L.red;

  const int g = (int)(blockIdx.x % (unsigned)a.NG);
  const int r = (int)(blockIdx.x / (unsigned)a.NG);
  const int n0 = g * a.TG;
  const int TG = a.TG, K = a.K, P = a.P;
  const int tid = threadIdx.x, T = blockDim.x;

  // taps and parameters of the group's trees (trees past N: zero weight)
  for (int i = tid; i < TG * NLEAF * K; i += T) {
    const int t = i / (NLEAF * K), lk = i - t * NLEAF * K;
    const int n = n0 + t;
    int4 e = make_int4(0, 0, 0, 0);
    if (n < a.N) {
      const int idx = n * NLEAF * K + lk;
      const int c_ = min(max(cm[idx], 0), a.C - 1);
      const int dh = min(max(ch[idx], 0), a.kernel - 1) - a.pad;
      const int dw = min(max(cw[idx], 0), a.kernel - 1) - a.pad;
      e = make_int4(c_ * HW + dh * a.W + dw, dh, dw, __float_as_int(wts ? wts[idx] : 1.0f));
    }
    taps[i] = e;
  }
  for (int i = tid; i < TG * NP; i += T) {
    const int t = i / NP, q = i - t * NP;
    const int n = min(n0 + t, a.N - 1);
    const float v = np[(int64_t)n * NP + q];
    if constexpr (!LUT) {
      par[i] = v;
    } else {
      constexpr int H2 = NP / 2;
      if constexpr (NODE == SLG_NODE_HYBRID) {
        par[i] = v;  // the values as they are (the forward's lookup)
      } else {
        // kept form: per group of corners its polynomial's coefficients
        // (lut_group_coeffs, as the forward keeps them)
        constexpr int LG = Nd::LG, GM = (1 << LG) - 1;
        float c[1 << LG];
#pragma unroll
        for (int u = 0; u <= GM; ++u) c[u] = np[(int64_t)n * NP + (q & ~GM) + u];
        lut_group_coeffs<LG>(c);
        float cq = c[0];
#pragma unroll
        for (int u = 1; u <= GM; ++u) cq = (q & GM) == u ? c[u] : cq;
        par[t * NPR + q] = cq;
      }
      // leaf differences D[j][qq] = s[p | bit j] - s[p] at the p with bit j set
#pragma unroll
      for (int j = 0; j < NLEAF; ++j) {
        if ((q >> j) & 1) {
          const int p0 = q & ~(1 << j);
          const int qq = ((p0 >> (j + 1)) << j) | (p0 & ((1 << j) - 1));
          raw[(t * NLEAF + j) * H2 + qq] = v - np[(int64_t)n * NP + p0];
        }
      }
    }
  }

  // this thread's tree and position slot in phase A
  const int ta = tid / a.TPT, ja = tid - ta * a.TPT;
  const bool tree_on = ta < TG && n0 + ta < a.N;
  float accw[NLEAF][KM];
#pragma unroll
  for (int l = 0; l < NLEAF; ++l)
#pragma unroll
    for (int k = 0; k < KM; ++k) accw[l][k] = 0.0f;
  float accn[NACC];
#pragma unroll
  for (int i = 0; i < NACC; ++i) accn[i] = 0.0f;

  const int b_begin = r * a.SPR, b_end = min(a.B, b_begin + a.SPR);
  for (int b = b_begin; b < b_end; ++b) {
    __syncthreads();  // the previous sample's reads are done (and the tables are staged)
    const float* xb = x + (int64_t)b * CHW;
    if constexpr (XS) {
      for (int i0 = tid; i0 < CHW; i0 += 4 * T) {  // four loads in flight per thread
        float t4[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) t4[u] = i0 + u * T < CHW ? xb[i0 + u * T] : 0.0f;
#pragma unroll
        for (int u = 0; u < 4; ++u)
          if (i0 + u * T < CHW) xs[i0 + u * T] = t4[u];
      }
      __syncthreads();
    }
    const float* xr = XS ? xs : xb;

    // ---- A: per (tree, routed output) ----
    if (tree_on) {
      const int n = n0 + ta;
      const int4* tp = taps + ta * NLEAF * K;
      const float* pr = par + ta * NPR;
      const float* rw = raw + ta * NLEAF * (NP / 2);
      for (int p = ja; p < P; p += a.TPT) {
        const int py = p / a.Wo, px = p - py * a.Wo;
        const int oy = POOL ? 2 * py : py, ox = POOL ? 2 * px : px;
        float v[NQ][NLEAF];
#pragma unroll
        for (int q = 0; q < NQ; ++q)
#pragma unroll
          for (int l = 0; l < NLEAF; ++l) v[q][l] = 0.0f;
#pragma unroll
        for (int k = 0; k < KM; ++k) {
          if (k == 0 || k < K) {  // K >= 1: step 0 always runs
#pragma unroll
            for (int l = 0; l < NLEAF; ++l) {
              const int4 e = tp[l * K + k];
#pragma unroll
              for (int q = 0; q < NQ; ++q) {
                const int y = oy + (q >> 1), xx = ox + (q & 1);
                const bool ok = (unsigned)(y + e.y) < (unsigned)a.H &&
                                (unsigned)(xx + e.z) < (unsigned)a.W;
                const float xv = ok ? xr[e.x + y * a.W + xx] : 0.0f;
                v[q][l] = fmaf(__int_as_float(e.w), xv, v[q][l]);
              }
            }
          }
        }
        int qs = 0;
        if constexpr (POOL) {
          float best = conv_tree_eval<NODE, NLEAF>(v[0], pr);
#pragma unroll
          for (int q = 1; q < 4; ++q) {
            const float val = conv_tree_eval<NODE, NLEAF>(v[q], pr);
            if (val > best) {
              best = val;
              qs = q;
            }
          }
        }
        float vs[NLEAF];
#pragma unroll
        for (int l = 0; l < NLEAF; ++l) {
          float sv = v[0][l];
#pragma unroll
          for (int q = 1; q < NQ; ++q) sv = qs == q ? v[q][l] : sv;
          vs[l] = sv;
        }
        const float gup = gy[((int64_t)b * a.N + n) * P + p];
        float gl[NLEAF];
        conv_tree_leaf_grad<NODE, NLEAF>(vs, pr, rw, gup, gl, accn);
        const int y = oy + (qs >> 1), xx = ox + (qs & 1);
#pragma unroll
        for (int l = 0; l < NLEAF; ++l) {
          if constexpr (LUT) vq[(ta * NLEAF + l) * P + p] = vs[l];
          gv[(ta * NLEAF + l) * P + p] = gl[l];
#pragma unroll
          for (int k = 0; k < KM; ++k) {
            if (k < K) {
              const int4 e = tp[l * K + k];
              const bool ok = (unsigned)(y + e.y) < (unsigned)a.H &&
                              (unsigned)(xx + e.z) < (unsigned)a.W;
              const float xv = ok ? xr[e.x + y * a.W + xx] : 0.0f;
              accw[l][k] = fmaf(gl[l], xv, accw[l][k]);
            }
          }
        }
        if constexpr (LUT) gq[ta * P + p] = gup;
        if constexpr (POOL) route[ta * P + p] = (unsigned char)qs;
      }
    }
    __syncthreads();

    // ---- B1: input gradient of every pixel from the group's taps ----
    // A wave takes 64 * ppl pixels of one channel (ppl = 1..PPL per lane) and
    // walks the channel's taps, bucketed by offset (dh, dw) where channels
    // hold enough taps: the output position, bounds and window slot are then
    // computed once per offset, and each tap costs two independent LDS reads
    // (route, leaf gradient) and an FMA. Taps are wave-uniform (scalar loads
    // from the table).
    if (gx_out != nullptr) {
      const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
      const int lane = tid & 63;
      constexpr int PPL = (LUT && NLEAF >= 5) ? 2 : 4;  // register budget of the big LUTs
      const int ppl = min(PPL, (HW + 63) >> 6);
      const int span = 64 * ppl;
      const int n_chunks = (HW + span - 1) / span;
      for (int ci = wave; ci < a.C * n_chunks; ci += (T >> 6)) {
        const int c = ci / n_chunks, chunk = ci - c * n_chunks;
        int hh[PPL], ww[PPL];
#pragma unroll
        for (int u = 0; u < PPL; ++u) {
          const int hw = chunk * span + u * 64 + lane;
          hh[u] = hw / a.W;
          ww[u] = hw - hh[u] * a.W;
        }
        float acc[PPL];
#pragma unroll
        for (int u = 0; u < PPL; ++u) acc[u] = 0.0f;
        const int kbase = (g * a.C + c) * a.KB;
        // KB == KK: one bucket per offset; KB == 1: the channel's taps in one
        // bucket, each with its own offset (for sparse channels)
        for (int kk = 0; kk < a.KB; ++kk) {
          const int j0 = tstart[kbase + kk], j1 = tstart[kbase + kk + 1];
          if (j0 == j1) continue;  // uniform
          int pp[PPL], qq[PPL];
          bool inb[PPL];
          auto place = [&](int dh, int dw) {
#pragma unroll
            for (int u = 0; u < PPL; ++u) {
              const int y = hh[u] - dh, xx = ww[u] - dw;  // the taps' output position
              if constexpr (POOL) {
                const int py = y >> 1, px = xx >> 1;
                inb[u] = u < ppl && y >= 0 && xx >= 0 && py < a.Ho && px < a.Wo;
                pp[u] = inb[u] ? py * a.Wo + px : 0;
                qq[u] = ((y & 1) << 1) | (xx & 1);
              } else {
                inb[u] = u < ppl && (unsigned)y < (unsigned)a.Ho && (unsigned)xx < (unsigned)a.Wo;
                pp[u] = inb[u] ? y * a.Wo + xx : 0;
                qq[u] = 0;
              }
            }
          };
          if (a.KB > 1) place(kk / a.kernel - a.pad, kk - (kk / a.kernel) * a.kernel - a.pad);
          for (int j = j0; j < j1; ++j) {
            const int4 en = tent[j];  // (leaf-gradient row base, route row base, offset, weight)
            if (a.KB == 1) place((en.z >> 8) - a.pad, (en.z & 255) - a.pad);
#pragma unroll
            for (int u = 0; u < PPL; ++u) {
              const float gg = gv[en.x + pp[u]];
              bool ok = inb[u];
              if constexpr (POOL) ok = ok && route[en.y + pp[u]] == (unsigned char)qq[u];
              acc[u] = fmaf(__int_as_float(en.w), ok ? gg : 0.0f, acc[u]);
            }
          }
        }
#pragma unroll
        for (int u = 0; u < PPL; ++u) {
          const int hw = chunk * span + u * 64 + lane;
          if (u < ppl && hw < HW) gx_out[((int64_t)g * a.B + b) * CHW + c * HW + hw] = acc[u];
        }
      }
    }

    // ---- B2 (LUT trees): corner gradients over the sample's outputs ----
    // corner = c1 + (c2 << H1): its weight is A(c1) * B(c2) with A the
    // product over the low H1 leaves (times the upstream gradient) and B
    // over the others. Item (tree, c1, position slot j) reads the leaf
    // values of positions p = j (mod J2) once and adds to all NC2 sums.
    if constexpr (LUT) {
      constexpr int H1 = NLEAF / 2, NC1 = 1 << H1, NC2 = 1 << (NLEAF - H1);
      const int J2 = a.J2, items = TG * NC1 * J2;
#pragma unroll
      for (int s2 = 0; s2 < NACC / NC2; ++s2) {
        const int it = tid + s2 * T;
        if (it < items) {
          const int t = it / (NC1 * J2), c1 = (it / J2) % NC1, j = it % J2;
          if (n0 + t < a.N) {
            for (int p = j; p < P; p += J2) {
              float lv[NLEAF];
#pragma unroll
              for (int l = 0; l < NLEAF; ++l) lv[l] = vq[(t * NLEAF + l) * P + p];
              float A = gq[t * P + p];
#pragma unroll
              for (int l = 0; l < H1; ++l) A *= ((c1 >> l) & 1) ? lv[l] : 1.0f - lv[l];
              float bw[NC2];
              bw[0] = A;
#pragma unroll
              for (int l = H1; l < NLEAF; ++l) {
                const int sz = 1 << (l - H1);
#pragma unroll
                for (int i = 0; i < sz; ++i) {
                  bw[i + sz] = bw[i] * lv[l];
                  bw[i] = bw[i] * (1.0f - lv[l]);
                }
              }
#pragma unroll
              for (int c2 = 0; c2 < NC2; ++c2) accn[s2 * NC2 + c2] += bw[c2];
            }
          }
        }
      }
    }
  }

  // ---- range sums, reduced over each tree's phase-A threads in LDS ----
  auto reduce_tree = [&](float val, float* dst, int stride, int col) {
    __syncthreads();
    red[tid] = tree_on ? val : 0.0f;
    __syncthreads();
    if (tid < TG && n0 + tid < a.N) {
      float sum = 0.0f;
      for (int j = 0; j < a.TPT; ++j) sum += red[tid * a.TPT + j];
      dst[(int64_t)(n0 + tid) * stride + col] = sum;
    }
  };
  float* pw = part_w + (int64_t)r * a.N * (NLEAF * K);
#pragma unroll
  for (int l = 0; l < NLEAF; ++l)
#pragma unroll
    for (int k = 0; k < KM; ++k)
      if (k < K) reduce_tree(accw[l][k], pw, NLEAF * K, l * K + k);
  float* pn = part_np + (int64_t)r * a.N * NP;
  if constexpr (!LUT) {
#pragma unroll
    for (int i = 0; i < NACC; ++i) reduce_tree(accn[i], pn, NP, i);
  } else {
    // corner sums reduced over the J2 position slots of each (tree, c1)
    constexpr int H1 = NLEAF / 2, NC1 = 1 << H1, NC2 = 1 << (NLEAF - H1);
    const int J2 = a.J2, items = TG * NC1 * J2;
#pragma unroll
    for (int s2 = 0; s2 < NACC / NC2; ++s2) {
      if (s2 * T >= items) break;  // uniform
#pragma unroll
      for (int c2 = 0; c2 < NC2; ++c2) {
        __syncthreads();
        red[tid] = accn[s2 * NC2 + c2];
        __syncthreads();
        const int grp = tid, first = s2 * T + grp * J2;  // item group (t, c1)
        if (grp * J2 < T && first < items) {
          const int t = first / (NC1 * J2), c1 = (first / J2) % NC1;
          if (n0 + t < a.N) {
            float sum = 0.0f;
            for (int j = 0; j < J2; ++j) sum += red[grp * J2 + j];
            pn[(int64_t)(n0 + t) * NP + c1 + (c2 << H1)] = sum;
          }
        }
      }
    }
  }
}

// gx[b][e] = sum over groups of part[g][b][e], groups ascending.
__global__ void __launch_bounds__(256) conv_bwd_sum_groups_kernel(const float* __restrict__ part,
                                                                  int NG, int64_t n,
                                                                  float* __restrict__ gx) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float s = 0.0f;
  for (int g = 0; g < NG; ++g) s += part[(int64_t)g * n + i];
  gx[i] = s;
}

// out[i] = sum over ranges r of part[r][i]: a workgroup takes 16 columns;
// its 16 thread rows sum the ranges r = row (mod 16) in ascending order, and
// the 16 row sums are added in row order (a fixed order on every call).
__global__ void __launch_bounds__(256) conv_bwd_sum_ranges_kernel(const float* __restrict__ part,
                                                                  int NR, int64_t n,
                                                                  float* __restrict__ out) {
  __shared__ float rs[16][17];
  const int col = threadIdx.x & 15, row = threadIdx.x >> 4;
  const int64_t i = (int64_t)blockIdx.x * 16 + col;
  float s = 0.0f;
  if (i < n)
    for (int r = row; r < NR; r += 16) s += part[(int64_t)r * n + i];
  rs[row][col] = s;
  __syncthreads();
  if (row == 0 && i < n) {
    float t = 0.0f;
    for (int q = 0; q < 16; ++q) t += rs[q][col];
    out[i] = t;
  }
}

// Table keys: tap (n, l, k) -> (group * C + channel) * KB + offset (KB =
// kernel^2, offset = ch * kernel + cw), or group * C + channel (KB = 1).
__global__ void __launch_bounds__(256) conv_bwd_keys_kernel(const int* __restrict__ cm,
                                                            const int* __restrict__ ch,
                                                            const int* __restrict__ cw, int R,
                                                            int LK, int TG, int C, int kernel,
                                                            int KB, int* __restrict__ keys) {
  const int r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= R) return;
  const int n = r / LK;
  const int c = min(max(cm[r], 0), C - 1);
  const int off = min(max(ch[r], 0), kernel - 1) * kernel + min(max(cw[r], 0), kernel - 1);
  keys[r] = KB == 1 ? (n / TG) * C + c : ((n / TG) * C + c) * KB + off;
}

// Table entries: sorted tap r -> (leaf-gradient row base (t * NLEAF + l) * P,
// route row base t * P, (ch << 8) | cw, weight), t = tree within its group.
__global__ void __launch_bounds__(256) conv_bwd_entries_kernel(const int* __restrict__ sorted,
                                                               int R, int NLEAF, int K, int TG,
                                                               int P, int kernel,
                                                               const int* __restrict__ ch,
                                                               const int* __restrict__ cw,
                                                               const float* __restrict__ wts,
                                                               int4* __restrict__ ent) {
  const int j = blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= R) return;
  const int r = sorted[j];
  const int n = r / (NLEAF * K), l = (r / K) % NLEAF;
  const int t = n % TG;
  const int off = (min(max(ch[r], 0), kernel - 1) << 8) | min(max(cw[r], 0), kernel - 1);
  ent[j] = make_int4((t * NLEAF + l) * P, t * P, off, __float_as_int(wts ? wts[r] : 1.0f));
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
struct ConvBwdPlan {
  bool XS;  // image staged in LDS
  int TG, TPT, threads, NG, NR, SPR, J2, KB;
  size_t lds;
  int64_t R;  // taps N * NLEAF * K
  // workspace (4-byte words): keys | table | entries (int4) | part_x | part_w | part_np
  int64_t keys_ints, table_ints, ent_ints, partx_floats, partw_floats, partn_floats;
  int64_t total() const {
    return keys_ints + table_ints + ent_ints + partx_floats + partw_floats + partn_floats;
  }
};

static int next_pow2(int v) {
  int p = 1;
  while (p < v) p <<= 1;
  return p;
}

template <int NODE, int NLEAF, bool POOL>
static bool conv_bwd_plan_t(int64_t B, int64_t C, int64_t H, int64_t W, int64_t N, int K,
                            int pad, int64_t Ho, int64_t Wo, ConvBwdPlan& p) {
  using Nd = ConvNode<NODE, NLEAF>;
  const int64_t CHW = C * H * W, P = Ho * Wo;
  const int64_t cap = std::min<int64_t>(device_lds_bytes(), 160 * 1024);
  if (CHW >= (1LL << 26) || P >= (1LL << 20) || P < 1 || C >= (1LL << 16)) return false;
  constexpr bool LUT = NODE != SLG_NODE_GATE16;
  constexpr int TMAX = conv_bwd_threads<NODE, NLEAF>();
  // largest tree group (a power of two) whose state fits LDS, with the image
  // staged or read through the caches
  auto best_tg = [&](bool xs, int& tpt, int& threads, size_t& lds) {
    for (int TG = std::min(TMAX, next_pow2((int)std::min<int64_t>(N, TMAX))); TG >= 1;
         TG >>= 1) {
      const ConvBwdLds L = conv_bwd_lds<NODE, NLEAF, POOL>(xs, (int)C, (int)CHW, TG, K, (int)P);
      const int TPT = std::min(TMAX / TG, next_pow2((int)P));
      const int th = (std::max(64, TG * TPT) + 63) & ~63;
      constexpr int H1 = NLEAF / 2, NC1 = 1 << H1, NC2 = 1 << (NLEAF - H1);
      const int slots = LUT ? (TG * NC1 + th - 1) / th : 0;  // (tree, c1) items per thread
      if ((int64_t)L.total * 4 <= cap && slots * NC2 <= kBwdNodeAcc) {
        tpt = TPT;
        threads = th;
        lds = (size_t)L.total * 4;
        return TG;
      }
    }
    return 0;
  };
  int tpt_s = 0, th_s = 0, tpt_g = 0, th_g = 0;
  size_t lds_s = 0, lds_g = 0;
  const int tg_s = best_tg(true, tpt_s, th_s, lds_s);
  const int tg_g = best_tg(false, tpt_g, th_g, lds_g);
  // stage the image unless that leaves room for fewer than 16 trees (or all
  // of them) while reading it through the caches fits more
  const bool xs = tg_s > 0 && (tg_s >= std::min<int64_t>(N, 16) || tg_g <= tg_s);
  p.XS = xs;
  p.TG = xs ? tg_s : tg_g;
  if (p.TG < 1) return false;
  p.TPT = xs ? tpt_s : tpt_g;
  p.threads = xs ? th_s : th_g;
  p.lds = xs ? lds_s : lds_g;
  p.NG = (int)cdiv(N, p.TG);
  p.J2 = 1;
  if (LUT) {  // position slots: fill the workgroup with (tree, c1, slot) items
    constexpr int NC1 = 1 << (NLEAF / 2);
    while (2 * p.J2 <= (int)P && (int64_t)p.TG * NC1 * 2 * p.J2 <= p.threads) p.J2 *= 2;
  }
  const int64_t per_cu = std::max<int64_t>(
      1, std::min<int64_t>(2048 / p.threads, (int64_t)(160 * 1024) / (int64_t)p.lds));
  const int64_t slots = per_cu * device_cus();
  int64_t NR = std::max<int64_t>(1, std::min<int64_t>(B, slots / p.NG));
  p.SPR = (int)cdiv(B, NR);
  p.NR = (int)cdiv(B, p.SPR);
  p.R = N * NLEAF * (int64_t)K;
  // bucket the taps by offset where a channel holds at least two per offset
  const int64_t kern = 2 * (int64_t)pad + 1;
  p.KB = (int64_t)p.TG * NLEAF * K >= 2 * kern * kern * C ? (int)(kern * kern) : 1;
  const int64_t nkeys = (int64_t)p.NG * C * p.KB;
  p.keys_ints = (p.R + 3) & ~3LL;
  p.table_ints = ref_table_ints(p.R, nkeys);
  p.ent_ints = 4 * p.R;
  p.partx_floats = p.NG > 1 ? (((int64_t)p.NG * B * CHW + 3) & ~3LL) : 0;
  p.partw_floats = ((int64_t)p.NR * N * NLEAF * K + 3) & ~3LL;
  p.partn_floats = ((int64_t)p.NR * N * Nd::NP + 3) & ~3LL;
  return true;
}

static int conv_bwd_leaves(int node, int depth, int arity) {
  if (node == SLG_NODE_GATE16) return (depth >= 1 && depth <= 3) ? (1 << depth) : -1;
  if (node == SLG_NODE_MULTILINEAR2 || node == SLG_NODE_HYBRID)
    return (depth == 1 && arity >= 2 && arity <= 6) ? arity : -1;
  return -1;
}

// Dispatch over (node, leaves, pool) with a callable taking the template
// arguments as integral constants.
template <typename F>
static int conv_bwd_dispatch(int node, int nleaf, bool pool, F&& f) {
#define SLG_CB(NODE_, NL_)                                                           \
  if (node == NODE_ && nleaf == NL_)                                                 \
    return pool ? f(std::integral_constant<int, NODE_>{}, std::integral_constant<int, NL_>{}, \
                    std::true_type{})                                                \
                : f(std::integral_constant<int, NODE_>{}, std::integral_constant<int, NL_>{}, \
                    std::false_type{});
  SLG_CB(SLG_NODE_GATE16, 2)
  SLG_CB(SLG_NODE_GATE16, 4)
  SLG_CB(SLG_NODE_GATE16, 8)
  SLG_CB(SLG_NODE_MULTILINEAR2, 2)
  SLG_CB(SLG_NODE_MULTILINEAR2, 3)
  SLG_CB(SLG_NODE_MULTILINEAR2, 4)
  SLG_CB(SLG_NODE_MULTILINEAR2, 5)
  SLG_CB(SLG_NODE_MULTILINEAR2, 6)
  SLG_CB(SLG_NODE_HYBRID, 2)
  SLG_CB(SLG_NODE_HYBRID, 3)
  SLG_CB(SLG_NODE_HYBRID, 4)
  SLG_CB(SLG_NODE_HYBRID, 5)
  SLG_CB(SLG_NODE_HYBRID, 6)
#undef SLG_CB
  set_error("conv_soft_bwd: unsupported leaves %d", nleaf);
  return SLG_E_UNSUPPORTED;
}

}  // namespace slg

using namespace slg;

extern "C" {

int64_t slg_conv_soft_bwd_workspace(int64_t B, int64_t C, int64_t H, int64_t W, int64_t N,
                                    int32_t node_kind, int32_t depth, int32_t arity, int32_t K,
                                    int32_t pad, int32_t pool) {
  const int nleaf = conv_bwd_leaves(node_kind, depth, arity);
  if (K < 1 || K > kBwdMaxK || B < 0 || C <= 0 || H <= 0 || W <= 0 || N <= 0 || pad < 0 ||
      pad > 4 || B >= (1LL << 31) || N >= (1LL << 20) || C >= (1LL << 20) || H >= 4096 ||
      W >= 4096)
    return -1;
  const int64_t Ho = pool ? H / 2 : H, Wo = pool ? W / 2 : W;
  if (Ho == 0 || Wo == 0) return 0;
  if (nleaf > 0 && N * nleaf * K < (1LL << 31)) {
    ConvBwdPlan p{};
    bool ok = false;
    conv_bwd_dispatch(node_kind, nleaf, pool != 0, [&](auto nd, auto nl, auto pl) {
      ok = conv_bwd_plan_t<decltype(nd)::value, decltype(nl)::value, decltype(pl)::value>(
          std::max<int64_t>(B, 1), C, H, W, N, K, pad, Ho, Wo, p);
      return 0;
    });
    if (ok) return p.total();
  }
  // trees the LDS kernel does not take (walsh, deeper LUT trees, images past
  // LDS): the generic kernels
  return conv_generic_bwd_workspace(B, C, H, W, N, node_kind, depth, arity, K, pad, pool != 0);
}

int slg_conv_soft_bwd(const float* x, int64_t B, int64_t C, int64_t H, int64_t W, int64_t N,
                      int32_t node_kind, int32_t depth, int32_t arity, int32_t K,
                      const float* node_param, const float* w, const int32_t* cm,
                      const int32_t* ch, const int32_t* cw, int32_t pad, int32_t pool,
                      const float* gy, float* gx, float* gw, float* gnp, float* workspace,
                      int64_t workspace_floats, slg_stream_t stream) {
  SLG_REQUIRE(node_param && cm && ch && cw && workspace && ((x && gy) || B == 0), SLG_E_ARG,
              "conv_soft_bwd: null pointer");
  SLG_REQUIRE(node_kind == SLG_NODE_GATE16 || node_kind == SLG_NODE_WALSH ||
                  node_kind == SLG_NODE_MULTILINEAR2 || node_kind == SLG_NODE_HYBRID,
              SLG_E_ARG, "conv_soft_bwd: node_kind %d", node_kind);
  const int nleaf = conv_bwd_leaves(node_kind, depth, arity);
  const bool generic = conv_generic_supported(node_kind, depth, arity);
  SLG_REQUIRE(nleaf > 0 || generic, SLG_E_UNSUPPORTED, "conv_soft_bwd: node %d depth %d / arity %d",
              node_kind, depth, arity);
  SLG_REQUIRE(K >= 1 && K <= kBwdMaxK, SLG_E_SHAPE, "conv_soft_bwd: K=%d outside 1..%d", K,
              kBwdMaxK);
  SLG_REQUIRE(B >= 0 && C > 0 && H > 0 && W > 0 && N > 0 && pad >= 0 && pad <= 4 &&
                  B < (1LL << 31) && N < (1LL << 20) && C < (1LL << 20) && H < 4096 &&
                  W < 4096 && N * std::max(nleaf, 1) * K < (1LL << 31),
              SLG_E_SHAPE, "conv_soft_bwd: bad sizes");
  const int kernel = 2 * pad + 1;  // 'same' convolution, stride 1 (models.py:222)
  const int64_t Ho = pool ? H / 2 : H, Wo = pool ? W / 2 : W;
  hipStream_t st = as_stream(stream);
  // the LDS kernel where its plan takes the shape, else the generic kernels
  // (the same choice as slg_conv_soft_bwd_workspace)
  bool lds_path = false;
  if (nleaf > 0) {
    ConvBwdPlan p0{};
    conv_bwd_dispatch(node_kind, nleaf, pool != 0, [&](auto nd, auto nl, auto pl) {
      lds_path = conv_bwd_plan_t<decltype(nd)::value, decltype(nl)::value, decltype(pl)::value>(
          std::max<int64_t>(B, 1), C, H, W, N, K, pad, std::max<int64_t>(Ho, 1),
          std::max<int64_t>(Wo, 1), p0);
      return 0;
    });
  }
  if (!lds_path) {
    SLG_REQUIRE(generic, SLG_E_UNSUPPORTED, "conv_soft_bwd: image of %lld floats does not fit LDS",
                (long long)(C * H * W));
    return conv_generic_bwd(x, B, C, H, W, N, node_kind, depth, arity, K, pad, pool != 0,
                            node_param, w, cm, ch, cw, gy, gx, gw, gnp, workspace,
                            workspace_floats, st);
  }
  const int64_t CHW = C * H * W;
  if (B == 0) {
    // no samples: zero weight / parameter gradients (a sum over no ranges)
    const int64_t NP = node_kind == SLG_NODE_GATE16 ? 4 * (nleaf - 1) : (1 << nleaf);
    const int64_t nw = N * nleaf * K;
    if (gw)
      hipLaunchKernelGGL(conv_bwd_sum_ranges_kernel, dim3((unsigned)cdiv(nw, 16)), dim3(256), 0,
                         st, workspace, 0, nw, gw);
    if (gnp)
      hipLaunchKernelGGL(conv_bwd_sum_ranges_kernel, dim3((unsigned)cdiv(N * NP, 16)),
                         dim3(256), 0, st, workspace, 0, N * NP, gnp);
    SLG_LAUNCH_CHECK("conv_soft_bwd zero");
    return 0;
  }
  SLG_REQUIRE(Ho > 0 && Wo > 0, SLG_E_SHAPE, "conv_soft_bwd: empty output map");
  return conv_bwd_dispatch(node_kind, nleaf, pool != 0, [&](auto nd, auto nl, auto pl) -> int {
    constexpr int NODE = decltype(nd)::value, NL = decltype(nl)::value;
    constexpr bool POOL = decltype(pl)::value;
    using Nd = ConvNode<NODE, NL>;
    ConvBwdPlan p{};
    SLG_REQUIRE((conv_bwd_plan_t<NODE, NL, POOL>(B, C, H, W, N, K, pad, Ho, Wo, p)),
                SLG_E_UNSUPPORTED, "conv_soft_bwd: image of %lld floats does not fit LDS",
                (long long)CHW);
    SLG_REQUIRE(workspace_floats >= p.total(), SLG_E_ARG,
                "conv_soft_bwd: workspace of %lld floats, %lld needed",
                (long long)workspace_floats, (long long)p.total());
    int* keys = reinterpret_cast<int*>(workspace);
    int* table = keys + p.keys_ints;
    int4* ent = reinterpret_cast<int4*>(table + p.table_ints);  // 16-byte aligned offsets
    float* partx = reinterpret_cast<float*>(ent) + p.ent_ints;
    float* partw = partx + p.partx_floats;
    float* partn = partw + p.partw_floats;
    const int R = (int)p.R;
    hipLaunchKernelGGL(conv_bwd_keys_kernel, dim3((unsigned)cdiv(R, 256)), dim3(256), 0, st, cm,
                       ch, cw, R, NL * K, p.TG, (int)C, kernel, p.KB, keys);
    RefTable tb{};
    int rc = build_ref_table(keys, R, (int64_t)p.NG * C * p.KB, table, st, &tb);
    if (rc) return rc;
    hipLaunchKernelGGL(conv_bwd_entries_kernel, dim3((unsigned)cdiv(R, 256)), dim3(256), 0, st,
                       tb.sorted, R, NL, K, p.TG, (int)(Ho * Wo), kernel, ch, cw, w, ent);
    SLG_LAUNCH_CHECK("conv_soft_bwd entries");

    ConvBwdArgs a{};
    a.C = (int)C; a.H = (int)H; a.W = (int)W; a.pad = pad; a.kernel = kernel;
    a.Ho = (int)Ho; a.Wo = (int)Wo; a.P = (int)(Ho * Wo);
    a.N = (int)N; a.K = K; a.TG = p.TG; a.TPT = p.TPT; a.NG = p.NG; a.SPR = p.SPR; a.B = (int)B;
    a.J2 = p.J2;
    a.KB = p.KB;
    // gx written directly when one group holds every tree; none when not wanted
    float* gxo = gx == nullptr ? nullptr : (p.NG > 1 ? partx : gx);
    auto kern = (K <= 4) ? (p.XS ? conv_soft_bwd_kernel<NODE, NL, POOL, 4, true>
                                 : conv_soft_bwd_kernel<NODE, NL, POOL, 4, false>)
                         : (p.XS ? conv_soft_bwd_kernel<NODE, NL, POOL, kBwdMaxK, true>
                                 : conv_soft_bwd_kernel<NODE, NL, POOL, kBwdMaxK, false>);
    if (p.lds > 65536) {
      hipError_t e = hipFuncSetAttribute((const void*)kern,
                                         hipFuncAttributeMaxDynamicSharedMemorySize, (int)p.lds);
      if (e != hipSuccess) {
        set_error("conv_soft_bwd: LDS %zu: %s", p.lds, hipGetErrorString(e));
        return (int)e;
      }
    }
    hipLaunchKernelGGL(kern, dim3((unsigned)(p.NG * p.NR)), dim3(p.threads), p.lds, st, x, gy, a,
                       node_param, w, cm, ch, cw, tb.start, ent, gxo, partw, partn);
    SLG_LAUNCH_CHECK("conv_soft_bwd");
    if (gx != nullptr && p.NG > 1) {
      const int64_t n = B * CHW;
      hipLaunchKernelGGL(conv_bwd_sum_groups_kernel, dim3((unsigned)cdiv(n, 256)), dim3(256), 0,
                         st, partx, p.NG, n, gx);
    }
    if (gw) {
      const int64_t n = N * NL * K;
      hipLaunchKernelGGL(conv_bwd_sum_ranges_kernel, dim3((unsigned)cdiv(n, 16)), dim3(256), 0,
                         st, partw, p.NR, n, gw);
    }
    if (gnp) {
      const int64_t n = N * Nd::NP;
      hipLaunchKernelGGL(conv_bwd_sum_ranges_kernel, dim3((unsigned)cdiv(n, 16)), dim3(256), 0,
                         st, partn, p.NR, n, gnp);
    }
    SLG_LAUNCH_CHECK("conv_soft_bwd sums");
    return 0;
  });
}

}  // extern "C"
