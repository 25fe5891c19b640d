// ConvLogicTree + OrPool for gfx950: soft (fp32) and hard (bit-packed), each
// with the 2x2 OR-pool fused so only the pooled map is written.
//
// Soft design: a workgroup owns S samples and every output channel. It
// stages the S input images in LDS with their zero padding, so every tap read
// is unconditional, and its waves take output channels in turn; the channel
// is wave-uniform, so tap offsets, leaf weights and node parameters sit in
// registers while the wave walks every 64-lane chunk of the workgroup's
// output positions. Two LDS layouts:
//  * row-major: plane (s, c) holds padded row r at r*RS with RS = W + pad
//    (the right padding of a row is the next row's left padding), plane size
//    (H+2pad)*RS + pad. Unpooled, lanes walk (row, column < RS) of each
//    sample and a chunk reads 64 consecutive floats; pooled, lanes walk
//    (pooled row, pooled column) and read each tap's 2x2 window as two pairs.
//  * phase-split (pooled, at most 16 taps per output): plane (s, c) is split
//    by (row parity, column parity) of the padded image into four sub-planes
//    of (Ho+pad) x (Wo+pad). Window position (dy, dx) of pooled output
//    (py, px) under tap (h, w) is sub-plane ((dy+h)&1, (dx+w)&1) at
//    (py + (dy+h)/2, px + (dx+w)/2), so lanes that walk (py, px < Wo+pad)
//    read consecutive floats of one sub-plane: four reads per tap at four
//    offsets held in registers.
//  * quad (pooled, phase-eligible taps, images small enough): four copies
//    of the padded image, shifted by (sy, sx) in {0,1}^2, stored as 2x2
//    blocks of four consecutive floats: block (by, bx) of copy (sy, sx)
//    holds padded pixels (2by+sy+dy, 2bx+sx+dx) as component 2dy+dx. The
//    2x2 window of pooled output (py, px) under tap (h, w) is then block
//    (py + h/2, px + w/2) of copy (h&1, w&1): one ds_read_b128 and one
//    address add per tap instead of four of each. Lanes walk exactly the
//    (py, px < Wo) outputs, so no lane idles on padding columns.
// Where lanes read consecutive floats, the sample stride is padded to equal
// the lanes per sample modulo 64, so that a chunk that spans two samples
// still hits 64 distinct LDS banks.
//
// Hard design: B-packed activations [C,H,W,nw] (64 samples per word).
// Threads walk (pooled position, word) with the word index fastest, so
// neighbouring lanes read neighbouring words of the same pixel; the output
// channel is the grid's y index, so leaf taps and truth tables are uniform.
#include <math.h>

#include "conv_tree.h"

namespace slg {

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ inline float sigmoidc(float z) { return 1.0f / (1.0f + expf(-z)); }

constexpr int kMaxK = 8;
constexpr int kQuadThreadsC = 1024;  // quad-layout workgroups (kQuadThreads)


// Layout choice and register budget of one kernel variant (host and device).
__host__ __device__ constexpr bool conv_phase_layout(bool pool, int nleaf, int km) {
  return pool && nleaf * km <= 16;
}

template <int NODE, int NLEAF, int KM, bool POOL>
struct ConvCfg {
  static constexpr bool PHASE = conv_phase_layout(POOL, NLEAF, KM);
  static constexpr int NW = PHASE ? 4 : 1;  // LDS offsets per tap
  static constexpr int NPR = ConvNode<NODE, NLEAF>::NPR;
  static constexpr int PARAMS = NLEAF * KM * (NW + 1) + NPR;  // per-channel registers
  static constexpr int REC = (PARAMS + 3) & ~3;               // record floats
  // eight waves per workgroup where the parameters leave room for two waves
  // per SIMD, else four
  static constexpr int THREADS = PARAMS <= 128 ? 512 : 256;
  // row-major records whose taps and weights fit the scalar file
  // (conv_params_record_split): those in scalar registers, the node
  // parameters in VGPRs, which leaves room for four waves per SIMD: such
  // kernels are built for up to 1024 threads and launched with 1024 where
  // one workgroup fills a CU's LDS, else 512 (two workgroups per CU)
  static constexpr bool SPLIT_OK = NW == 1 && 2 * NLEAF * KM <= 48 &&
                                   ConvNode<NODE, NLEAF>::NPR % 4 == 0;
  static constexpr int SPLIT_THREADS = 1024;
};

// Threads per workgroup of conv_soft_kernel (at most; see SPLIT_OK).
template <int NODE, int NLEAF, int KM, bool POOL, bool REC, bool QUAD>
__host__ __device__ constexpr int conv_soft_threads() {
  using Cfg = ConvCfg<NODE, NLEAF, KM, POOL>;
  return QUAD ? kQuadThreadsC : (REC && Cfg::SPLIT_OK ? Cfg::SPLIT_THREADS : Cfg::THREADS);
}

// LDS floats after the S staged samples: 64 dump slots, one per lane, that
// take the staged floats no window reads.
constexpr int kConvExtra = 64;

// LDS geometry of one launch (see the layouts above).
struct ConvGeom {
  int RS;     // row stride: W + pad (row-major) or Wo + pad (sub-plane rows)
  int PR;     // sub-plane rows Ho + pad (phase-split), 0 otherwise
  int PP;     // sub-plane size PR * RS (phase-split), 0 otherwise
  int plane;  // channel stride
  int SST;    // sample stride
  int LPS;    // lanes per sample
  int BH, BW; // quad: blocks per copy (rows, columns); pair: half-rows and
              // pairs per row of a copy; 0 otherwise
  int PAIR;   // 1: the pair layout
};

// One output channel's parameters in registers: LDS tap offsets, leaf
// weights and node parameters.
template <int NODE, int NLEAF, int KM, int NW>
struct ConvParams {
  int off[NLEAF][KM][NW];
  float wt[NLEAF][KM];
  float par[ConvNode<NODE, NLEAF>::NPR];
};

// LDS offset of tap (c, h, w) for window position q = 2*dy + dx (NW = 4,
// phase-split) or the tap itself (NW = 1, row-major).
__host__ __device__ inline int conv_tap_offset(const ConvGeom& g, int NW, int c, int h, int w,
                                               int q) {
  if (g.PAIR) {  // pair: the tap's pair in rows h (q = 0) and h + 1 (q = 1), in pair units
    const int Y = h + q;
    return q < 2 ? c * (g.plane / 2) + (w & 1) * 2 * g.BH * g.BW + (Y & 1) * g.BH * g.BW +
                       (Y >> 1) * g.BW + (w >> 1)
                 : 0;
  }
  if (g.BH > 0)  // quad: the tap's block in float4 units, in slot q = 0
    return q == 0 ? (c * g.plane) / 4 + ((h & 1) * 2 + (w & 1)) * g.BH * g.BW +
                        (h >> 1) * g.BW + (w >> 1)
                  : 0;
  if (NW == 1) return c * g.plane + h * g.RS + w;
  const int Y = (q >> 1) + h, X = (q & 1) + w;
  return c * g.plane + (Y & 1) * 2 * g.PP + (X & 1) * g.PP + (Y >> 1) * g.RS + (X >> 1);
}

// Channel parameters from separate arrays (slg_conv_soft_fwd). The index nv
// is a vector register (the same value in every lane), so the loads are
// vector loads and the parameters stay in VGPRs: there are too many for the
// scalar file, and an FMA takes one scalar operand on gfx9.
template <int NODE, int NLEAF, int KM, int NW>
__device__ inline void conv_params_arrays(ConvParams<NODE, NLEAF, KM, NW>& P, int nv, int K,
                                          int C, int kernel, const ConvGeom& g, const float* np,
                                          const float* wts, const int* cm, const int* ch,
                                          const int* cw) {
#pragma unroll
  for (int l = 0; l < NLEAF; ++l) {
#pragma unroll
    for (int k = 0; k < KM; ++k) {
      if (k < K) {
        const int idx = (nv * NLEAF + l) * K + k;
        const int c_ = min(max(cm[idx], 0), C - 1);
        const int h_ = min(max(ch[idx], 0), kernel - 1);
        const int w_ = min(max(cw[idx], 0), kernel - 1);
#pragma unroll
        for (int q = 0; q < NW; ++q) P.off[l][k][q] = conv_tap_offset(g, NW, c_, h_, w_, q);
        P.wt[l][k] = wts ? wts[idx] : 1.0f;
      } else {
#pragma unroll
        for (int q = 0; q < NW; ++q) P.off[l][k][q] = 0;
        P.wt[l][k] = 0.0f;
      }
    }
  }
  constexpr int NP = ConvNode<NODE, NLEAF>::NP;
  if constexpr (NODE != SLG_NODE_MULTILINEAR2) {  // gate16 coefficients, hybrid values
#pragma unroll
    for (int i = 0; i < NP; ++i) P.par[i] = np[(int64_t)nv * NP + i];
  } else {
    constexpr int LG = ConvNode<NODE, NLEAF>::LG;
#pragma unroll
    for (int g = 0; g < (NP >> LG); ++g) {
      float c[1 << LG];
#pragma unroll
      for (int i = 0; i < (1 << LG); ++i) c[i] = np[(int64_t)nv * NP + (g << LG) + i];
      lut_group_coeffs<LG>(c);
#pragma unroll
      for (int i = 0; i < (1 << LG); ++i) P.par[(g << LG) + i] = c[i];
    }
  }
}

// Channel parameters from a record (slg_conv_soft_records): R floats laid
// out as ConvParams (offsets, weights, node parameters), read with 16-byte
// vector loads.
template <int NODE, int NLEAF, int KM, int NW, int R>
__device__ inline void conv_params_record(ConvParams<NODE, NLEAF, KM, NW>& P, const float* rec,
                                          int nv) {
  // the floats in use: records of phase-eligible trees keep room for four
  // offsets per tap, the pair layout fills two
  constexpr int USED = (NLEAF * KM * (NW + 1) + ConvNode<NODE, NLEAF>::NPR + 3) & ~3;
  static_assert(USED <= R, "the record holds the parameters");
  float v[USED];
  const float4* r4 = reinterpret_cast<const float4*>(rec + (int64_t)nv * R);
#pragma unroll
  for (int q = 0; q < USED / 4; ++q) {
    const float4 t = r4[q];
    v[4 * q] = t.x; v[4 * q + 1] = t.y; v[4 * q + 2] = t.z; v[4 * q + 3] = t.w;
  }
  constexpr int LK = NLEAF * KM;
#pragma unroll
  for (int l = 0; l < NLEAF; ++l)
#pragma unroll
    for (int k = 0; k < KM; ++k) {
#pragma unroll
      for (int q = 0; q < NW; ++q) P.off[l][k][q] = __float_as_int(v[(l * KM + k) * NW + q]);
      P.wt[l][k] = v[LK * NW + l * KM + k];
    }
#pragma unroll
  for (int i = 0; i < ConvNode<NODE, NLEAF>::NPR; ++i) P.par[i] = v[LK * (NW + 1) + i];
}

// Channel parameters from a record with the taps and weights read at the
// wave-uniform channel n (scalar loads: scalar registers, no vector memory
// traffic per lane) and the node parameters at the same channel held in a
// vector register nv (vector loads: VGPRs, since an FMA takes one scalar
// operand and the tree's FMAs would take two).
template <int NODE, int NLEAF, int KM, int NW, int R>
__device__ inline void conv_params_record_split(ConvParams<NODE, NLEAF, KM, NW>& P,
                                                const float* rec, int n, int nv) {
  constexpr int LK = NLEAF * KM;
  constexpr int NPR = ConvNode<NODE, NLEAF>::NPR;
  static_assert((LK * (NW + 1)) % 4 == 0 && NPR % 4 == 0, "16-byte record parts");
  float v[LK * (NW + 1)];
  const float4* r4 = reinterpret_cast<const float4*>(rec + (int64_t)n * R);
#pragma unroll
  for (int q = 0; q < LK * (NW + 1) / 4; ++q) {
    const float4 t = r4[q];
    v[4 * q] = t.x; v[4 * q + 1] = t.y; v[4 * q + 2] = t.z; v[4 * q + 3] = t.w;
  }
#pragma unroll
  for (int l = 0; l < NLEAF; ++l)
#pragma unroll
    for (int k = 0; k < KM; ++k) {
#pragma unroll
      for (int q = 0; q < NW; ++q) P.off[l][k][q] = __float_as_int(v[(l * KM + k) * NW + q]);
      P.wt[l][k] = v[LK * NW + l * KM + k];
    }
  const float4* p4 = reinterpret_cast<const float4*>(rec + (int64_t)nv * R + LK * (NW + 1));
#pragma unroll
  for (int q = 0; q < NPR / 4; ++q) {
    const float4 t = p4[q];
    P.par[4 * q] = t.x; P.par[4 * q + 1] = t.y; P.par[4 * q + 2] = t.z; P.par[4 * q + 3] = t.w;
  }
}

// Channel parameters from a quad record: the records of phase-eligible
// trees keep their phase size R, but a quad-layout record packs one offset
// per tap (float4 units), then the weights, then the node parameters, so
// only 2*L*KM + NPR floats are read.
template <int NODE, int NLEAF, int KM, int NW, int R>
__device__ inline void conv_params_record_quad(ConvParams<NODE, NLEAF, KM, NW>& P, const float* rec,
                                               int nv) {
  constexpr int LK = NLEAF * KM;
  constexpr int NPR = ConvNode<NODE, NLEAF>::NPR;
  constexpr int USED = (2 * LK + NPR + 3) & ~3;
  static_assert(USED <= R, "quad records fit the phase record size");
  float v[USED];
  const float4* r4 = reinterpret_cast<const float4*>(rec + (int64_t)nv * R);
#pragma unroll
  for (int q = 0; q < USED / 4; ++q) {
    const float4 t = r4[q];
    v[4 * q] = t.x; v[4 * q + 1] = t.y; v[4 * q + 2] = t.z; v[4 * q + 3] = t.w;
  }
#pragma unroll
  for (int l = 0; l < NLEAF; ++l)
#pragma unroll
    for (int k = 0; k < KM; ++k) {
      P.off[l][k][0] = __float_as_int(v[l * KM + k]);
#pragma unroll
      for (int q = 1; q < NW; ++q) P.off[l][k][q] = 0;
      P.wt[l][k] = v[LK + l * KM + k];
    }
#pragma unroll
  for (int i = 0; i < NPR; ++i) P.par[i] = v[2 * LK + i];
}

// Quad-layout workgroups: 16 waves (the layout takes most of the LDS, so one
// workgroup per CU; its per-tap state is one offset, which leaves room in
// 128 VGPRs).
constexpr int kQuadThreads = kQuadThreadsC;

// SWAP (pooled row-major layout only): lanes of odd pooled columns take the
// window's two columns in the other order, so that each of the four reads
// of a tap hits even and odd LDS banks alike (in index order every lane of
// a read is on a bank of one parity). Each lane keeps its order for every
// leaf and tap, and the pooled output is the maximum over the four
// positions, so the result is the same.
//
// RSC (pooled row-major layout only): the row stride g.RS as a compile-time
// constant (0: read from g), so that a window's second row is an immediate
// offset of the first row's LDS read and each tap takes one address add (two
// with SWAP) instead of two (four).
template <int NODE, int NLEAF, bool POOL, int KM, bool REC, bool QUAD, bool SWAP = false,
          int RSC = 0>
__global__ void __launch_bounds__((conv_soft_threads<NODE, NLEAF, KM, POOL, REC, QUAD>()))
conv_soft_kernel(const float* __restrict__ x, int B, int C, int H, int W, int N, int K, int kernel,
                 int pad, ConvGeom g, const float* __restrict__ np, const float* __restrict__ wts,
                 const int* __restrict__ cm, const int* __restrict__ ch, const int* __restrict__ cw,
                 const float* __restrict__ rec, int S, float* __restrict__ out, int Ho, int Wo) {
  using Cfg = ConvCfg<NODE, NLEAF, KM, POOL>;
  constexpr bool PHASE = Cfg::PHASE && !QUAD;
  constexpr int NW = Cfg::NW;
  static_assert(!QUAD || Cfg::PHASE, "the quad layout keeps the phase records");
  extern __shared__ float lds[];
  const int b0 = blockIdx.x * S;
  const int ns = min(S, B - b0);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nwaves = blockDim.x >> 6;

  // Stage the images: clear the region, then scatter the ns*C*H*W input
  // floats (contiguous in memory) to their padded positions. Every thread
  // issues kStage loads before it writes them, so that the copy is not one
  // load latency per row.
  if constexpr (QUAD) {  // the quad region is a whole number of 16-byte blocks
    for (int i = threadIdx.x; i < ns * g.SST / 4; i += blockDim.x)
      reinterpret_cast<f32x4*>(lds)[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  } else {
    for (int i = threadIdx.x; i < ns * g.SST; i += blockDim.x) lds[i] = 0.0f;
  }
  __syncthreads();
  {
    // Thread t takes elements e = t + i*T (T = blockDim.x) and steps its
    // (sample, channel, row, column) by T's decomposition with carries, so
    // that no element needs a division.
    const int HW = H * W;
    const int total = ns * C * HW;
    const int T = blockDim.x;
    const __amdgpu_buffer_rsrc_t src = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(x + (int64_t)b0 * C * HW), (short)0, total * 4, kBufferWord3);
    const int tx = T % W, ty = (T / W) % H, tc = (T / HW) % C, ts = T / (HW * C);
    int px = threadIdx.x % W, py = (threadIdx.x / W) % H, pc = (threadIdx.x / HW) % C,
        ps = threadIdx.x / (HW * C);
    const int dump = S * g.SST + lane;
    constexpr int kStage = 8;
    for (int e0 = threadIdx.x; e0 < total; e0 += kStage * T) {
      float v[kStage];
#pragma unroll
      for (int u = 0; u < kStage; ++u)  // offsets past the images read 0
        v[u] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(src, (e0 + u * T) * 4, 0, 0));
#pragma unroll
      for (int u = 0; u < kStage; ++u) {
        int at;
        bool keep = ps < ns;
        if constexpr (QUAD) {
          // one float to each copy whose blocks hold the pixel
          const int Y = py + pad, X = px + pad;
          const int sb = __umul24(ps, g.SST) + __umul24(pc, g.plane);
#pragma unroll
          for (int sy = 0; sy < 2; ++sy)
#pragma unroll
            for (int sx = 0; sx < 2; ++sx) {
              const int by = (Y - sy) >> 1, bx = (X - sx) >> 1;
              const bool in = keep && Y >= sy && X >= sx && by < g.BH && bx < g.BW;
              const int a = sb + 4 * (__umul24(sy * 2 + sx, g.BH * g.BW) + __umul24(by, g.BW) + bx) +
                            ((Y - sy) & 1) * 2 + ((X - sx) & 1);
              lds[in ? a : dump] = v[u];
            }
          at = 0;
          keep = false;  // written above; the common store below goes to the dump slot
        } else if constexpr (PHASE) {
          const int Y = py + pad, X = px + pad;
          keep = keep && (Y >> 1) < g.PR && (X >> 1) < g.RS;  // rows/columns no window reads
          at = ((Y & 1) ? 2 * g.PP : 0) + ((X & 1) ? g.PP : 0) + __umul24(Y >> 1, g.RS) + (X >> 1);
        } else {
          at = __umul24(py + pad, g.RS) + pad + px;
        }
        // elements that are not kept go to this lane's dump slot
        if constexpr (!QUAD) lds[keep ? __umul24(ps, g.SST) + __umul24(pc, g.plane) + at : dump] = v[u];
        px += tx;
        const int cy = px >= W;
        px -= cy ? W : 0;
        py += ty + cy;
        const int cc = py >= H;
        py -= cc ? H : 0;
        pc += tc + cc;
        const int cs = pc >= C;
        pc -= cs ? C : 0;
        ps += ts + cs;
      }
    }
  }
  __syncthreads();

  const int P = Ho * Wo;
  const int nchunks = (ns * g.LPS + 63) / 64;
  // Quad layout: a wave takes four channels at once, one per 16-lane LDS
  // conflict group of ds_read_b128 (lanes 0-3, 12-15, 20-27 / 4-11, 16-19,
  // 28-31, and the same in the upper half), each group walking 16
  // consecutive outputs; the chunks of 16 leave fewer idle lanes at the end
  // of a sample than chunks of 64. Otherwise one channel per wave.
  constexpr int CPW = QUAD ? 4 : 1;       // channels per wave
  constexpr int LPC = 64 / CPW;           // lanes per channel
  const int cslot = QUAD ? 2 * (lane >> 5) + (__popc((lane >> 2) & 7) & 1) : 0;
  const int rank = QUAD ? (((lane & 31) >> 3) * 4 + (lane & 3)) : lane;
  const int nchunks_c = QUAD ? (ns * g.LPS + LPC - 1) / LPC : nchunks;
  // row-major records whose taps and weights fit the scalar file: those in
  // scalar registers, the node parameters in VGPRs
  constexpr bool SPLIT = REC && !QUAD && Cfg::SPLIT_OK;
  auto load = [&](ConvParams<NODE, NLEAF, KM, NW>& Pr, int n) {
    int nv;  // the channel in a vector register: vector loads, VGPR parameters
    if constexpr (QUAD) nv = min(n + cslot, N - 1);
    else asm volatile("v_mov_b32 %0, %1" : "=v"(nv) : "s"(n));
    if constexpr (REC && QUAD) conv_params_record_quad<NODE, NLEAF, KM, NW, Cfg::REC>(Pr, rec, nv);
    else if constexpr (SPLIT) conv_params_record_split<NODE, NLEAF, KM, NW, Cfg::REC>(Pr, rec, n, nv);
    else if constexpr (REC) conv_params_record<NODE, NLEAF, KM, NW, Cfg::REC>(Pr, rec, nv);
    else conv_params_arrays<NODE, NLEAF, KM, NW>(Pr, nv, K, C, kernel, g, np, wts, cm, ch, cw);
  };

  ConvParams<NODE, NLEAF, KM, NW> Pc;
  if (wave * CPW < N) load(Pc, wave * CPW);
  // the lane's output (sample, row, column) advances by LPC outputs per
  // chunk, carried incrementally (no division per chunk): pooled row-major
  // lanes walk rows of Wo columns, the others rows of RS columns (those >= Wo
  // idle), LPS lanes per sample; the quad layout takes one sample
  constexpr bool LINEAR = PHASE || !POOL;
  const int WW = QUAD ? Wo : (LINEAR ? g.RS : Wo);
  const int HH = QUAD ? (1 << 30) : g.LPS / WW;
  const int l_s = QUAD ? 0 : rank / g.LPS, l_rem = QUAD ? rank : rank - l_s * g.LPS;
  const int l_row = l_rem / WW, l_col = l_rem - (l_rem / WW) * WW;
  const int d_s = QUAD ? 0 : LPC / g.LPS, d_rem = QUAD ? LPC : LPC - d_s * g.LPS;
  const int d_row = d_rem / WW, d_col = d_rem - d_row * WW;
  for (int nb = wave * CPW; nb < N; nb += nwaves * CPW) {
    const int n = nb + cslot;  // this lane's channel
    float* out_n = out + ((int64_t)b0 * N + min(n, N - 1)) * P;  // quad: sample b0
    int q_s = l_s, q_row = l_row, q_col = l_col;
    for (int chunk = 0; chunk < nchunks_c; ++chunk) {
      const int q = chunk * LPC + rank;
      // idle lanes (past the workgroup's samples) read at the start of the
      // staged region
      const int s = q_s, row = q_row, col = q_col;
      bool active = (QUAD ? q < ns * g.LPS : s < ns) && n < N;
      q_col += d_col;
      if (q_col >= WW) { q_col -= WW; ++q_row; }
      q_row += d_row;
      if (q_row >= HH) { q_row -= HH; ++q_s; }
      q_s += d_s;
      active = active && col < Wo;
      const int p = (int)__umul24(row, Wo) + col;
      const int bofs = QUAD ? 4 * ((int)__umul24(row, g.BW) + col)
                            : (LINEAR ? q - (int)__umul24(s, g.LPS)
                                      : 2 * (int)__umul24(row, g.RS) + 2 * col);
      const float* base = lds + (active ? __umul24(s, g.SST) + bofs : 0);
      static_assert(!SWAP || (POOL && !PHASE && !QUAD), "SWAP is for the pooled row-major layout");
      static_assert(RSC == 0 || (POOL && !PHASE && !QUAD), "RSC is for the pooled row-major layout");
      const int RS = RSC > 0 ? RSC : g.RS;
      const int sw = SWAP ? (col & 1) : 0;
      const float* bq0 = base + sw;
      const float* bq1 = base + 1 - sw;

      // Tap k of every leaf per step: the guard k < K is uniform, and one
      // step issues all NLEAF * NQ LDS reads before its first wait. With
      // every candidate slot in use (K == KM) the steps are pipelined: the
      // reads of step k+1 go out before the FMAs of step k.
      constexpr int NQ = POOL ? 4 : 1;
      float v[NQ][NLEAF];
#pragma unroll
      for (int l = 0; l < NLEAF; ++l)
#pragma unroll
        for (int qq = 0; qq < NQ; ++qq) v[qq][l] = 0.0f;
      auto read_step = [&](int k, float (&t)[NLEAF][NQ]) {
#pragma unroll
        for (int l = 0; l < NLEAF; ++l) {
          if constexpr (QUAD) {
            const f32x4 w4 = reinterpret_cast<const f32x4*>(base)[Pc.off[l][k][0]];
#pragma unroll
            for (int qq = 0; qq < 4; ++qq) t[l][qq] = w4[qq];
          } else if constexpr (PHASE) {
#pragma unroll
            for (int qq = 0; qq < 4; ++qq) t[l][qq] = base[Pc.off[l][k][qq]];
          } else if constexpr (SWAP) {
            const int o = Pc.off[l][k][0];
            const float* ta = bq0 + o;
            const float* tb = bq1 + o;
            t[l][0] = ta[0];
            t[l][1] = tb[0];
            t[l][2] = ta[RS];
            t[l][3] = tb[RS];
          } else {
            const float* t0 = base + Pc.off[l][k][0];
            t[l][0] = t0[0];
            if constexpr (POOL) {
              t[l][1] = t0[1];
              t[l][2] = t0[RS];
              t[l][3] = t0[RS + 1];
            }
          }
        }
      };
      auto fma_step = [&](int k, const float (&t)[NLEAF][NQ]) {
#pragma unroll
        for (int l = 0; l < NLEAF; ++l)
#pragma unroll
          for (int qq = 0; qq < NQ; ++qq) v[qq][l] = fmaf(Pc.wt[l][k], t[l][qq], v[qq][l]);
      };
      if (QUAD && K == KM) {
        float t[2][NLEAF][NQ];
        read_step(0, t[0]);
#pragma unroll
        for (int k = 0; k < KM; ++k) {
          if (k + 1 < KM) read_step(k + 1, t[(k + 1) & 1]);
          fma_step(k, t[k & 1]);
        }
      } else {
#pragma unroll
        for (int k = 0; k < KM; ++k) {
          if (k == 0 || k < K) {  // K >= 1: step 0 always runs
            float t[NLEAF][NQ];
            read_step(k, t);
            __builtin_amdgcn_sched_barrier(0);  // all reads of the step, then the FMAs
            fma_step(k, t);
          }
        }
      }
      float best = -INFINITY;
#pragma unroll
      for (int qq = 0; qq < NQ; ++qq) {
        const float val = conv_tree_eval<NODE, NLEAF>(v[qq], Pc.par);
        best = fmaxf(best, val);
      }
      if constexpr (QUAD) {
        if (active) out_n[p] = best;
      } else {
        if (active) out[((int64_t)(b0 + s) * N + n) * P + p] = best;
      }
    }
    if (nb + nwaves * CPW < N) load(Pc, nb + nwaves * CPW);
  }
}

// Quad layout, persistent: workgroup w takes samples w, w + grid, ... and
// keeps one staged sample in LDS. The padding blocks are cleared once (the
// staging writes only image pixels); the next sample's C*H*W floats ride in
// registers (at most kQuadRegs per thread) while this sample computes, so
// the input's HBM latency overlaps the compute; after the last read of the
// sample they are scattered into the four copies. The arithmetic per output
// is conv_soft_kernel's, in the same order.
constexpr int kQuadRegs = 7;

template <int NODE, int NLEAF, int KM, bool REC>
__global__ void __launch_bounds__(kQuadThreads)
conv_soft_quad_kernel(const float* __restrict__ x, int B, int C, int H, int W, int N, int K,
                      int kernel, int pad, ConvGeom g, const float* __restrict__ np,
                      const float* __restrict__ wts, const int* __restrict__ cm,
                      const int* __restrict__ ch, const int* __restrict__ cw,
                      const float* __restrict__ rec, float* __restrict__ out, int Ho, int Wo) {
  using Cfg = ConvCfg<NODE, NLEAF, KM, true>;
  static_assert(Cfg::PHASE, "the quad layout keeps the phase records");
  constexpr int NW = Cfg::NW;
  constexpr int CPW = 4, LPC = 16;
  extern __shared__ float lds[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nwaves = blockDim.x >> 6;
  const int T = blockDim.x;
  const int HW = H * W, total = C * HW;
  const int P = Ho * Wo;

  for (int i = threadIdx.x; i < g.SST / 4 + kConvExtra / 4; i += T)
    reinterpret_cast<f32x4*>(lds)[i] = f32x4{0.f, 0.f, 0.f, 0.f};

  // this thread's elements e = tid + u*T of a sample
  float pf[kQuadRegs];
  auto issue = [&](int b) {
    const __amdgpu_buffer_rsrc_t src = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(x + (int64_t)b * total), (short)0, total * 4, kBufferWord3);
#pragma unroll
    for (int u = 0; u < kQuadRegs; ++u)  // offsets past the image read 0
      pf[u] = __uint_as_float(
          __builtin_amdgcn_raw_buffer_load_b32(src, (threadIdx.x + u * T) * 4, 0, 0));
  };
  const int dump = g.SST + lane;
  auto scatter = [&] {
    const int tx = T % W, ty = (T / W) % H, tc = T / HW;
    int px = threadIdx.x % W, py = (threadIdx.x / W) % H, pc = threadIdx.x / HW;
#pragma unroll
    for (int u = 0; u < kQuadRegs; ++u) {
      const int Y = py + pad, X = px + pad;
      const int sb = __umul24(pc, g.plane);
      const bool keep = pc < C;
#pragma unroll
      for (int sy = 0; sy < 2; ++sy)
#pragma unroll
        for (int sx = 0; sx < 2; ++sx) {
          const int by = (Y - sy) >> 1, bx = (X - sx) >> 1;
          const bool in = keep && Y >= sy && X >= sx && by < g.BH && bx < g.BW;
          const int a = sb + 4 * (__umul24(sy * 2 + sx, g.BH * g.BW) + __umul24(by, g.BW) + bx) +
                        ((Y - sy) & 1) * 2 + ((X - sx) & 1);
          lds[in ? a : dump] = pf[u];
        }
      px += tx;
      const int cy = px >= W;
      px -= cy ? W : 0;
      py += ty + cy;
      const int cc = py >= H;
      py -= cc ? H : 0;
      pc += tc + cc;
    }
  };

  // four channels per wave on the ds_read_b128 conflict groups (see
  // conv_soft_kernel's quad path)
  const int cslot = 2 * (lane >> 5) + (__popc((lane >> 2) & 7) & 1);
  const int rank = ((lane & 31) >> 3) * 4 + (lane & 3);
  // lanes walk rows of WW = g.RS columns: Wo, or BW (the copies' blocks per
  // row) where runs of 16 consecutive outputs would put two blocks of one
  // bank class in a conflict group; lanes on a padding column read their
  // own block (in bounds: at most one block past a copy) and store nothing
  const int WW = g.RS;
  const int nchunks = (Ho * WW + LPC - 1) / LPC;
  const int d_row = LPC / WW, d_col = LPC - d_row * WW;
  auto load = [&](ConvParams<NODE, NLEAF, KM, NW>& Pr, int nb) {
    const int nv = min(nb + cslot, N - 1);
    if constexpr (REC) conv_params_record_quad<NODE, NLEAF, KM, NW, Cfg::REC>(Pr, rec, nv);
    else conv_params_arrays<NODE, NLEAF, KM, NW>(Pr, nv, K, C, kernel, g, np, wts, cm, ch, cw);
  };
  // with one channel group per wave the parameters stay for every sample
  const bool one_group = N <= nwaves * CPW;
  ConvParams<NODE, NLEAF, KM, NW> Pc;
  if (one_group && wave * CPW < N) load(Pc, wave * CPW);

  if (blockIdx.x < (unsigned)B) issue(blockIdx.x);
  __syncthreads();  // cleared before the first scatter
  for (int b = blockIdx.x; b < B; b += gridDim.x) {
    scatter();
    __syncthreads();
    if (b + (int)gridDim.x < B) issue(b + gridDim.x);
    for (int nb = wave * CPW; nb < N; nb += nwaves * CPW) {
      if (!one_group) load(Pc, nb);
      const int n = nb + cslot;
      float* out_n = out + ((int64_t)b * N + min(n, N - 1)) * P;
      int q_row = rank / WW, q_col = rank - (rank / WW) * WW;
      for (int chunk = 0; chunk < nchunks; ++chunk) {
        const int q = chunk * LPC + rank;
        const bool inside = q < Ho * WW;
        const int row = q_row, col = q_col;
        const bool active = inside && col < Wo && n < N;
        q_col += d_col;
        q_row += d_row;
        if (q_col >= WW) { q_col -= WW; ++q_row; }
        const f32x4* base =
            reinterpret_cast<const f32x4*>(lds) + (inside ? (int)__umul24(row, g.BW) + col : 0);
        float v[4][NLEAF];
#pragma unroll
        for (int l = 0; l < NLEAF; ++l)
#pragma unroll
          for (int qq = 0; qq < 4; ++qq) v[qq][l] = 0.0f;
#pragma unroll
        for (int k = 0; k < KM; ++k) {
          if (k == 0 || k < K) {  // K >= 1: step 0 always runs
            f32x4 t[NLEAF];
#pragma unroll
            for (int l = 0; l < NLEAF; ++l) t[l] = base[Pc.off[l][k][0]];
#pragma unroll
            for (int l = 0; l < NLEAF; ++l)
#pragma unroll
              for (int qq = 0; qq < 4; ++qq) v[qq][l] = fmaf(Pc.wt[l][k], t[l][qq], v[qq][l]);
          }
        }
        float best = -INFINITY;
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) best = fmaxf(best, conv_tree_eval<NODE, NLEAF>(v[qq], Pc.par));
        if (active) out_n[(int)__umul24(row, Wo) + col] = best;
      }
    }
    __syncthreads();  // every read of this sample precedes the next scatter
  }
}

// Pair layout (pooled, phase-eligible taps, images whose four quad copies
// do not fit one workgroup's LDS but two copies do): copy sx in {0, 1} of
// the padded image holds, by row parity ry and half-row iy, BW pairs of
// floats per row, pair j being padded pixels (2iy+ry, 2j+sx) and
// (2iy+ry, 2j+sx+1). The 2x2 window of pooled output (py, px) under tap
// (h, w) is pair px + w/2 of copy w&1 in rows 2py+h and 2py+h+1: two
// ds_read_b64 at two per-tap offsets (pair units) from the lane's pair
// q = py*BW + px. Lanes walk (py, px < BW), one channel per chunk, so the
// 32 lanes of a b64 conflict group read 32 consecutive pairs of one row
// parity. Persistent like conv_soft_quad_kernel (one staged sample per
// workgroup, the next one's C*H*W floats in registers); a wave takes one
// channel at a time with its parameters in scalar registers (uniform loads
// through the scalar cache), so that a channel's parameters cost no vector
// memory or LDS traffic per sample. The arithmetic per output is
// conv_soft_kernel's, in the same order.
constexpr int kPairRegs = 13;
constexpr int kPairMaxChunks = 2;

template <int NODE, int NLEAF, int KM, bool REC>
__global__ void __launch_bounds__(kQuadThreads)
conv_soft_pair_kernel(const float* __restrict__ x, int B, int C, int H, int W, int N, int K,
                      int kernel, int pad, ConvGeom g, const float* __restrict__ np,
                      const float* __restrict__ wts, const int* __restrict__ cm,
                      const int* __restrict__ ch, const int* __restrict__ cw,
                      const float* __restrict__ rec, float* __restrict__ out, int Ho, int Wo) {
  using Cfg = ConvCfg<NODE, NLEAF, KM, true>;
  static_assert(Cfg::PHASE, "the pair layout keeps the phase records");
  constexpr int NW = 2;
  extern __shared__ float lds[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nwaves = blockDim.x >> 6;
  const int T = blockDim.x;
  const int HW = H * W, total = C * HW;
  const int P = Ho * Wo;
  const int BH = g.BH, BW = g.BW;
  const int HALF = 2 * BH * BW;  // floats of one row-parity plane of a copy

  for (int i = threadIdx.x; i < (g.SST + kConvExtra) / 4; i += T)
    reinterpret_cast<f32x4*>(lds)[i] = f32x4{0.f, 0.f, 0.f, 0.f};

  // this thread's elements e = tid + u*T of a sample
  float pf[kPairRegs];
  auto issue = [&](int b) {
    const __amdgpu_buffer_rsrc_t src = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(x + (int64_t)b * total), (short)0, total * 4, kBufferWord3);
#pragma unroll
    for (int u = 0; u < kPairRegs; ++u)  // offsets past the image read 0
      pf[u] = __uint_as_float(
          __builtin_amdgcn_raw_buffer_load_b32(src, (threadIdx.x + u * T) * 4, 0, 0));
  };
  const int dump = g.SST + lane;
  auto scatter = [&] {
    const int tx = T % W, ty = (T / W) % H, tc = T / HW;
    int px = threadIdx.x % W, py = (threadIdx.x / W) % H, pc = threadIdx.x / HW;
#pragma unroll
    for (int u = 0; u < kPairRegs; ++u) {
      const int Y = py + pad, X = px + pad;
      const bool keep = pc < C && (Y >> 1) < BH;
      const int rb = __umul24(pc, g.plane) + (Y & 1) * HALF + __umul24(Y >> 1, 2 * BW);
#pragma unroll
      for (int sx = 0; sx < 2; ++sx) {
        const int Xs = X - sx;
        const bool in = keep && Xs >= 0 && (Xs >> 1) < BW;
        lds[in ? rb + sx * 2 * HALF + Xs : dump] = pf[u];  // pair Xs/2, element Xs&1
      }
      px += tx;
      const int cy = px >= W;
      px -= cy ? W : 0;
      py += ty + cy;
      const int cc = py >= H;
      py -= cc ? H : 0;
      pc += tc + cc;
    }
  };

  // the lane's pair, output index and activity per chunk (the same for every
  // channel and sample); lanes past the sample's LPS read the pair of the
  // lane 32 below, which keeps a conflict group's pairs distinct
  int qp[kPairMaxChunks], pidx[kPairMaxChunks];
  bool act[kPairMaxChunks];
  const int nchunks = (g.LPS + 63) / 64;
#pragma unroll
  for (int c = 0; c < kPairMaxChunks; ++c) {
    const int q = c * 64 + lane;
    const int py = q / BW, px = q - py * BW;
    act[c] = q < g.LPS && px < Wo;
    pidx[c] = py * Wo + px;
    qp[c] = q < g.LPS ? q : max(0, min(q - 32, g.LPS - 1));
  }

  auto load = [&](ConvParams<NODE, NLEAF, KM, NW>& Pr, int n) {
    if constexpr (REC) conv_params_record<NODE, NLEAF, KM, NW, Cfg::REC>(Pr, rec, n);
    else conv_params_arrays<NODE, NLEAF, KM, NW>(Pr, n, K, C, kernel, g, np, wts, cm, ch, cw);
  };
  const bool one_group = N <= nwaves;
  ConvParams<NODE, NLEAF, KM, NW> Pc;
  if (one_group && wave < N) load(Pc, wave);

  if (blockIdx.x < (unsigned)B) issue(blockIdx.x);
  __syncthreads();  // cleared before the first scatter
  for (int b = blockIdx.x; b < B; b += gridDim.x) {
    scatter();
    __syncthreads();
    if (b + (int)gridDim.x < B) issue(b + gridDim.x);
    for (int n = wave; n < N; n += nwaves) {
      if (!one_group) load(Pc, n);
      float* out_n = out + ((int64_t)b * N + n) * P;
#pragma unroll
      for (int c = 0; c < kPairMaxChunks; ++c) {
        if (c >= nchunks) break;
        const f32x2* base = reinterpret_cast<const f32x2*>(lds) + qp[c];
        float v[4][NLEAF];
#pragma unroll
        for (int l = 0; l < NLEAF; ++l)
#pragma unroll
          for (int qq = 0; qq < 4; ++qq) v[qq][l] = 0.0f;
#pragma unroll
        for (int k = 0; k < KM; ++k) {
          if (k == 0 || k < K) {  // K >= 1: step 0 always runs
            f32x2 t0[NLEAF], t1[NLEAF];
#pragma unroll
            for (int l = 0; l < NLEAF; ++l) {
              t0[l] = base[Pc.off[l][k][0]];
              t1[l] = base[Pc.off[l][k][1]];
            }
#pragma unroll
            for (int l = 0; l < NLEAF; ++l) {
              v[0][l] = fmaf(Pc.wt[l][k], t0[l][0], v[0][l]);
              v[1][l] = fmaf(Pc.wt[l][k], t0[l][1], v[1][l]);
              v[2][l] = fmaf(Pc.wt[l][k], t1[l][0], v[2][l]);
              v[3][l] = fmaf(Pc.wt[l][k], t1[l][1], v[3][l]);
            }
          }
        }
        float best = -INFINITY;
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) best = fmaxf(best, conv_tree_eval<NODE, NLEAF>(v[qq], Pc.par));
        if (act[c]) out_n[pidx[c]] = best;
      }
    }
    __syncthreads();  // every read of this sample precedes the next scatter
  }
}

// Pair layout with flat lanes: lane f of a sample's chunks takes output
// f % P of channel f / P (P = Ho*Wo pooled outputs), so that every lane of
// a chunk computes an output even where P is far from a multiple of 64 (a
// one-channel chunk of the pair kernel leaves 64 - P lanes of a 7x7 map
// idle, and a 3x3 map fills 9 of 16). Each lane reads its channel's
// parameters from a table that the workgroup stages in LDS once, so a chunk
// that spans channels costs LDS reads, not vector memory traffic: per
// channel FW floats, for each tap step k the LDS byte offsets of both
// window rows and the weight of every leaf (KS floats, read as the step
// starts, so that only one step's worth is held in registers), then the
// node parameters. Staging, layout and arithmetic per output are
// conv_soft_pair_kernel's, in the same order.
template <int NODE, int NLEAF, int KM>
struct FlatRec {
  static constexpr int KS = (3 * NLEAF + 3) & ~3;                    // floats per tap step
  static constexpr int NPR4 = (ConvNode<NODE, NLEAF>::NPR + 3) & ~3;  // node parameters
  static constexpr int FW = KM * KS + NPR4;                           // floats per channel
};

template <int NODE, int NLEAF, int KM, bool REC>
__global__ void __launch_bounds__(kQuadThreads)
conv_soft_flat_kernel(const float* __restrict__ x, int B, int C, int H, int W, int N, int K,
                      int kernel, int pad, ConvGeom g, const float* __restrict__ np,
                      const float* __restrict__ wts, const int* __restrict__ cm,
                      const int* __restrict__ ch, const int* __restrict__ cw,
                      const float* __restrict__ rec, float* __restrict__ out, int Ho, int Wo) {
  using Cfg = ConvCfg<NODE, NLEAF, KM, true>;
  static_assert(Cfg::PHASE, "the pair layout keeps the phase records");
  constexpr int NW = 2;
  constexpr int NPR = ConvNode<NODE, NLEAF>::NPR;
  constexpr int FW = FlatRec<NODE, NLEAF, KM>::FW, KS = FlatRec<NODE, NLEAF, KM>::KS;
  constexpr int NPR4 = FlatRec<NODE, NLEAF, KM>::NPR4;
  extern __shared__ float lds[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nwaves = blockDim.x >> 6;
  const int T = blockDim.x;
  const int HW = H * W, total = C * HW;
  const int P = Ho * Wo;
  const int BH = g.BH, BW = g.BW;
  const int HALF = 2 * BH * BW;
  float* table = lds + g.SST + kConvExtra;

  for (int i = threadIdx.x; i < (g.SST + kConvExtra) / 4; i += T)
    reinterpret_cast<f32x4*>(lds)[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  // the parameter table: per tap step, the LDS byte offsets of the two
  // window rows and the weight of every leaf; then the node parameters
  for (int n = threadIdx.x; n < N; n += T) {
    ConvParams<NODE, NLEAF, KM, NW> Pr;
    if constexpr (REC) conv_params_record<NODE, NLEAF, KM, NW, Cfg::REC>(Pr, rec, n);
    else conv_params_arrays<NODE, NLEAF, KM, NW>(Pr, n, K, C, kernel, g, np, wts, cm, ch, cw);
    float* tr = table + n * FW;
#pragma unroll
    for (int k = 0; k < KM; ++k) {
#pragma unroll
      for (int l = 0; l < NLEAF; ++l) {
        tr[k * KS + 3 * l] = __int_as_float(Pr.off[l][k][0] * 8);
        tr[k * KS + 3 * l + 1] = __int_as_float(Pr.off[l][k][1] * 8);
        tr[k * KS + 3 * l + 2] = Pr.wt[l][k];
      }
#pragma unroll
      for (int i = 3 * NLEAF; i < KS; ++i) tr[k * KS + i] = 0.0f;
    }
#pragma unroll
    for (int i = 0; i < NPR4; ++i) tr[KM * KS + i] = i < NPR ? Pr.par[i] : 0.0f;
  }

  float pf[kPairRegs];
  auto issue = [&](int b) {
    const __amdgpu_buffer_rsrc_t src = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(x + (int64_t)b * total), (short)0, total * 4, kBufferWord3);
#pragma unroll
    for (int u = 0; u < kPairRegs; ++u)  // offsets past the image read 0
      pf[u] = __uint_as_float(
          __builtin_amdgcn_raw_buffer_load_b32(src, (threadIdx.x + u * T) * 4, 0, 0));
  };
  const int dump = g.SST + lane;
  auto scatter = [&] {
    const int tx = T % W, ty = (T / W) % H, tc = T / HW;
    int px = threadIdx.x % W, py = (threadIdx.x / W) % H, pc = threadIdx.x / HW;
#pragma unroll
    for (int u = 0; u < kPairRegs; ++u) {
      const int Y = py + pad, X = px + pad;
      const bool keep = pc < C && (Y >> 1) < BH;
      const int rb = __umul24(pc, g.plane) + (Y & 1) * HALF + __umul24(Y >> 1, 2 * BW);
#pragma unroll
      for (int sx = 0; sx < 2; ++sx) {
        const int Xs = X - sx;
        const bool in = keep && Xs >= 0 && (Xs >> 1) < BW;
        lds[in ? rb + sx * 2 * HALF + Xs : dump] = pf[u];
      }
      px += tx;
      const int cy = px >= W;
      px -= cy ? W : 0;
      py += ty + cy;
      const int cc = py >= H;
      py -= cc ? H : 0;
      pc += tc + cc;
    }
  };

  // the lane's first (channel, pooled row, column) and the step between a
  // wave's chunks (64 * nwaves outputs), carried incrementally
  const int NP_ = N * P;
  const int nchunks = (NP_ + 63) / 64;
  const int f0 = wave * 64 + lane;
  const int n0 = f0 / P, p0 = f0 - (f0 / P) * P;
  const int r0 = p0 / Wo, c0 = p0 - (p0 / Wo) * Wo;
  const int dF = 64 * nwaves;
  const int dn = dF / P, dp = dF - dn * P;
  const int dr = dp / Wo, dc = dp - dr * Wo;

  if (blockIdx.x < (unsigned)B) issue(blockIdx.x);
  __syncthreads();  // cleared and the table written before the first scatter
  for (int b = blockIdx.x; b < B; b += gridDim.x) {
    scatter();
    __syncthreads();
    if (b + (int)gridDim.x < B) issue(b + gridDim.x);
    float* out_b = out + (int64_t)b * NP_;
    int n = n0, row = r0, col = c0;
    for (int c = wave; c < nchunks; c += nwaves) {
      const int f = c * 64 + lane;
      const bool active = f < NP_;
      const int nn = active ? n : N - 1;
      const int q = active ? (int)__umul24(row, BW) + col : 0;
      const uint32_t qb = (uint32_t)q * 8u;
      const float* trow = table + nn * FW;  // the lane's channel in the table
      float v[4][NLEAF];
#pragma unroll
      for (int l = 0; l < NLEAF; ++l)
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) v[qq][l] = 0.0f;
#pragma unroll
      for (int k = 0; k < KM; ++k) {
        if (k == 0 || k < K) {  // K >= 1: step 0 always runs
          float st[KS];  // this step's offsets and weights
#pragma unroll
          for (int i = 0; i < KS / 4; ++i) {
            const f32x4 v4 = reinterpret_cast<const f32x4*>(trow + k * KS)[i];
            st[4 * i] = v4[0]; st[4 * i + 1] = v4[1]; st[4 * i + 2] = v4[2]; st[4 * i + 3] = v4[3];
          }
          f32x2 t0[NLEAF], t1[NLEAF];
#pragma unroll
          for (int l = 0; l < NLEAF; ++l) {
            const uint32_t a0 = qb + (uint32_t)__float_as_int(st[3 * l]);
            const uint32_t a1 = qb + (uint32_t)__float_as_int(st[3 * l + 1]);
            t0[l] = *reinterpret_cast<const f32x2*>(reinterpret_cast<const char*>(lds) + a0);
            t1[l] = *reinterpret_cast<const f32x2*>(reinterpret_cast<const char*>(lds) + a1);
          }
#pragma unroll
          for (int l = 0; l < NLEAF; ++l) {
            const float w = st[3 * l + 2];
            v[0][l] = fmaf(w, t0[l][0], v[0][l]);
            v[1][l] = fmaf(w, t0[l][1], v[1][l]);
            v[2][l] = fmaf(w, t1[l][0], v[2][l]);
            v[3][l] = fmaf(w, t1[l][1], v[3][l]);
          }
        }
      }
      // node parameters: into registers, except a hybrid LUT's, which is
      // read at a data-dependent address and so stays in LDS
      float best = -INFINITY;
      if constexpr (NODE == SLG_NODE_HYBRID) {
#pragma unroll
        for (int qq = 0; qq < 4; ++qq)
          best = fmaxf(best, conv_tree_eval<NODE, NLEAF>(v[qq], trow + KM * KS));
      } else {
        float par[NPR4];
#pragma unroll
        for (int i = 0; i < NPR4 / 4; ++i) {
          const f32x4 v4 = reinterpret_cast<const f32x4*>(trow + KM * KS)[i];
          par[4 * i] = v4[0]; par[4 * i + 1] = v4[1]; par[4 * i + 2] = v4[2]; par[4 * i + 3] = v4[3];
        }
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) best = fmaxf(best, conv_tree_eval<NODE, NLEAF>(v[qq], par));
      }
      if (active) out_b[f] = best;
      // next chunk of this wave
      n += dn;
      col += dc;
      row += dr;
      if (col >= Wo) { col -= Wo; ++row; }
      if (row >= Ho) { row -= Ho; ++n; }
    }
    __syncthreads();  // every read of this sample precedes the next scatter
  }
}

template <int NODE, int NLEAF, bool POOL>
__global__ void __launch_bounds__(256)
conv_hard_kernel(const uint64_t* __restrict__ xp, int C, int H, int W, int nw, int N,
                 const int* __restrict__ leaf, const uint64_t* __restrict__ tt, int kernel, int pad,
                 uint64_t* __restrict__ out, int Ho, int Wo) {
  const int n = blockIdx.y;
  const int P = Ho * Wo;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)P * nw) return;
  const int p = (int)(i / nw), w = (int)(i - (int64_t)p * nw);
  const int oy = (p / Wo) * (POOL ? 2 : 1);
  const int ox = (p % Wo) * (POOL ? 2 : 1);
  int lc[NLEAF], lh[NLEAF], lw[NLEAF];
#pragma unroll
  for (int l = 0; l < NLEAF; ++l) {
    const int code = leaf[n * NLEAF + l];
    lc[l] = min(max(code >> 8, 0), C - 1);
    lh[l] = min((code >> 4) & 15, kernel - 1);
    lw[l] = min(code & 15, kernel - 1);
  }
  const uint64_t T = tt[n];
  uint64_t acc = 0;
#pragma unroll
  for (int q = 0; q < (POOL ? 4 : 1); ++q) {
    const int py = oy + (q >> 1), px = ox + (q & 1);
    uint64_t v[NLEAF];
#pragma unroll
    for (int l = 0; l < NLEAF; ++l) {
      const int iy = py + lh[l] - pad, ix = px + lw[l] - pad;
      v[l] = (iy >= 0 && iy < H && ix >= 0 && ix < W)
                 ? xp[(((int64_t)lc[l] * H + iy) * W + ix) * nw + w]
                 : 0ull;
    }
    uint64_t val;
    if constexpr (NODE == SLG_NODE_GATE16) {
      int nb = 0;
#pragma unroll
      for (int cnt = NLEAF; cnt > 1; cnt >>= 1) {
#pragma unroll
        for (int m = 0; m < cnt / 2; ++m) {
          const uint32_t g = (uint32_t)(T >> (4 * (nb + m))) & 15u;
          const uint64_t a = v[2 * m], b = v[2 * m + 1];
          const uint64_t t0 = 0ull - (uint64_t)(g & 1u), t1 = 0ull - (uint64_t)((g >> 1) & 1u);
          const uint64_t t2 = 0ull - (uint64_t)((g >> 2) & 1u), t3 = 0ull - (uint64_t)((g >> 3) & 1u);
          v[m] = (a & ((b & t3) | (~b & t2))) | (~a & ((b & t1) | (~b & t0)));
        }
        nb += cnt / 2;
      }
      val = v[0];
    } else {
      // Shannon mux tree over address bits (leaf j = address bit j),
      // silogic/nodes.py:183-189
      uint64_t t[1 << (NLEAF - 1)];
#pragma unroll
      for (int m = 0; m < (1 << (NLEAF - 1)); ++m) {
        const uint64_t e0 = 0ull - ((T >> (2 * m)) & 1ull);
        const uint64_t e1 = 0ull - ((T >> (2 * m + 1)) & 1ull);
        t[m] = (v[0] & e1) | (~v[0] & e0);
      }
#pragma unroll
      for (int j = 1; j < NLEAF; ++j) {
#pragma unroll
        for (int m = 0; m < (1 << (NLEAF - 1 - j)); ++m)
          t[m] = (v[j] & t[2 * m + 1]) | (~v[j] & t[2 * m]);
      }
      val = t[0];
    }
    acc |= val;
  }
  out[((int64_t)n * P + p) * nw + w] = acc;
}

// ---------------------------------------------------------------------------
// prep kernels
// ---------------------------------------------------------------------------
__constant__ float c_basis_conv[16][4] = {
    {0, 0, 0, 0}, {0, 0, 0, 1}, {0, 1, 0, -1}, {0, 1, 0, 0}, {0, 0, 1, -1}, {0, 0, 1, 0},
    {0, 1, 1, -2}, {0, 1, 1, -1}, {1, -1, -1, 1}, {1, -1, -1, 2}, {1, 0, -1, 0},
    {1, 0, -1, 1}, {1, -1, 0, 0}, {1, -1, 0, 1}, {1, 0, 0, -1}, {1, 0, 0, 0}};
__constant__ uint8_t c_tt16_conv[16] = {0x0, 0x8, 0x4, 0xC, 0x2, 0xA, 0x6, 0xE,
                                        0x1, 0x9, 0x5, 0xD, 0x3, 0xB, 0x7, 0xF};

__global__ void conv_soft_prep_kernel(const float* __restrict__ conn, int N, int leaves, int K,
                                      int node, int nodes, int arity, const float* __restrict__ raw,
                                      float* __restrict__ w, float* __restrict__ np) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  for (int l = 0; l < leaves; ++l) {
    const int64_t base = ((int64_t)n * leaves + l) * K;
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
  if (node == SLG_NODE_GATE16) {
    for (int j = 0; j < nodes; ++j) {
      const float* g = raw + ((int64_t)n * nodes + j) * 16;
      float m = g[0];
      for (int i = 1; i < 16; ++i) m = fmaxf(m, g[i]);
      float e[16], sum = 0.f;
      for (int i = 0; i < 16; ++i) { e[i] = expf(g[i] - m); sum += e[i]; }
      float acc[4] = {0.f, 0.f, 0.f, 0.f};
      for (int i = 0; i < 16; ++i) {
        const float pr = e[i] / sum;
        for (int q = 0; q < 4; ++q) acc[q] += pr * c_basis_conv[i][q];
      }
      for (int q = 0; q < 4; ++q) np[((int64_t)n * nodes + j) * 4 + q] = acc[q];
    }
  } else {
    const int P = 1 << arity;
    for (int q = 0; q < P; ++q) np[(int64_t)n * P + q] = sigmoidc(raw[(int64_t)n * P + q]);
  }
}

// Per-channel records for conv_soft_kernel<..., REC = true>, R floats per
// channel: [0, L*KM*NW) LDS offsets of the KM taps of every leaf, NW per tap
// (ConvParams order; clamped taps; taps k >= K get offset 0 and weight 0),
// then L*KM softmax leaf weights, then the node parameters (gate16:
// softmax(logits) @ BASIS per node; LUT: sigmoid(s) of the even corners,
// then odd - even differences), zeros to R. One thread per record word, so
// that the loads of different words overlap.
// ARR: from the separate arrays of slg_conv_soft_fwd instead (conn = the
// leaf weights w [N,L,K], raw = the node parameters as that entry point takes
// them: gate16 coefficients, LUT corner values), so that the records hold
// what conv_params_arrays computes in the kernel, bit for bit.
template <bool ARR>
__global__ void conv_soft_records_kernel(const float* __restrict__ conn, const int* __restrict__ cm,
                                         const int* __restrict__ ch, const int* __restrict__ cw,
                                         int N, int leaves, int K, int KM, int NW, int node,
                                         int arity, const float* __restrict__ raw, int C,
                                         int kernel, ConvGeom g, int R, float* __restrict__ rec) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (int64_t)N * R) return;
  const int n = (int)(t / R), slot = (int)(t - (int64_t)n * R);
  const int LK = leaves * KM;
  float v = 0.0f;
  if (slot < LK * (NW + 1)) {
    const bool is_off = slot < LK * NW;
    const int lk = is_off ? slot / NW : slot - LK * NW;
    const int l = lk / KM, k = lk - l * KM;
    const int64_t base = ((int64_t)n * leaves + l) * K;
    if (k < K) {
      if (is_off) {
        const int c_ = min(max(cm[base + k], 0), C - 1);
        const int h_ = min(max(ch[base + k], 0), kernel - 1);
        const int w_ = min(max(cw[base + k], 0), kernel - 1);
        v = __int_as_float(conv_tap_offset(g, NW, c_, h_, w_, slot - lk * NW));
      } else if (!conn) {
        v = 1.0f;
      } else if (ARR) {
        v = conn[base + k];
      } else {
        float c[kMaxK];
#pragma unroll
        for (int j = 0; j < kMaxK; ++j) c[j] = j < K ? conn[base + j] : -INFINITY;
        float m = c[0];
#pragma unroll
        for (int j = 1; j < kMaxK; ++j) m = fmaxf(m, c[j]);
        float sum = 0.f;
#pragma unroll
        for (int j = 0; j < kMaxK; ++j) sum += j < K ? expf(c[j] - m) : 0.f;
        v = expf(conn[base + k] - m) / sum;
      }
    }
  } else if (ARR && node != SLG_NODE_MULTILINEAR2) {  // gate16 coefficients, hybrid values
    const int q = slot - LK * (NW + 1);
    const int NP = node == SLG_NODE_GATE16 ? 4 * (leaves - 1) : (1 << arity);
    if (q < NP) v = raw[(int64_t)n * NP + q];
  } else if (node == SLG_NODE_GATE16) {
    const int q = slot - LK * (NW + 1), j = q >> 2;
    if (j < leaves - 1) {
      const float* gl = raw + ((int64_t)n * (leaves - 1) + j) * 16;
      float e[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) e[i] = gl[i];
      float m = e[0];
#pragma unroll
      for (int i = 1; i < 16; ++i) m = fmaxf(m, e[i]);
      float sum = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) { e[i] = expf(e[i] - m); sum += e[i]; }
      float acc = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) acc += (e[i] / sum) * c_basis_conv[i][q & 3];
      v = acc;
    }
  } else if (node == SLG_NODE_HYBRID) {
    const int P = 1 << arity, q = slot - LK * (NW + 1);
    if (q < P) v = sigmoidc(raw[(int64_t)n * P + q]);
  } else {
    // the kept form of conv_tree.h: per group of corners, its polynomial's
    // coefficients (lut_group_coeffs over the group's corner values: the
    // sigmoid of the logits, or the values as given)
    const int P = 1 << arity, q = slot - LK * (NW + 1);
    const float* s_ = raw + (int64_t)n * P;
    auto val = [&](int i) { return ARR ? s_[i] : sigmoidc(s_[i]); };
    if (q < P) {
      if (arity >= 3) {
        float c[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) c[i] = val((q & ~7) + i);
        lut_group_coeffs<3>(c);
        v = c[q & 7];
      } else if (arity == 2) {
        float c[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) c[i] = val(i);
        lut_group_coeffs<2>(c);
        v = c[q & 3];
      } else {
        float c[2] = {val(0), val(1)};
        lut_group_coeffs<1>(c);
        v = c[q & 1];
      }
    }
  }
  rec[t] = v;
}

// Hard parameters of up to kMaxConvPrepBlocks conv blocks in one launch, one
// thread per output channel; workgroups map to blocks through blk_start.
// gate16 logits are read per tree level in place (level l: [N, 2^(depth-1-l),
// 16] with row stride rstride[l] floats), the way the reference's hard tree
// walks its per-level parameters (layers.py:515-527); multilinear nodes use
// raw[0] = [N, 2^arity].
constexpr int kMaxConvPrepBlocks = 8;
struct ConvPrepBlock {
  const int* cm;
  const int* ch;
  const int* cw;
  const float* conn;
  const float* raw[4];
  int rstride[4];
  int* leaf;
  uint64_t* tt;
  int N, leaves, K, node, depth, arity;
};
struct ConvPrepNet {
  ConvPrepBlock b[kMaxConvPrepBlocks];
  int blk_start[kMaxConvPrepBlocks + 1];
  int n;
};

__global__ void __launch_bounds__(128) conv_hard_prep_kernel(ConvPrepNet net) {
  int k = 0;
  while (k + 1 < net.n && (int)blockIdx.x >= net.blk_start[k + 1]) ++k;
  const ConvPrepBlock& P = net.b[k];
  const int n = ((int)blockIdx.x - net.blk_start[k]) * blockDim.x + threadIdx.x;
  if (n >= P.N) return;
  const int leaves = P.leaves, K = P.K;
  for (int l = 0; l < leaves; ++l) {
    const int64_t base = ((int64_t)n * leaves + l) * K;
    int c = 0;
    if (P.conn) {  // first index of the max, as torch.argmax (layers.py:511-513)
      float bv = P.conn[base];
      for (int j = 1; j < K; ++j)
        if (P.conn[base + j] > bv) { bv = P.conn[base + j]; c = j; }
    }
    P.leaf[n * leaves + l] =
        (P.cm[base + c] << 8) | ((P.ch[base + c] & 15) << 4) | (P.cw[base + c] & 15);
  }
  uint64_t t = 0;
  if (P.node == SLG_NODE_GATE16) {
    int j = 0;
    for (int lv = 0; lv < P.depth; ++lv) {
      const int m = 1 << (P.depth - 1 - lv);
      const float* row = P.raw[lv] + (int64_t)n * P.rstride[lv];
      for (int i = 0; i < m; ++i, ++j) {
        const float* g = row + i * 16;
        int bi = 0;
        float bv = g[0];
        for (int q = 1; q < 16; ++q)
          if (g[q] > bv) { bv = g[q]; bi = q; }
        t |= (uint64_t)c_tt16_conv[bi] << (4 * j);
      }
    }
  } else {
    const int Pn = 1 << P.arity;
    for (int q = 0; q < Pn; ++q)
      if (P.raw[0][(int64_t)n * P.rstride[0] + q] > 0.0f) t |= 1ull << q;
  }
  P.tt[n] = t;
}

// size x size max pool with stride size and floor (F.max_pool2d(x, s, s)),
// the window scanned row-major.
template <typename T>
__global__ void orpool_kernel(const T* __restrict__ x, int64_t BC, int H, int W, int size,
                              T* __restrict__ out) {
  const int Ho = H / size, Wo = W / size;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= BC * Ho * Wo) return;
  const int64_t bc = i / (Ho * Wo);
  const int r = (int)(i - bc * Ho * Wo);
  const int py = r / Wo, px = r - (r / Wo) * Wo;
  const T* src = x + bc * H * W + (int64_t)(size * py) * W + size * px;
  T m = src[0];
  for (int dy = 0; dy < size; ++dy)
    for (int dx = 0; dx < size; ++dx) {
      const T v = src[dy * W + dx];
      m = m > v ? m : v;
    }
  out[i] = m;
}

// ---------------------------------------------------------------------------
// launch helpers
// ---------------------------------------------------------------------------
struct ConvSoftArgs {
  const float* x; int64_t B, C, H, W, N; int K, kernel, pad;
  const float* np; const float* w; const int* cm; const int* ch; const int* cw;
  float* out; int64_t Ho, Wo;
  const float* rec;  // records (REC kernels) or null
};

// Quad geometry (pooled; see the layouts above): BH x BW blocks per copy
// cover every window of Ho x Wo pooled outputs under kernel x kernel taps.
static ConvGeom conv_geom_quad(int64_t C, int64_t Ho, int64_t Wo, int kernel) {
  ConvGeom g{};
  g.BH = (int)(Ho + (kernel - 1) / 2);
  g.BW = (int)(Wo + (kernel - 1) / 2);
  g.plane = 16 * g.BH * g.BW;  // floats: four copies of BH x BW blocks of four
  g.LPS = (int)(Ho * Wo);
  g.SST = (int)(C * g.plane);
  g.RS = (int)Wo;  // the persistent kernel's lane walk (conv_quad_walk)
  return g;
}

// b128 conflict groups of the persistent quad kernel's chunks whose 16 blocks
// (one per lane, outputs walked in rows of ww columns) hold two distinct
// blocks of one bank class (block mod 16), over one channel's chunks.
static int quad_colliding_groups(int64_t Ho, int64_t Wo, int BW, int64_t ww) {
  const int64_t n = Ho * ww;
  int bad = 0;
  for (int64_t c0 = 0; c0 < n; c0 += 16) {
    int seen[16];
    for (int i = 0; i < 16; ++i) seen[i] = -1;
    bool clash = false;
    for (int64_t q = c0; q < std::min<int64_t>(c0 + 16, n); ++q) {
      const int64_t row = q / ww, col = q % ww;
      if (col >= Wo) continue;
      const int blk = (int)(row * BW + col);
      if (seen[blk & 15] >= 0 && seen[blk & 15] != blk) clash = true;
      seen[blk & 15] = blk;
    }
    bad += clash;
  }
  return bad;
}

// The persistent quad kernel walks rows of BW columns (padding lanes idle)
// where the dense walk has a bank-class collision in most 16-lane groups and
// the padded walk takes at most 1/8 more chunks.
static int conv_quad_walk(int64_t Ho, int64_t Wo, int BW) {
  const int64_t dense = cdiv(Ho * Wo, 16), padded = cdiv(Ho * BW, 16);
  if (8 * padded > 9 * dense) return (int)Wo;
  return 2 * quad_colliding_groups(Ho, Wo, BW, Wo) > dense &&
                 quad_colliding_groups(Ho, Wo, BW, BW) < quad_colliding_groups(Ho, Wo, BW, Wo)
             ? BW
             : (int)Wo;
}

// The quad layout is used for pooled blocks with phase-eligible taps whose
// four image copies fit the LDS of one workgroup.
static bool conv_use_quad(bool pool, int nleaf, int km, int64_t C, int64_t Ho, int64_t Wo,
                          int kernel) {
  if (!conv_phase_layout(pool, nleaf, km) || Ho <= 0 || Wo <= 0) return false;
  if (C * 16 * (Ho + kernel) * (Wo + kernel) >= (1LL << 29)) return false;
  const ConvGeom g = conv_geom_quad(C, Ho, Wo, kernel);
  const int64_t cap = std::min<int64_t>(device_lds_bytes(), 160 * 1024);
  return (int64_t)g.SST * 4 + kConvExtra * 4 <= cap;
}

// Pair geometry (pooled; see the layouts above): BH half-rows of BW pairs per
// row parity and copy cover every window of Ho x Wo pooled outputs.
static ConvGeom conv_geom_pair(int64_t C, int64_t Ho, int64_t Wo, int kernel) {
  ConvGeom g{};
  g.BH = (int)(Ho + (kernel - 1) / 2);
  g.BW = (int)(Wo + (kernel - 1) / 2);
  g.plane = 8 * g.BH * g.BW;  // floats: two copies of two row parities of BH x BW pairs
  g.LPS = (int)(Ho * g.BW);
  g.SST = (int)(C * g.plane);
  g.PAIR = 1;
  return g;
}

// Floats per channel of the flat pair kernel's parameter table (FlatRec::FW).
static int conv_flat_fw(int node, int nleaf, int km) {
  const int npr = node == SLG_NODE_GATE16 ? 4 * (nleaf - 1) : (1 << nleaf);
  return km * ((3 * nleaf + 3) & ~3) + ((npr + 3) & ~3);
}

// Flat lanes where the parameter table fits beside the image and a
// channel's pooled map is not a whole number of 64-lane chunks.
static bool conv_pair_flat(const ConvGeom& g, int64_t N, int64_t Ho, int64_t Wo, int fw) {
  const int64_t cap = std::min<int64_t>(device_lds_bytes(), 160 * 1024);
  if (((int64_t)g.SST + kConvExtra + N * fw) * 4 > cap) return false;
  return (Ho * Wo) % 64 != 0;
}

enum { kLayoutPlain = 0, kLayoutQuad = 1, kLayoutPair = 2 };

// Layout of a pooled block with phase-eligible taps: quad where its four
// copies fit one workgroup's LDS and a channel's outputs fill at least 7/8
// of its 16-lane groups; else pair where the two pair copies fit, the image
// rides in kPairRegs registers per thread and either the flat kernel's
// parameter table fits too or a channel's lanes take at most kPairMaxChunks
// chunks; else quad where it fits; else the phase-split layout.
static int conv_pooled_layout(bool pool, int node, int nleaf, int km, int64_t C, int64_t H,
                              int64_t W, int64_t Ho, int64_t Wo, int kernel, int64_t N) {
  if (!conv_phase_layout(pool, nleaf, km) || Ho <= 0 || Wo <= 0) return kLayoutPlain;
  const bool quad = conv_use_quad(pool, nleaf, km, C, Ho, Wo, kernel);
  bool pair = C * H * W <= (int64_t)kPairRegs * kQuadThreads &&
              C * 8 * (Ho + kernel) * (Wo + kernel) < (1LL << 29);
  bool flat = false;
  if (pair) {
    const ConvGeom g = conv_geom_pair(C, Ho, Wo, kernel);
    const int64_t cap = std::min<int64_t>(device_lds_bytes(), 160 * 1024);
    flat = conv_pair_flat(g, N, Ho, Wo, conv_flat_fw(node, nleaf, km));
    pair = (int64_t)g.SST * 4 + kConvExtra * 4 <= cap && (flat || g.LPS <= 64 * kPairMaxChunks);
  }
  if (quad) {
    const int64_t P = Ho * Wo, lanes = 16 * cdiv(P, 16);
    return (pair && flat && 8 * P < 7 * lanes) ? kLayoutPair : kLayoutQuad;
  }
  return pair ? kLayoutPair : kLayoutPlain;
}

// LDS geometry for images (C, H, W) with 'same' padding pad, pooled to
// (Ho, Wo) or not (Ho = H, Wo = W).
static ConvGeom conv_geom(int64_t C, int64_t H, int64_t W, int pad, bool pool, bool phase,
                          int64_t Ho, int64_t Wo) {
  ConvGeom g{};
  if (phase) {
    g.RS = (int)(Wo + pad);
    g.PR = (int)(Ho + pad);
    g.PP = g.PR * g.RS;
    g.plane = 4 * g.PP;
    g.LPS = (int)Ho * g.RS;
  } else {
    g.RS = (int)(W + pad);
    g.plane = (int)((H + 2 * pad) * g.RS + pad);
    g.LPS = pool ? (int)(Ho * Wo) : (int)H * g.RS;
  }
  int64_t sst = C * g.plane;
  if (phase || !pool) sst += (((int64_t)g.LPS - sst) % 64 + 64) % 64;  // sst = LPS (mod 64)
  g.SST = (int)sst;
  return g;
}

// LDS cycles of the four reads of a tap over a wave's first chunk in the
// pooled row-major layout, modelled as 32 banks of 4 bytes served per half
// wave (distinct words of one bank serialise, equal words broadcast), with
// the window's columns in index order (swap = false) or swapped on odd
// pooled columns. The counters of the config blocks follow this model's
// ratios.
static int pooled_read_cycles(const ConvGeom& g, int Wo, bool swap) {
  int total = 0;
  for (int i = 0; i < 4; ++i) {
    for (int h = 0; h < 2; ++h) {
      int words[32][32], n[32] = {0}, worst = 0;
      for (int ln = 32 * h; ln < 32 * h + 32; ++ln) {
        const int s = ln / g.LPS, rem = ln % g.LPS, row = rem / Wo, col = rem % Wo;
        const int sw = swap ? (col & 1) : 0;
        const int dy = i >> 1, dx = (i & 1) ^ sw;
        const int w = s * g.SST + 2 * row * g.RS + 2 * col + dy * g.RS + dx;
        const int b = w & 31;
        bool seen = false;
        for (int j = 0; j < n[b]; ++j) seen = seen || words[b][j] == w;
        if (!seen) words[b][n[b]++] = w;
        worst = std::max(worst, n[b]);
      }
      total += worst;
    }
  }
  return total;
}

// The swapped order where the model halves the reads' cycles: from at least
// 6 per read with a runtime row stride (two VALU adds more per tap: worth it
// where the reads stall), from any count with a constant one (`cheap`: one
// add more per tap; config 5 block 0, 2 -> 1 modelled cycles per read:
// 196 -> 174 us).
static bool conv_swap_pays(const ConvGeom& g, int Wo, bool cheap) {
  const int plain = pooled_read_cycles(g, Wo, false), swapped = pooled_read_cycles(g, Wo, true);
  return (cheap || plain >= 24) && 2 * swapped <= plain;
}

template <int NODE, int NLEAF, bool POOL, int KM, bool REC, bool QUAD>
static int launch_conv_soft_k(const ConvSoftArgs& a, hipStream_t st) {
  using Cfg = ConvCfg<NODE, NLEAF, KM, POOL>;
  const ConvGeom g = QUAD ? conv_geom_quad(a.C, a.Ho, a.Wo, a.kernel)
                          : conv_geom(a.C, a.H, a.W, a.pad, POOL, Cfg::PHASE, a.Ho, a.Wo);
  const int64_t per_sample = (int64_t)g.SST * 4;
  const int64_t cap = std::min<int64_t>(device_lds_bytes(), 160 * 1024);
  SLG_REQUIRE(per_sample + kConvExtra * 4 <= cap && (int64_t)a.C * a.H * a.W * 4 < (1LL << 31),
              SLG_E_UNSUPPORTED, "conv_soft: one image (%lld B) exceeds LDS",
              (long long)per_sample);
  // Samples per workgroup: two chunks per channel where the images are
  // small; up to half the LDS so that two workgroups share a CU, or all of it
  // when half would leave most lanes of a chunk idle; at least one workgroup
  // per CU.
  const int64_t room = cap - kConvExtra * 4;
  int64_t S = std::max<int64_t>(1, cdiv(128, g.LPS));
  const int64_t s_half = (cap / 2 - kConvExtra * 4) / per_sample;
  if (s_half >= 1 && s_half * g.LPS >= 64) S = std::min(S, s_half);
  else S = std::min(S, std::max<int64_t>(1, std::min(room / per_sample, cdiv(64, g.LPS))));
  S = std::min<int64_t>(S, std::max<int64_t>(1, a.B / device_cus()));
  S = std::min<int64_t>(S, a.B);
  if (QUAD) S = 1;
  const size_t lds = (size_t)(S * per_sample + kConvExtra * 4);
  if constexpr (QUAD && POOL) {
    if (a.C * a.H * a.W <= (int64_t)kQuadRegs * kQuadThreads) {
      auto qk = conv_soft_quad_kernel<NODE, NLEAF, KM, REC>;
      if (lds > 65536) {
        hipError_t e = hipFuncSetAttribute((const void*)qk,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) {
          set_error("conv_soft: LDS %zu: %s", lds, hipGetErrorString(e));
          return (int)e;
        }
      }
      const int64_t grid = std::min<int64_t>(a.B, device_cus());
      ConvGeom gq = g;
      gq.RS = conv_quad_walk(a.Ho, a.Wo, g.BW);
      hipLaunchKernelGGL(qk, dim3((unsigned)grid), dim3(kQuadThreads), lds, st, a.x, (int)a.B,
                         (int)a.C, (int)a.H, (int)a.W, (int)a.N, a.K, a.kernel, a.pad, gq, a.np,
                         a.w, a.cm, a.ch, a.cw, a.rec, a.out, (int)a.Ho, (int)a.Wo);
      SLG_LAUNCH_CHECK("conv_soft");
      return 0;
    }
  }
  auto kern = conv_soft_kernel<NODE, NLEAF, POOL, KM, REC, QUAD>;
  if constexpr (POOL && !Cfg::PHASE && !QUAD) {
    // LUT trees of 5-6 leaves (VALU-bound): the row strides of 16- and
    // 32-wide images with 'same' padding 1 as constants
    constexpr bool kRsc = NODE == SLG_NODE_MULTILINEAR2 && NLEAF >= 5 && KM == 4;
    const bool swap = conv_swap_pays(g, (int)a.Wo, kRsc && (g.RS == 17 || g.RS == 33));
    if (swap) kern = conv_soft_kernel<NODE, NLEAF, POOL, KM, REC, QUAD, true>;
    if constexpr (kRsc) {
      if (g.RS == 17) kern = swap ? conv_soft_kernel<NODE, NLEAF, POOL, KM, REC, QUAD, true, 17>
                                  : conv_soft_kernel<NODE, NLEAF, POOL, KM, REC, QUAD, false, 17>;
      if (g.RS == 33) kern = swap ? conv_soft_kernel<NODE, NLEAF, POOL, KM, REC, QUAD, true, 33>
                                  : conv_soft_kernel<NODE, NLEAF, POOL, KM, REC, QUAD, false, 33>;
    }
  }
  if (lds > 65536) {
    hipError_t e = hipFuncSetAttribute((const void*)kern,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) {
      set_error("conv_soft: LDS %zu: %s", lds, hipGetErrorString(e));
      return (int)e;
    }
  }
  int threads = conv_soft_threads<NODE, NLEAF, KM, POOL, REC, QUAD>();
  if (REC && !QUAD && Cfg::SPLIT_OK && 2 * (int64_t)lds <= cap) threads = 512;
  hipLaunchKernelGGL(kern, dim3((unsigned)cdiv(a.B, S)), dim3(threads),
                     lds, st, a.x,
                     (int)a.B, (int)a.C, (int)a.H, (int)a.W, (int)a.N, a.K, a.kernel, a.pad, g,
                     a.np, a.w, a.cm, a.ch, a.cw, a.rec, (int)S, a.out, (int)a.Ho, (int)a.Wo);
  SLG_LAUNCH_CHECK("conv_soft");
  return 0;
}

template <int NODE, int NLEAF, int KM, bool REC>
static int launch_conv_soft_pair(const ConvSoftArgs& a, hipStream_t st) {
  const ConvGeom g = conv_geom_pair(a.C, a.Ho, a.Wo, a.kernel);
  constexpr int FW = FlatRec<NODE, NLEAF, KM>::FW;
  const bool flat = conv_pair_flat(g, a.N, a.Ho, a.Wo, FW);
  const size_t lds = (size_t)(g.SST + kConvExtra + (flat ? a.N * FW : 0)) * 4;
  auto pk = flat ? conv_soft_flat_kernel<NODE, NLEAF, KM, REC>
                 : conv_soft_pair_kernel<NODE, NLEAF, KM, REC>;
  if (lds > 65536) {
    hipError_t e =
        hipFuncSetAttribute((const void*)pk, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) {
      set_error("conv_soft: LDS %zu: %s", lds, hipGetErrorString(e));
      return (int)e;
    }
  }
  const int64_t grid = std::min<int64_t>(a.B, device_cus());
  hipLaunchKernelGGL(pk, dim3((unsigned)grid), dim3(kQuadThreads), lds, st, a.x, (int)a.B,
                     (int)a.C, (int)a.H, (int)a.W, (int)a.N, a.K, a.kernel, a.pad, g, a.np, a.w,
                     a.cm, a.ch, a.cw, a.rec, a.out, (int)a.Ho, (int)a.Wo);
  SLG_LAUNCH_CHECK("conv_soft");
  return 0;
}

template <int NODE, int NLEAF, bool POOL>
static int launch_conv_soft(const ConvSoftArgs& a, hipStream_t st) {
  // taps per leaf: 4 registers when K <= 4 (TopK k=4, fixed wiring), else 8
  if (a.K <= 4) {
    if constexpr (conv_phase_layout(POOL, NLEAF, 4)) {
      const int lay = conv_pooled_layout(POOL, NODE, NLEAF, 4, a.C, a.H, a.W, a.Ho, a.Wo,
                                         a.kernel, a.N);
      if (lay == kLayoutQuad)
        return a.rec ? launch_conv_soft_k<NODE, NLEAF, POOL, 4, true, true>(a, st)
                     : launch_conv_soft_k<NODE, NLEAF, POOL, 4, false, true>(a, st);
      if (lay == kLayoutPair)
        return a.rec ? launch_conv_soft_pair<NODE, NLEAF, 4, true>(a, st)
                     : launch_conv_soft_pair<NODE, NLEAF, 4, false>(a, st);
    }
    return a.rec ? launch_conv_soft_k<NODE, NLEAF, POOL, 4, true, false>(a, st)
                 : launch_conv_soft_k<NODE, NLEAF, POOL, 4, false, false>(a, st);
  }
  if constexpr (conv_phase_layout(POOL, NLEAF, kMaxK)) {
    const int lay = conv_pooled_layout(POOL, NODE, NLEAF, kMaxK, a.C, a.H, a.W, a.Ho, a.Wo,
                                       a.kernel, a.N);
    if (lay == kLayoutQuad)
      return a.rec ? launch_conv_soft_k<NODE, NLEAF, POOL, kMaxK, true, true>(a, st)
                   : launch_conv_soft_k<NODE, NLEAF, POOL, kMaxK, false, true>(a, st);
    if (lay == kLayoutPair)
      return a.rec ? launch_conv_soft_pair<NODE, NLEAF, kMaxK, true>(a, st)
                   : launch_conv_soft_pair<NODE, NLEAF, kMaxK, false>(a, st);
  }
  return a.rec ? launch_conv_soft_k<NODE, NLEAF, POOL, kMaxK, true, false>(a, st)
               : launch_conv_soft_k<NODE, NLEAF, POOL, kMaxK, false, false>(a, st);
}

template <bool POOL>
static int conv_soft_dispatch(const ConvSoftArgs& a, int node, int nleaf, hipStream_t st) {
  if (node == SLG_NODE_GATE16) {
    switch (nleaf) {
      case 2: return launch_conv_soft<SLG_NODE_GATE16, 2, POOL>(a, st);
      case 4: return launch_conv_soft<SLG_NODE_GATE16, 4, POOL>(a, st);
      case 8: return launch_conv_soft<SLG_NODE_GATE16, 8, POOL>(a, st);
      case 16: return launch_conv_soft<SLG_NODE_GATE16, 16, POOL>(a, st);
      default: break;
    }
  } else if (node == SLG_NODE_MULTILINEAR2) {
    switch (nleaf) {
      case 2: return launch_conv_soft<SLG_NODE_MULTILINEAR2, 2, POOL>(a, st);
      case 3: return launch_conv_soft<SLG_NODE_MULTILINEAR2, 3, POOL>(a, st);
      case 4: return launch_conv_soft<SLG_NODE_MULTILINEAR2, 4, POOL>(a, st);
      case 5: return launch_conv_soft<SLG_NODE_MULTILINEAR2, 5, POOL>(a, st);
      case 6: return launch_conv_soft<SLG_NODE_MULTILINEAR2, 6, POOL>(a, st);
      default: break;
    }
  }
  if (node == SLG_NODE_HYBRID) {
    switch (nleaf) {
      case 2: return launch_conv_soft<SLG_NODE_HYBRID, 2, POOL>(a, st);
      case 3: return launch_conv_soft<SLG_NODE_HYBRID, 3, POOL>(a, st);
      case 4: return launch_conv_soft<SLG_NODE_HYBRID, 4, POOL>(a, st);
      case 5: return launch_conv_soft<SLG_NODE_HYBRID, 5, POOL>(a, st);
      case 6: return launch_conv_soft<SLG_NODE_HYBRID, 6, POOL>(a, st);
      default: break;
    }
  }
  set_error("conv_soft: unsupported leaves %d", nleaf);
  return SLG_E_UNSUPPORTED;
}

template <int NODE, int NLEAF, bool POOL>
static int launch_conv_hard(const uint64_t* xp, int64_t C, int64_t H, int64_t W, int64_t nw,
                            int64_t N, const int* leaf, const uint64_t* tt, int kernel, int pad,
                            uint64_t* out, int64_t Ho, int64_t Wo, hipStream_t st) {
  const int64_t n = Ho * Wo * nw;
  SLG_REQUIRE(n < (1LL << 40) && N < 65536, SLG_E_SHAPE, "conv_hard: too large");
  hipLaunchKernelGGL((conv_hard_kernel<NODE, NLEAF, POOL>), dim3((unsigned)cdiv(n, 256), (unsigned)N),
                     dim3(256), 0, st, xp, (int)C, (int)H, (int)W, (int)nw, (int)N, leaf, tt,
                     kernel, pad, out, (int)Ho, (int)Wo);
  SLG_LAUNCH_CHECK("conv_hard");
  return 0;
}

template <bool POOL>
static int conv_hard_dispatch(int node, int nleaf, const uint64_t* xp, int64_t C, int64_t H,
                              int64_t W, int64_t nw, int64_t N, const int* leaf, const uint64_t* tt,
                              int kernel, int pad, uint64_t* out, int64_t Ho, int64_t Wo,
                              hipStream_t st) {
#define SLG_CH(ND, NL) \
  return launch_conv_hard<ND, NL, POOL>(xp, C, H, W, nw, N, leaf, tt, kernel, pad, out, Ho, Wo, st)
  if (node == SLG_NODE_GATE16) {
    switch (nleaf) {
      case 2: SLG_CH(SLG_NODE_GATE16, 2);
      case 4: SLG_CH(SLG_NODE_GATE16, 4);
      case 8: SLG_CH(SLG_NODE_GATE16, 8);
      case 16: SLG_CH(SLG_NODE_GATE16, 16);
      default: break;
    }
  } else {
    switch (nleaf) {
      case 2: SLG_CH(SLG_NODE_MULTILINEAR2, 2);
      case 3: SLG_CH(SLG_NODE_MULTILINEAR2, 3);
      case 4: SLG_CH(SLG_NODE_MULTILINEAR2, 4);
      case 5: SLG_CH(SLG_NODE_MULTILINEAR2, 5);
      case 6: SLG_CH(SLG_NODE_MULTILINEAR2, 6);
      default: break;
    }
  }
#undef SLG_CH
  set_error("conv_hard: unsupported leaves %d", nleaf);
  return SLG_E_UNSUPPORTED;
}

static int node_leaves(int node, int depth, int arity) {
  if (node == SLG_NODE_GATE16) return (depth >= 1 && depth <= 4) ? (1 << depth) : -1;
  if (node == SLG_NODE_MULTILINEAR2 || node == SLG_NODE_HYBRID)
    return (depth == 1 && arity >= 2 && arity <= 6) ? arity : -1;
  return -1;
}

// Records of slg_conv_soft_records (ARR = false: from the connection logits
// and raw node parameters) or slg_conv_soft_records_arrays (ARR = true: from
// slg_conv_soft_fwd's separate arrays), for the layout the forward picks.
template <bool ARR>
static int conv_records_launch(const float* conn, const int32_t* cm, const int32_t* ch,
                               const int32_t* cw, int64_t N, int32_t K, int32_t node_kind,
                               int32_t depth, int32_t arity, const float* raw, int64_t C,
                               int64_t H, int64_t W, int32_t pad, int32_t pool, float* rec,
                               slg_stream_t stream) {
  SLG_REQUIRE(cm && ch && cw && raw && rec, SLG_E_ARG, "conv_soft_records: null pointer");
  const int nleaf = node_leaves(node_kind, depth, arity);
  SLG_REQUIRE(nleaf > 0, SLG_E_UNSUPPORTED, "conv_soft_records: depth %d / arity %d", depth, arity);
  SLG_REQUIRE(K >= 1 && K <= kMaxK, SLG_E_SHAPE, "conv_soft_records: K=%d outside 1..%d", K, kMaxK);
  SLG_REQUIRE(N > 0 && N < (1LL << 20) && C > 0 && C < (1LL << 20) && H > 0 && H < 4096 &&
                  W > 0 && W < 4096 && pad >= 0 && pad <= 4,
              SLG_E_SHAPE, "conv_soft_records: bad sizes");
  const int km = K <= 4 ? 4 : kMaxK;
  const bool phase = conv_phase_layout(pool != 0, nleaf, km);
  const int64_t Ho = pool ? H / 2 : H, Wo = pool ? W / 2 : W;
  SLG_REQUIRE(C * ((H + 2 * pad) * (W + 2 * pad) + 64) < (1LL << 31), SLG_E_SHAPE,
              "conv_soft_records: image too large");
  // the layout the forward will choose for these shapes (quad offsets sit in
  // slot 0 of the phase records, pair offsets in slots 0 and 1)
  const int lay = conv_pooled_layout(pool != 0, node_kind, nleaf, km, C, H, W, Ho, Wo,
                                     2 * pad + 1, N);
  const bool quad = lay == kLayoutQuad, pair = lay == kLayoutPair;
  const ConvGeom g = quad ? conv_geom_quad(C, Ho, Wo, 2 * pad + 1)
                          : (pair ? conv_geom_pair(C, Ho, Wo, 2 * pad + 1)
                                  : conv_geom(C, H, W, pad, pool != 0, phase, Ho, Wo));
  const int R = (int)slg_conv_soft_record_floats(node_kind, depth, arity, K, pool);
  hipLaunchKernelGGL(conv_soft_records_kernel<ARR>, dim3((unsigned)cdiv(N * R, 256)), dim3(256),
                     0, as_stream(stream), conn, cm, ch, cw, (int)N, nleaf, K, km,
                     quad ? 1 : (pair ? 2 : (phase ? 4 : 1)), node_kind, arity, raw, (int)C,
                     2 * pad + 1, g, R, rec);
  SLG_LAUNCH_CHECK("conv_soft_records");
  return 0;
}

}  // namespace slg

using namespace slg;

extern "C" {

int slg_conv_soft_fwd(const float* x, int64_t B, int64_t C, int64_t H, int64_t W, int64_t N,
                      int32_t node_kind, int32_t depth, int32_t arity, int32_t K,
                      const float* node_param, const float* w, const int32_t* cm, const int32_t* ch,
                      const int32_t* cw, int32_t pad, int32_t pool, float* out, slg_stream_t stream) {
  SLG_REQUIRE(node_param && cm && ch && cw && ((x && out) || B == 0), SLG_E_ARG,
              "conv_soft: null pointer");
  SLG_REQUIRE(node_kind == SLG_NODE_GATE16 || node_kind == SLG_NODE_WALSH ||
                  node_kind == SLG_NODE_MULTILINEAR2 || node_kind == SLG_NODE_HYBRID,
              SLG_E_ARG, "conv_soft: node_kind %d", node_kind);
  const int nleaf = node_leaves(node_kind, depth, arity);
  const bool generic = conv_generic_supported(node_kind, depth, arity);
  SLG_REQUIRE(nleaf > 0 || generic, SLG_E_UNSUPPORTED, "conv_soft: node %d depth %d / arity %d",
              node_kind, depth, arity);
  SLG_REQUIRE(K >= 1 && K <= kMaxK, SLG_E_SHAPE, "conv_soft: K=%d outside 1..%d", K, kMaxK);
  SLG_REQUIRE(B >= 0 && C > 0 && H > 0 && W > 0 && N > 0 && pad >= 0 && pad <= 4 &&
                  B < (1LL << 31) && N < (1LL << 20) && C < (1LL << 20) && H < 4096 && W < 4096,
              SLG_E_SHAPE, "conv_soft: bad sizes");
  const int kernel = 2 * pad + 1;  // 'same' convolution, stride 1 (models.py:222)
  const int64_t Hf = H + 2 * pad - kernel + 1, Wf = W + 2 * pad - kernel + 1;
  const int64_t Ho = pool ? Hf / 2 : Hf, Wo = pool ? Wf / 2 : Wf;
  if (B == 0 || Ho == 0 || Wo == 0) return 0;
  if (nleaf > 0) {
    ConvSoftArgs a{x, B, C, H, W, N, K, kernel, pad, node_param, w, cm, ch, cw, out, Ho, Wo,
                   nullptr};
    const int rc = pool ? conv_soft_dispatch<true>(a, node_kind, nleaf, as_stream(stream))
                        : conv_soft_dispatch<false>(a, node_kind, nleaf, as_stream(stream));
    // an image that does not fit LDS goes to the generic kernel (nothing was
    // launched: the rejection comes before the launch)
    if (rc != SLG_E_UNSUPPORTED || !generic) return rc;
  }
  return conv_generic_fwd(x, B, C, H, W, N, node_kind, depth, arity, K, kernel, pad, pool != 0,
                          node_param, w, cm, ch, cw, out, Ho, Wo, as_stream(stream));
}

int slg_conv_soft_lds_fit(int64_t C, int64_t H, int64_t W, int32_t node_kind, int32_t depth,
                          int32_t arity, int32_t K, int32_t pad, int32_t pool) {
  const int nleaf = node_leaves(node_kind, depth, arity);
  if (nleaf <= 0 || K < 1 || K > kMaxK || C <= 0 || H <= 0 || W <= 0 || pad < 0 || pad > 4 ||
      C >= (1LL << 20) || H >= 4096 || W >= 4096)
    return 0;
  const int kernel = 2 * pad + 1;
  const int64_t Hf = H + 2 * pad - kernel + 1, Wf = W + 2 * pad - kernel + 1;
  const int64_t Ho = pool ? Hf / 2 : Hf, Wo = pool ? Wf / 2 : Wf;
  const int km = K <= 4 ? 4 : kMaxK;
  const ConvGeom g = conv_geom(C, H, W, pad, pool != 0, conv_phase_layout(pool != 0, nleaf, km),
                               Ho, Wo);
  const int64_t cap = std::min<int64_t>(device_lds_bytes(), 160 * 1024);
  return ((int64_t)g.SST * 4 + kConvExtra * 4 <= cap && C * H * W * 4 < (1LL << 31)) ? 1 : 0;
}

int64_t slg_conv_soft_record_floats(int32_t node_kind, int32_t depth, int32_t arity, int32_t K,
                                    int32_t pool) {
  const int nleaf = node_leaves(node_kind, depth, arity);
  if (nleaf <= 0 || K < 1 || K > kMaxK) return -1;
  const int km = K <= 4 ? 4 : kMaxK;
  const int nw = conv_phase_layout(pool != 0, nleaf, km) ? 4 : 1;
  const int npr = node_kind == SLG_NODE_GATE16 ? 4 * (nleaf - 1) : (1 << nleaf);
  return (nleaf * km * (nw + 1) + npr + 3) & ~3;
}

int slg_conv_soft_records(const float* conn, const int32_t* cm, const int32_t* ch,
                          const int32_t* cw, int64_t N, int32_t K, int32_t node_kind, int32_t depth,
                          int32_t arity, const float* raw, int64_t C, int64_t H, int64_t W,
                          int32_t pad, int32_t pool, float* rec, slg_stream_t stream) {
  return conv_records_launch<false>(conn, cm, ch, cw, N, K, node_kind, depth, arity, raw, C, H, W,
                                    pad, pool, rec, stream);
}

int slg_conv_soft_records_arrays(const float* node_param, const float* w, const int32_t* cm,
                                 const int32_t* ch, const int32_t* cw, int64_t N, int32_t K,
                                 int32_t node_kind, int32_t depth, int32_t arity, int64_t C,
                                 int64_t H, int64_t W, int32_t pad, int32_t pool, float* rec,
                                 slg_stream_t stream) {
  SLG_REQUIRE(node_kind == SLG_NODE_GATE16 || node_kind == SLG_NODE_MULTILINEAR2 ||
                  node_kind == SLG_NODE_HYBRID,
              SLG_E_ARG, "conv_soft_records_arrays: node_kind %d", node_kind);
  return conv_records_launch<true>(w, cm, ch, cw, N, K, node_kind, depth, arity, node_param, C,
                                   H, W, pad, pool, rec, stream);
}

int slg_conv_soft_fwd_records(const float* x, int64_t B, int64_t C, int64_t H, int64_t W,
                              int64_t N, int32_t node_kind, int32_t depth, int32_t arity, int32_t K,
                              const float* rec, int32_t pad, int32_t pool, float* out,
                              slg_stream_t stream) {
  SLG_REQUIRE(rec && ((x && out) || B == 0), SLG_E_ARG, "conv_soft_records: null pointer");
  SLG_REQUIRE(node_kind == SLG_NODE_GATE16 || node_kind == SLG_NODE_MULTILINEAR2 ||
                  node_kind == SLG_NODE_HYBRID,
              SLG_E_ARG, "conv_soft: node_kind %d", node_kind);
  const int nleaf = node_leaves(node_kind, depth, arity);
  SLG_REQUIRE(nleaf > 0, SLG_E_UNSUPPORTED, "conv_soft: depth %d / arity %d", depth, arity);
  SLG_REQUIRE(K >= 1 && K <= kMaxK, SLG_E_SHAPE, "conv_soft: K=%d outside 1..%d", K, kMaxK);
  SLG_REQUIRE(B >= 0 && C > 0 && H > 0 && W > 0 && N > 0 && pad >= 0 && pad <= 4 &&
                  B < (1LL << 31) && N < (1LL << 20) && C < (1LL << 20) && H < 4096 && W < 4096,
              SLG_E_SHAPE, "conv_soft: bad sizes");
  const int kernel = 2 * pad + 1;
  const int64_t Hf = H + 2 * pad - kernel + 1, Wf = W + 2 * pad - kernel + 1;
  const int64_t Ho = pool ? Hf / 2 : Hf, Wo = pool ? Wf / 2 : Wf;
  if (B == 0 || Ho == 0 || Wo == 0) return 0;
  ConvSoftArgs a{x, B, C, H, W, N, K, kernel, pad, nullptr, nullptr, nullptr, nullptr, nullptr,
                 out, Ho, Wo, rec};
  return pool ? conv_soft_dispatch<true>(a, node_kind, nleaf, as_stream(stream))
              : conv_soft_dispatch<false>(a, node_kind, nleaf, as_stream(stream));
}

int slg_tree_conv_fwd(const float* x, int64_t B, int64_t C, int64_t H, int64_t W, int64_t N,
                      int32_t depth, int32_t K, const float* coef, const float* w, const int32_t* cm,
                      const int32_t* ch, const int32_t* cw, int32_t stride, int32_t pad, int64_t Ho,
                      int64_t Wo, float* out, slg_stream_t stream) {
  SLG_REQUIRE(stride == 1, SLG_E_UNSUPPORTED, "tree_conv: stride %d (only 1)", stride);
  SLG_REQUIRE(Ho == H && Wo == W, SLG_E_UNSUPPORTED,
              "tree_conv: only 'same' convolutions (kernel = 2*pad+1) are supported");
  return slg_conv_soft_fwd(x, B, C, H, W, N, SLG_NODE_GATE16, depth, 2, K, coef, w, cm, ch, cw,
                           pad, 0, out, stream);
}

int slg_conv_soft_prep(const float* conn, int64_t N, int32_t leaves, int32_t K, int32_t node_kind,
                       int32_t depth, int32_t arity, const float* raw, float* w, float* node_param,
                       slg_stream_t stream) {
  SLG_REQUIRE(raw && w && node_param, SLG_E_ARG, "conv_soft_prep: null pointer");
  const int nleaf = node_leaves(node_kind, depth, arity);
  SLG_REQUIRE(nleaf > 0 && nleaf == leaves, SLG_E_UNSUPPORTED, "conv_soft_prep: leaves %d", leaves);
  SLG_REQUIRE(N > 0 && N < (1LL << 31) && K >= 1 && K <= 64, SLG_E_SHAPE, "conv_soft_prep: sizes");
  hipLaunchKernelGGL(conv_soft_prep_kernel, dim3((unsigned)cdiv(N, 128)), dim3(128), 0,
                     as_stream(stream), conn, (int)N, leaves, K, node_kind, nleaf - 1, arity, raw, w,
                     node_param);
  SLG_LAUNCH_CHECK("conv_soft_prep");
  return 0;
}

static int conv_prep_block(ConvPrepBlock& P, const int32_t* cm, const int32_t* ch,
                           const int32_t* cw, const float* conn, int64_t N, int32_t K,
                           int32_t node_kind, int32_t depth, int32_t arity, int32_t* leaf,
                           uint64_t* tt) {
  SLG_REQUIRE(cm && ch && cw && leaf && tt, SLG_E_ARG, "conv_hard_prep: null pointer");
  const int nleaf = node_leaves(node_kind, depth, arity);
  SLG_REQUIRE(nleaf > 0, SLG_E_UNSUPPORTED, "conv_hard_prep: depth %d / arity %d", depth, arity);
  SLG_REQUIRE(N > 0 && N < (1LL << 31) && N * nleaf < (1LL << 31) && K >= 1 && K <= 64,
              SLG_E_SHAPE, "conv_hard_prep: sizes");
  P = ConvPrepBlock{};
  P.cm = cm;
  P.ch = ch;
  P.cw = cw;
  P.conn = conn;
  P.leaf = leaf;
  P.tt = tt;
  P.N = (int)N;
  P.leaves = nleaf;
  P.K = K;
  P.node = node_kind;
  P.depth = depth;
  P.arity = arity;
  return 0;
}

static int launch_conv_prep(ConvPrepNet& net, hipStream_t stream) {
  int blocks = 0;
  for (int k = 0; k < net.n; ++k) {
    net.blk_start[k] = blocks;
    blocks += (int)cdiv(net.b[k].N, 128);
  }
  net.blk_start[net.n] = blocks;
  hipLaunchKernelGGL(conv_hard_prep_kernel, dim3((unsigned)blocks), dim3(128), 0, stream, net);
  SLG_LAUNCH_CHECK("conv_hard_prep");
  return 0;
}

int slg_conv_hard_prep(const int32_t* cm, const int32_t* ch, const int32_t* cw, const float* conn,
                       int64_t N, int32_t leaves, int32_t K, int32_t node_kind, int32_t depth,
                       int32_t arity, const float* raw, int32_t* leaf, uint64_t* tt,
                       slg_stream_t stream) {
  SLG_REQUIRE(raw, SLG_E_ARG, "conv_hard_prep: null pointer");
  ConvPrepNet net{};
  net.n = 1;
  ConvPrepBlock& P = net.b[0];
  if (int rc = conv_prep_block(P, cm, ch, cw, conn, N, K, node_kind, depth, arity, leaf, tt))
    return rc;
  SLG_REQUIRE(leaves == P.leaves, SLG_E_UNSUPPORTED, "conv_hard_prep: leaves %d", leaves);
  if (node_kind == SLG_NODE_GATE16) {
    // concatenated levels [N, 2^depth - 1, 16]: level l starts after the
    // 2^depth - 2^(depth-l) nodes of the levels before it
    const int nodes = P.leaves - 1;
    for (int lv = 0; lv < depth; ++lv) {
      P.raw[lv] = raw + (int64_t)16 * (P.leaves - (P.leaves >> lv));
      P.rstride[lv] = nodes * 16;
    }
  } else {
    P.raw[0] = raw;
    P.rstride[0] = 1 << arity;
  }
  return launch_conv_prep(net, as_stream(stream));
}

int slg_conv_hard_prep_net(int32_t n_blocks, const int32_t* const* cm, const int32_t* const* ch,
                           const int32_t* const* cw, const float* const* conn,
                           const float* const* raw, const int64_t* N, const int32_t* K,
                           const int32_t* node_kind, const int32_t* depth, const int32_t* arity,
                           int32_t* const* leaf, uint64_t* const* tt, slg_stream_t stream) {
  SLG_REQUIRE(n_blocks >= 1 && n_blocks <= kMaxConvPrepBlocks, SLG_E_SHAPE,
              "conv_hard_prep_net: %d blocks outside 1..%d", n_blocks, kMaxConvPrepBlocks);
  SLG_REQUIRE(cm && ch && cw && conn && raw && N && K && node_kind && depth && arity && leaf && tt,
              SLG_E_ARG, "conv_hard_prep_net: null array");
  ConvPrepNet net{};
  net.n = n_blocks;
  int64_t total = 0;
  for (int k = 0; k < n_blocks; ++k) {
    ConvPrepBlock& P = net.b[k];
    if (int rc = conv_prep_block(P, cm[k], ch[k], cw[k], conn[k], N[k], K[k], node_kind[k],
                                 depth[k], arity[k], leaf[k], tt[k]))
      return rc;
    total += cdiv(N[k], 128);
    const float* const* r = raw + 4 * k;
    if (node_kind[k] == SLG_NODE_GATE16) {
      for (int lv = 0; lv < depth[k]; ++lv) {
        SLG_REQUIRE(r[lv], SLG_E_ARG, "conv_hard_prep_net: block %d level %d logits null", k, lv);
        P.raw[lv] = r[lv];
        P.rstride[lv] = 16 << (depth[k] - 1 - lv);
      }
    } else {
      SLG_REQUIRE(r[0], SLG_E_ARG, "conv_hard_prep_net: block %d logits null", k);
      P.raw[0] = r[0];
      P.rstride[0] = 1 << arity[k];
    }
  }
  SLG_REQUIRE(total < (1LL << 31), SLG_E_SHAPE, "conv_hard_prep_net: sizes");
  return launch_conv_prep(net, as_stream(stream));
}

int slg_conv_hard_fwd(const uint64_t* xp, int64_t C, int64_t H, int64_t W, int64_t nw, int64_t N,
                      int32_t node_kind, int32_t depth, int32_t arity, const int32_t* leaf,
                      const uint64_t* tt, int32_t kernel, int32_t pad, int32_t pool, uint64_t* out,
                      slg_stream_t stream) {
  SLG_REQUIRE(leaf && tt && ((xp && out) || nw == 0), SLG_E_ARG, "conv_hard: null pointer");
  const int nleaf = node_leaves(node_kind, depth, arity);
  SLG_REQUIRE(nleaf > 0, SLG_E_UNSUPPORTED, "conv_hard: depth %d / arity %d", depth, arity);
  SLG_REQUIRE(C > 0 && H > 0 && W > 0 && nw >= 0 && N > 0 && kernel >= 1 && kernel <= 15 &&
                  pad >= 0 && H < 4096 && W < 4096 && C < (1LL << 23),
              SLG_E_SHAPE, "conv_hard: bad sizes");
  const int64_t Hf = H + 2 * pad - kernel + 1, Wf = W + 2 * pad - kernel + 1;
  SLG_REQUIRE(Hf > 0 && Wf > 0, SLG_E_SHAPE, "conv_hard: empty output");
  const int64_t Ho = pool ? Hf / 2 : Hf, Wo = pool ? Wf / 2 : Wf;
  if (nw == 0 || Ho == 0 || Wo == 0) return 0;
  hipStream_t st = as_stream(stream);
  return pool ? conv_hard_dispatch<true>(node_kind, nleaf, xp, C, H, W, nw, N, leaf, tt, kernel,
                                         pad, out, Ho, Wo, st)
              : conv_hard_dispatch<false>(node_kind, nleaf, xp, C, H, W, nw, N, leaf, tt, kernel,
                                          pad, out, Ho, Wo, st);
}

int slg_orpool(const void* x, int32_t dtype, int64_t B, int64_t C, int64_t H, int64_t W,
               int32_t size, void* out, slg_stream_t stream) {
  SLG_REQUIRE((x && out) || B == 0, SLG_E_ARG, "orpool: null pointer");
  SLG_REQUIRE(dtype == 0 || dtype == 1, SLG_E_ARG, "orpool: dtype %d", dtype);
  SLG_REQUIRE(size >= 1 && size <= 64, SLG_E_SHAPE, "orpool: size %d", size);
  SLG_REQUIRE(B >= 0 && C > 0 && H > 0 && W > 0 && B * C * H * W < (1LL << 46), SLG_E_SHAPE,
              "orpool: bad sizes");
  const int64_t n = B * C * (H / size) * (W / size);
  if (n == 0) return 0;
  if (dtype == 0)
    hipLaunchKernelGGL(orpool_kernel<float>, dim3((unsigned)cdiv(n, 256)), dim3(256), 0,
                       as_stream(stream), (const float*)x, B * C, (int)H, (int)W, (int)size,
                       (float*)out);
  else
    hipLaunchKernelGGL(orpool_kernel<uint8_t>, dim3((unsigned)cdiv(n, 256)), dim3(256), 0,
                       as_stream(stream), (const uint8_t*)x, B * C, (int)H, (int)W, (int)size,
                       (uint8_t*)out);
  SLG_LAUNCH_CHECK("orpool");
  return 0;
}

}  // extern "C"
