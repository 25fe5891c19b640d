// Bit-packed hard path for gfx950: packing, hard-parameter prep, packed FC
// layers, the depth-fused FC network with its GroupSum popcount, and the
// packed GroupSum.
//
// Packed words carry 64 samples (one wavefront ballot). A gate16 node on two
// words is three bit-field-inserts per 32-bit half:
//   out = bfi(a, bfi(b, T3, T2), bfi(b, T1, T0)),  T_g = tt bit g ? ~0 : 0,
// so one output word costs the same whatever the gate, with no branching.
#include <type_traits>

#include "fc_net.h"
#include "pack_cols.h"
#include "slg_common.h"

namespace slg {

template <typename WT>
__device__ inline WT gate_word(WT a, WT b, uint32_t tt) {
  // T_g = all-ones iff tt bit g (sign-extending 1-bit field extract; the
  // builtin's result type is unsigned, so widen through int)
  const WT t0 = (WT)(int64_t)(int)__builtin_amdgcn_sbfe((int)tt, 0, 1);
  const WT t1 = (WT)(int64_t)(int)__builtin_amdgcn_sbfe((int)tt, 1, 1);
  const WT t2 = (WT)(int64_t)(int)__builtin_amdgcn_sbfe((int)tt, 2, 1);
  const WT t3 = (WT)(int64_t)(int)__builtin_amdgcn_sbfe((int)tt, 3, 1);
  const WT hi = (b & t3) | (~b & t2);  // a = 1: addresses 3 (b=1), 2 (b=0)
  const WT lo = (b & t1) | (~b & t0);  // a = 0: addresses 1 (b=1), 0 (b=0)
  return (a & hi) | (~a & lo);
}

// 64x64 bit transpose across a wavefront: lane r holds row r; afterwards
// lane r holds column r (bit c of the result = bit r of lane c's input).
// Stage s swaps bit s of the row index with bit s of the column index.
__device__ inline uint64_t transpose64(uint64_t v, int lane) {
  const uint64_t masks[6] = {0x00000000FFFFFFFFull, 0x0000FFFF0000FFFFull,
                             0x00FF00FF00FF00FFull, 0x0F0F0F0F0F0F0F0Full,
                             0x3333333333333333ull, 0x5555555555555555ull};
#pragma unroll
  for (int i = 0; i < 6; ++i) {
    const int s = 32 >> i;
    const uint64_t m = masks[i];
    const uint32_t lo = __shfl_xor((uint32_t)v, s);
    const uint32_t hi = __shfl_xor((uint32_t)(v >> 32), s);
    const uint64_t other = ((uint64_t)hi << 32) | lo;
    if (lane & s) v = (v & ~m) | ((other & ~m) >> s);
    else v = (v & m) | ((other & m) << s);
  }
  return v;
}

// ---------------------------------------------------------------------------
// pack / unpack
// ---------------------------------------------------------------------------
// A lane takes V consecutive features and builds their 64-sample words in
// registers (pack_cols); the four waves of a workgroup take four consecutive
// words. A feature's bit is (x >= 1) for fp32, (x != 0) for bytes. V = 4
// reads four features of a row as one vector (D % 4 == 0, aligned input).
// LAYOUT 0 writes the reference layout [D][nw]; LAYOUT 1 writes word-major
// [nw][D], where one 64-sample column of all features is contiguous (the
// fused network kernel's input).
template <typename T, int LAYOUT, int V>
__global__ void __launch_bounds__(256) pack_kernel(const T* __restrict__ x, int B, int D, int nw,
                                                   int dtiles, uint64_t* __restrict__ xp) {
  const int lane = threadIdx.x & 63;
  const int w = (int)(blockIdx.x / (uint32_t)dtiles) * 4 + (int)(threadIdx.x >> 6);
  const int d0 = (int)(blockIdx.x % (uint32_t)dtiles) * 64 * V + lane * V;
  if (w >= nw || d0 >= D) return;                       // no barriers below
  int src[V];
#pragma unroll
  for (int v = 0; v < V; ++v) src[v] = min(d0 + v, D - 1);  // tail lanes: stores are guarded
  uint64_t word[V];
  pack_cols<V, V == 4>(x + (int64_t)w * 64 * D, D, min(64, B - w * 64), src,
                       [](T v, int) {
                         if constexpr (sizeof(T) == 1) return v != 0;
                         else return v >= (T)1;
                       },
                       word);
#pragma unroll
  for (int v = 0; v < V; ++v) {
    if (d0 + v < D) {
      if constexpr (LAYOUT == 0) xp[(int64_t)(d0 + v) * nw + w] = word[v];
      else xp[(int64_t)w * D + d0 + v] = word[v];
    }
  }
}

__global__ void __launch_bounds__(256) unpack_kernel(const uint64_t* __restrict__ xp, int B, int D,
                                                     int nw, uint8_t* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)B * D) return;
  const int b = (int)(i / D), d = (int)(i % D);
  out[i] = (uint8_t)((xp[(int64_t)d * nw + (b >> 6)] >> (b & 63)) & 1ull);
}

// ---------------------------------------------------------------------------
// hard parameter prep (FC)
// ---------------------------------------------------------------------------
// TRUTH_TABLES of silogic/functional.py:50-69 as 4-bit codes (bit g = output
// at address g = (a<<1)|b): code = c0 | (c0+c2)<<1 | (c0+c1)<<2 | (sum)<<3.
__constant__ uint8_t c_tt16[16] = {0x0, 0x8, 0x4, 0xC, 0x2, 0xA, 0x6, 0xE,
                                   0x1, 0x9, 0x5, 0xD, 0x3, 0xB, 0x7, 0xF};

__device__ inline int argmax_first(const float* p, int n) {
  int bi = 0;
  float bv = p[0];
  for (int i = 1; i < n; ++i)
    if (p[i] > bv) { bv = p[i]; bi = i; }
  return bi;
}

// Hard code of output o: wiring by argmax over the K candidates (first index
// on ties), truth table of the node, indices clamped into [0, IN).
__device__ inline uint2 hard_code(const int32_t* __restrict__ cand, const float* __restrict__ conn,
                                  int o, int K, int IN, int node, const float* __restrict__ raw) {
  int idx[2];
  for (int s = 0; s < 2; ++s) {
    if (conn) {  // TopK: cand[o, s, argmax conn[o, s, :]] (connectomes.py:129-132)
      const int64_t base = ((int64_t)o * 2 + s) * K;
      idx[s] = cand[base + argmax_first(conn + base, K)];
    } else {     // fixed: idx[o, s]
      idx[s] = cand[(int64_t)o * 2 + s];
    }
    idx[s] = min(max(idx[s], 0), IN - 1);
  }
  uint32_t tt = 0;
  if (node == SLG_NODE_GATE16) {  // nodes.py:100-106
    tt = c_tt16[argmax_first(raw + (int64_t)o * 16, 16)];
  } else if (node == SLG_NODE_WALSH) {
    // nodes.py:152-156: z = ((t0*1 + t1*u0) + t2*u1) + t3*u0*u1, u = 2x-1,
    // summed left to right in fp32 as torch's CPU sum over the size-4 dim.
    const float t0 = raw[o * 4 + 0], t1 = raw[o * 4 + 1], t2 = raw[o * 4 + 2], t3 = raw[o * 4 + 3];
    for (int g = 0; g < 4; ++g) {
      const float u0 = (g >> 1) ? 1.0f : -1.0f;  // a
      const float u1 = (g & 1) ? 1.0f : -1.0f;   // b
      float z = t0;  // products by +-1 are exact, so contraction cannot change z
      z = z + t1 * u0;
      z = z + t2 * u1;
      z = z + t3 * (u0 * u1);
      if (z > 0.0f) tt |= 1u << g;
    }
  } else {  // multilinear arity 2: bit g = logits[a + 2b] > 0 (nodes.py:183-189)
    for (int g = 0; g < 4; ++g) {
      const int a = g >> 1, b = g & 1;
      if (raw[o * 4 + a + 2 * b] > 0.0f) tt |= 1u << g;
    }
  }
  return make_uint2((uint32_t)idx[0], (uint32_t)idx[1] | (tt << 28));
}

__global__ void fc_hard_prep_kernel(const int32_t* __restrict__ cand, const float* __restrict__ conn,
                                    int OUT, int K, int IN, int node, const float* __restrict__ raw,
                                    uint2* __restrict__ codes) {
  const int o = blockIdx.x * blockDim.x + threadIdx.x;
  if (o >= OUT) return;
  codes[o] = hard_code(cand, conn, o, K, IN, node, raw);
}

// Codes of several layers in one launch; each workgroup serves one layer.
constexpr int kMaxPrepLayers = 16;
constexpr int kMaxCompactIn = 1 << 14;
struct HardPrepLayer {
  const int32_t* cand;
  const float* conn;
  const float* raw;
  uint2* codes;
  int in_dim, out_dim, K, node;
  int vec;  // parameters 16-byte aligned: the K = 8 path may use vector loads
};
struct HardPrepNet {
  HardPrepLayer L[kMaxPrepLayers];
  int blk_start[kMaxPrepLayers + 1];
  int n;
};

// Compact code of the depth-fused network (inputs at most 16384 wide):
// b | a << 14 | tt << 28, 4 bytes per output.
__device__ inline uint32_t compact_code(uint2 c) {
  return (c.y & 0x3FFFu) | ((c.x & 0x3FFFu) << 14) | (c.y & 0xF0000000u);
}

// hard_code for TopK layers with K = 8, every parameter of the output loaded
// before any is used (16-byte loads: 2 x 8 candidates, 2 x 8 connection
// logits, the node's 16 or 4 parameters), instead of a load per step of the
// argmax loops. Same argmax (first index on ties), truth table and clamp.
__device__ inline uint2 hard_code_k8(const int32_t* __restrict__ cand,
                                     const float* __restrict__ conn, int o, int IN, int node,
                                     const float* __restrict__ raw) {
  const int4* c4 = reinterpret_cast<const int4*>(cand + (int64_t)o * 16);
  const float4* f4 = reinterpret_cast<const float4*>(conn + (int64_t)o * 16);
  const int4 ca[4] = {c4[0], c4[1], c4[2], c4[3]};
  const float4 cf[4] = {f4[0], f4[1], f4[2], f4[3]};
  float r[16];
  if (node == SLG_NODE_GATE16) {
    const float4* r4 = reinterpret_cast<const float4*>(raw + (int64_t)o * 16);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float4 t = r4[q];
      r[4 * q] = t.x; r[4 * q + 1] = t.y; r[4 * q + 2] = t.z; r[4 * q + 3] = t.w;
    }
  } else {
    const float4 t = reinterpret_cast<const float4*>(raw + (int64_t)o * 4)[0];
    r[0] = t.x; r[1] = t.y; r[2] = t.z; r[3] = t.w;
#pragma unroll
    for (int i = 4; i < 16; ++i) r[i] = 0.0f;
  }
  int idx[2];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const float c[8] = {cf[2 * s].x, cf[2 * s].y, cf[2 * s].z, cf[2 * s].w,
                        cf[2 * s + 1].x, cf[2 * s + 1].y, cf[2 * s + 1].z, cf[2 * s + 1].w};
    int k[8] = {ca[2 * s].x, ca[2 * s].y, ca[2 * s].z, ca[2 * s].w,
                ca[2 * s + 1].x, ca[2 * s + 1].y, ca[2 * s + 1].z, ca[2 * s + 1].w};
    // opaque values: the select stays a register select instead of an
    // indexed read of a stack copy of k
#pragma unroll
    for (int i = 0; i < 8; ++i) asm volatile("" : "+v"(k[i]));
    float bv = c[0];
    int bi = k[0];
#pragma unroll
    for (int i = 1; i < 8; ++i)
      if (c[i] > bv) { bv = c[i]; bi = k[i]; }
    idx[s] = min(max(bi, 0), IN - 1);
  }
  uint32_t tt = 0;
  if (node == SLG_NODE_GATE16) {
    float bv = r[0];
    int bi = 0;
#pragma unroll
    for (int i = 1; i < 16; ++i)
      if (r[i] > bv) { bv = r[i]; bi = i; }
    tt = c_tt16[bi];
  } else if (node == SLG_NODE_WALSH) {  // as hard_code
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const float u0 = (g >> 1) ? 1.0f : -1.0f, u1 = (g & 1) ? 1.0f : -1.0f;
      float z = r[0];
      z = z + r[1] * u0;
      z = z + r[2] * u1;
      z = z + r[3] * (u0 * u1);
      if (z > 0.0f) tt |= 1u << g;
    }
  } else {
#pragma unroll
    for (int g = 0; g < 4; ++g)
      if (r[(g >> 1) + 2 * (g & 1)] > 0.0f) tt |= 1u << g;
  }
  return make_uint2((uint32_t)idx[0], (uint32_t)idx[1] | (tt << 28));
}

__global__ void __launch_bounds__(256) fc_hard_prep_net_kernel(HardPrepNet net, int compact) {
  int l = 0;
  while (l + 1 < net.n && (int)blockIdx.x >= net.blk_start[l + 1]) ++l;
  const HardPrepLayer& L = net.L[l];
  const int o = ((int)blockIdx.x - net.blk_start[l]) * blockDim.x + threadIdx.x;
  if (o >= L.out_dim) return;
  const uint2 c = (L.K == 8 && L.conn && L.vec)
                      ? hard_code_k8(L.cand, L.conn, o, L.in_dim, L.node, L.raw)
                      : hard_code(L.cand, L.conn, o, L.K, L.in_dim, L.node, L.raw);
  if (compact) reinterpret_cast<uint32_t*>(L.codes)[o] = compact_code(c);
  else L.codes[o] = c;
}

// ---------------------------------------------------------------------------
// one packed FC layer
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256) fc_hard_layer_kernel(const uint64_t* __restrict__ xin, int nw,
                                                            const uint2* __restrict__ codes, int OUT,
                                                            uint64_t* __restrict__ xout) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)OUT * nw) return;
  const int o = (int)(i / nw), w = (int)(i % nw);
  const uint2 c = codes[o];
  const uint64_t a = xin[(int64_t)c.x * nw + w];
  const uint64_t b = xin[(int64_t)(c.y & 0x0FFFFFFFu) * nw + w];
  xout[i] = gate_word<uint64_t>(a, b, c.y >> 28);
}


// One-layer networks at small batches (a conv network's head on a few
// sample words): the fused kernel's one workgroup per word would leave most
// CUs idle and stage every input word in LDS although each gate reads two.
// Here workgroup (w, c) evaluates the G = W / C gates of class c on word w
// straight from the packed words in memory, writes them to LDS and counts
// them as the fused kernel's GroupSum does (class_count, wave 0): nw * C
// workgroups, the logits the same integers. Codes: compact codes in index
// order, or (type-placed, with a plan) stored thread-major at TM slots per
// thread, output o at (o % 1024) * TM + o / 1024. (Two-layer heads, layer 0
// evaluated per workgroup from memory, measured no faster than the fused
// kernel at config 3's head and are left to it.)
template <int LAYOUT>
__global__ void __launch_bounds__(kHeadThreads)
fc_hard_head_kernel(const uint64_t* __restrict__ xp, int B, int nw, int in0, int G, int C,
                    const uint32_t* __restrict__ codes, int tm, const int32_t* plan,
                    float* __restrict__ logits) {
  extern __shared__ __align__(16) unsigned char smem[];
  uint64_t* cls = reinterpret_cast<uint64_t*>(smem);
  const int w = blockIdx.x, c = blockIdx.y;
  if (plan && !plan_fits(plan, tm, in0)) {   // typed codes placed for another layout
    if (threadIdx.x < 64 && w * 64 + (int)threadIdx.x < B)
      logits[(int64_t)(w * 64 + threadIdx.x) * C + c] = __int_as_float(0x7FC00000);
    return;
  }
  for (int i = threadIdx.x; i < G; i += kHeadThreads) {
    const int o = c * G + i;
    const uint32_t code = codes[tm ? (o & (kNetThreads - 1)) * tm + (o >> 10) : o];
    // the prep keeps operands below the width; a read never leaves it
    const int a = min((int)((code >> 14) & 0x3FFFu), in0 - 1);
    const int b = min((int)(code & 0x3FFFu), in0 - 1);
    const uint64_t va = LAYOUT == 0 ? xp[(int64_t)a * nw + w] : xp[(int64_t)w * in0 + a];
    const uint64_t vb = LAYOUT == 0 ? xp[(int64_t)b * nw + w] : xp[(int64_t)w * in0 + b];
    cls[i] = gate_compact<uint64_t>(va, vb, code);
  }
  __syncthreads();
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    const int n = class_count<2>(reinterpret_cast<const uint32_t*>(cls), G, lane);
    const int b = w * 64 + lane;
    if (b < B) logits[(int64_t)b * C + c] = (float)n;
  }
}

static int launch_head(const uint64_t* xp, int in_kind, int64_t B, int64_t IN0, int64_t width,
                       int C, const uint32_t* codes, int tm, const int32_t* plan, float* logits,
                       hipStream_t st) {
  const int64_t nw = cdiv(B, 64);
  const int G = (int)(width / C);
  auto kern = in_kind == 2 ? fc_hard_head_kernel<0> : fc_hard_head_kernel<1>;
  hipLaunchKernelGGL(kern, dim3((unsigned)nw, (unsigned)C), dim3(kHeadThreads), (size_t)G * 8, st,
                     xp, (int)B, (int)nw, (int)IN0, G, C, codes, tm, plan, logits);
  SLG_LAUNCH_CHECK("fc_hard_head");
  return 0;
}

// A row element's bit: x >= 1 for fp32, x != 0 for bytes.
template <typename IT>
__device__ inline bool input_bit(IT v) {
  if constexpr (sizeof(IT) == 1) return v != 0;
  else return v >= (IT)1;
}

// One element of a row through a buffer resource (offsets past it read 0).
template <typename IT>
__device__ inline IT load_row(__amdgpu_buffer_rsrc_t r, int voff) {
  if constexpr (sizeof(IT) == 1) return (IT)__builtin_amdgcn_raw_buffer_load_b8(r, voff, 0, 0);
  else return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, voff, 0, 0));
}

// The tile's rows [B][in0] (fp32: bit = x >= 1; bytes: bit = x != 0) packed
// into LDS words, sample b0 + s at bit s: thread t builds the words of
// features 4t + 4096k from 4-feature vectors (16 bytes of fp32, 4 bytes of
// uint8; in0 % 4 == 0 and an aligned row pointer), else of features
// t + 1024k one at a time, RB rows in flight. The rows are read through a
// buffer resource spanning the tile's samples that exist: rows past it
// read 0, bit 0, with no clamp or branch.
template <typename IT, typename WT>
__device__ __forceinline__ void rows_to_lds(WT* lds, const IT* __restrict__ x, int B, int in0,
                                            int b0) {
  constexpr int SPW = (int)sizeof(WT) * 8;
  constexpr int RB = 16;
  const int nr = max(0, min(SPW, B - b0));
  const int rowb = in0 * (int)sizeof(IT);
  const __amdgpu_buffer_rsrc_t r =
      uniform_rsrc(x + (int64_t)min(b0, B) * in0, nr * rowb);
  const bool vec = in0 % 4 == 0 && (uintptr_t)x % (4 * sizeof(IT)) == 0;
  if (vec) {
    for (int f = threadIdx.x * 4; f < in0; f += 4 * kNetThreads) {
      WT w[4] = {0, 0, 0, 0};
      const int v0 = f * (int)sizeof(IT);
#pragma unroll
      for (int c = 0; c < SPW; c += RB) {
        uint32_t m[4] = {0u, 0u, 0u, 0u};
        if constexpr (sizeof(IT) == 4) {
          typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
          u32x4 q[RB];
#pragma unroll
          for (int i = 0; i < RB; ++i)
            q[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, v0 + (c + i) * rowb, 0, 0));
#pragma unroll
          for (int i = RB - 1; i >= 0; --i) {
#pragma unroll
            for (int v = 0; v < 4; ++v)
              m[v] = (m[v] << 1) | (__uint_as_float(q[i][v]) >= 1.0f ? 1u : 0u);
          }
        } else {
          uint32_t q[RB];
#pragma unroll
          for (int i = 0; i < RB; ++i) q[i] = __builtin_amdgcn_raw_buffer_load_b32(r, v0 + (c + i) * rowb, 0, 0);
#pragma unroll
          for (int i = RB - 1; i >= 0; --i) {
#pragma unroll
            for (int v = 0; v < 4; ++v) m[v] = (m[v] << 1) | (((q[i] >> (8 * v)) & 0xFFu) ? 1u : 0u);
          }
        }
#pragma unroll
        for (int v = 0; v < 4; ++v) w[v] |= (WT)m[v] << c;
      }
#pragma unroll
      for (int v = 0; v < 4; ++v) lds[f + v] = w[v];
    }
  } else {
    for (int f = threadIdx.x; f < in0; f += kNetThreads) {
      WT w = 0;
      const int v0 = f * (int)sizeof(IT);
#pragma unroll
      for (int c = 0; c < SPW; c += RB) {
        IT q[RB];
#pragma unroll
        for (int i = 0; i < RB; ++i) q[i] = load_row<IT>(r, v0 + (c + i) * rowb);
        uint32_t m = 0;
#pragma unroll
        for (int i = RB - 1; i >= 0; --i) m = (m << 1) | (input_bit(q[i]) ? 1u : 0u);
        w |= (WT)m << c;
      }
      lds[f] = w;
    }
  }
}

// Input: LAYOUT 0 = packed [in0][nw] (reference layout), 1 = packed
// [nw][in0], 2 = fp32 rows [B][in0], 3 = uint8 rows (packed per tile here,
// for inputs the streaming rows kernel does not take: more than 1024
// features or 32-sample tiles).
template <int LAYOUT, typename WT, int MAXO, bool TYPED>
__global__ void __launch_bounds__(kNetThreads)
fc_hard_net_packed_kernel(NetDesc desc, const void* __restrict__ xin, int B, int nw,
                          float* __restrict__ logits) {
  const_netdesc_t& d = *(const_netdesc_t*)__builtin_amdgcn_kernarg_segment_ptr();
  constexpr int SPW = (int)sizeof(WT) * 8;
  if constexpr (TYPED) {
    if (!plan_fits(d.plan, MAXO, d.in0)) {
      nan_logits(logits, B, d.C);
      return;
    }
  }
  extern __shared__ __align__(16) unsigned char smem[];
  WT* lds = reinterpret_cast<WT*>(smem);
  const int tile = blockIdx.x;
  uint32_t cb[MAXO];
  if constexpr (TYPED) load_codes_tm(cb, d.codes[0]);
  else load_codes(cb, d.codes[0], d.width[0]);
  if constexpr (LAYOUT >= 2) {
    using IT = std::conditional_t<LAYOUT == 2, float, uint8_t>;
    rows_to_lds<IT, WT>(lds, (const IT*)xin, B, d.in0, tile * SPW);
  } else {
    const uint64_t* xp = (const uint64_t*)xin;
    const int w64 = tile / (64 / SPW);
    for (int i = threadIdx.x; i < d.in0; i += kNetThreads) {
      const uint64_t word = LAYOUT == 0 ? xp[(int64_t)i * nw + w64] : xp[(int64_t)w64 * d.in0 + i];
      if constexpr (SPW == 64) lds[i] = (WT)word;
      else lds[i] = (WT)(word >> (32 * (tile & 1)));
    }
  }
  __syncthreads();
  net_tile_layers<WT, MAXO, TYPED>(d, lds, cb, tile, B, logits);
}

// Unpacked rows [B][in0] (fp32, or uint8) with the packing fused: thread f
// owns feature f (in0 <= 1024) and builds its 64-sample word with coalesced
// row reads (lanes = consecutive features). Workgroups are persistent; the
// next tile's rows stream in during the current tile's layers: layer l
// issues chunk l (spl samples) and folds chunk l-2, so each chunk has two
// layers of time to arrive from HBM; chunks are issued after the layer's
// code prefetch so that waiting for codes never waits for input bytes
// (vector loads retire in order). The rows are read through a raw buffer
// resource spanning the tile's samples that exist: the hardware returns 0
// for any offset past it (the padding samples of the last tile read as 0,
// bit 0), so the loads need no clamps or branches.
// The tile's rows as a wave-uniform buffer resource.
template <typename IT>
__device__ inline __amdgpu_buffer_rsrc_t tile_rows(const IT* x, int B, int in0, int b0) {
  const int64_t rows = max(0, min(64, B - b0));
  return uniform_rsrc(x + (int64_t)min(b0, B) * in0, (int)(rows * in0 * (int64_t)sizeof(IT)));
}

// The next tile streams as chunks of CH samples (16 for networks of up to 4
// layers, 11 for deeper ones, so the stream spreads over every layer):
// chunk c is issued during layer c and folded during layer c + 2 (or after
// the last layer); chunks no layer issued load after the last layer. The
// last chunk may run past sample 63: those rows lie past the tile's buffer
// resource and read 0.
template <int CH>
constexpr int n_chunks() { return (64 + CH - 1) / CH; }

template <int CH, typename IT>
__device__ inline void issue_chunk(IT (&val)[CH], __amdgpu_buffer_rsrc_t r, int voff0,
                                   int rowb, int chunk) {
  const int v = voff0 + chunk * CH * rowb;
#pragma unroll
  for (int j = 0; j < CH; ++j) val[j] = load_row<IT>(r, v + j * rowb);
}

// Horner order (bit j ends at position j) keeps every constant inline: a
// select of 1 << j would hold the large shifts in registers.
template <int CH, typename IT>
__device__ inline void fold_chunk(uint64_t& word, const IT (&val)[CH], int chunk) {
  uint32_t bits = 0;
#pragma unroll
  for (int j = CH - 1; j >= 0; --j) bits = (bits << 1) | (input_bit(val[j]) ? 1u : 0u);
  word |= (uint64_t)bits << (chunk * CH);
}

template <typename IT, int MAXO, bool TYPED, int CH>
__global__ void __launch_bounds__(kNetThreads)
fc_hard_net_rows_kernel(NetDesc desc, const IT* __restrict__ x, int B, int n_tiles,
                        float* __restrict__ logits) {
  constexpr int NCH = n_chunks<CH>();
  const_netdesc_t& d = *(const_netdesc_t*)__builtin_amdgcn_kernarg_segment_ptr();
  if constexpr (TYPED) {
    if (!plan_fits(d.plan, MAXO, d.in0)) {
      nan_logits(logits, B, d.C);
      return;
    }
  }
  extern __shared__ __align__(16) unsigned char smem[];
  uint64_t* lds = reinterpret_cast<uint64_t*>(smem);
  const int f = threadIdx.x;
  const bool fv = f < d.in0;
  const int voff0 = f * (int)sizeof(IT);
  const int rowb = d.in0 * (int)sizeof(IT);
  const int L = d.n_layers;
  IT val0[CH], val1[CH];
  int tile = blockIdx.x;
  uint64_t word = 0;
  {
    // first tile: two chunks in flight at a time
    const __amdgpu_buffer_rsrc_t r = tile_rows(x, B, d.in0, tile * 64);
    issue_chunk<CH>(val0, r, voff0, rowb, 0);
    issue_chunk<CH>(val1, r, voff0, rowb, 1);
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      if (c & 1) {
        fold_chunk<CH>(word, val1, c);
        if (c + 2 < NCH) issue_chunk<CH>(val1, r, voff0, rowb, c + 2);
      } else {
        fold_chunk<CH>(word, val0, c);
        if (c + 2 < NCH) issue_chunk<CH>(val0, r, voff0, rowb, c + 2);
      }
    }
  }
  uint32_t cb[MAXO];
  if constexpr (TYPED) load_codes_tm(cb, d.codes[0]);
  else load_codes(cb, d.codes[0], d.width[0]);
  // typed: the plan row of the layer about to run and the codes pointer of
  // the one after it are scalar-loaded a layer ahead, so no layer starts
  // with two dependent scalar-load round trips after its barrier
  PlanRow pc{};
  const uint32_t* cn = nullptr;
  if constexpr (TYPED) {
    pc = plan_row(d.plan, 0);
    cn = d.codes[L > 1 ? 1 : 0];
  }

  for (; tile < n_tiles; tile += gridDim.x) {
    if (fv) lds[f] = word;
    __syncthreads();
    const __amdgpu_buffer_rsrc_t r = tile_rows(x, B, d.in0, (tile + gridDim.x) * 64);
    uint64_t nword = 0;
    int cur = 0, nxt = d.maxw, cur_w = d.in0;
    // Layer l streams chunk l into val(l & 1) and folds chunk l - 2 from it.
    // Every layer issues its chunk (past the fourth the offsets are past the
    // tile's resource and read 0 without memory traffic) and the loop is
    // unrolled by two, so each layer issues the same loads into the same
    // registers: the compiler then waits only for the loads a step needs.
    auto layer = [&](int l, IT (&val)[CH]) __attribute__((always_inline)) {
      const int W = d.width[l];
      const int ln = (l + 1 < L) ? l + 1 : 0;  // after the last layer: layer 0 of the next tile
      uint32_t nb[MAXO];
      PlanRow pn{};
      const uint32_t* cnn = nullptr;
      if constexpr (TYPED) {
        load_codes_tm(nb, cn);
        pn = plan_row(d.plan, ln);
        cnn = d.codes[(ln + 1 < L) ? ln + 1 : 0];
      } else {
        load_codes(nb, d.codes[ln], d.width[ln]);
      }
      auto rows_work = [&]() __attribute__((always_inline)) {
        if (l >= 2 && l - 2 < NCH) fold_chunk<CH>(nword, val, l - 2);
        issue_chunk<CH>(val, r, voff0, rowb, l);
      };
      constexpr int GRP = (MAXO % 2 == 0 && MAXO > 4) ? MAXO / 2 : MAXO;
      if constexpr (TYPED && CH < 16) {
        // the row work overlaps the first operand reads (16-sample chunks
        // hold too many registers for that)
        typed_step<uint64_t, MAXO, GRP>(lds, cur, nxt, pc, cb, rows_work);
      } else if constexpr (TYPED) {
        rows_work();
        typed_step<uint64_t, MAXO, GRP>(lds, cur, nxt, pc, cb, NoWork());
      } else {
        rows_work();
        layer_step<uint64_t, MAXO, GRP>(lds, cur, nxt, W, cb);
        if (d.wire_r > 0 && cur_w == W) keep_inputs<uint64_t, MAXO>(lds, cur, nxt, min(d.wire_r, W));
      }
      __syncthreads();
      const int t = cur; cur = nxt; nxt = t;
      cur_w = W;
#pragma unroll
      for (int j = 0; j < MAXO; ++j) cb[j] = nb[j];
      if constexpr (TYPED) {
        pc = pn;
        cn = cnn;
      }
    };
    for (int l = 0; l < L; l += 2) {
      layer(l, val0);
      if (l + 1 < L) layer(l + 1, val1);
    }
    // chunks issued during the last two layers, then chunks no layer issued
    for (int c = max(0, L - 2); c < min(L, NCH); ++c) {
      if (c & 1) fold_chunk<CH>(nword, val1, c);
      else fold_chunk<CH>(nword, val0, c);
    }
    for (int c = L; c < NCH; ++c) {
      issue_chunk<CH>(val0, r, voff0, rowb, c);
      fold_chunk<CH>(nword, val0, c);
    }
    // every chunk is folded: the chunk registers hold nothing the next tile
    // reads before writing, but the layer loop's control flow does not show
    // it; constants here let the GroupSum below have those registers
#pragma unroll
    for (int j = 0; j < CH; ++j) val0[j] = val1[j] = (IT)0;
    groupsum_tile<uint64_t>(lds + cur, cur_w, d.C, tile * 64, B, logits);
    __syncthreads();
    word = fv ? nword : 0ull;
  }
}

// ---------------------------------------------------------------------------
// operand placement for the fused network (bank-aware output order)
// ---------------------------------------------------------------------------
// In the fused network a wave's operand reads are ds_read_b64 of random
// activation words, served per 32-lane half with one cycle per distinct word
// of each bank class (word index mod 32). A layer's outputs may sit at any
// slot of its activation buffer as long as the next layer reads them there,
// so the outputs of every layer but the last are placed so that the 32
// outputs computed by one half-wave (32 consecutive slots, a "group") read
// operands of distinct bank classes, as far as the counts allow:
//  * Latin part: output o with operand classes (ca, cb) and rank k among
//    the outputs of its (ca, cb) cell (in index order) goes to lane ca of
//    group r + 32k, r = (cb - ca) mod 32, while that group exists. In every
//    group lane c then reads a-class c and b-class (g + c) mod 32: no
//    conflict on either read.
//  * the rest of a-class c takes the free lane-c slots, first in groups
//    whose Latin part lacks its b-class, in ascending order;
//  * what is left fills the remaining free slots in index order.
// The next layer's operand indices are renamed to the slots; the last layer
// keeps its order (the GroupSum reads its class blocks). The result is a
// relabelling of the circuit: the logits are the same bits. Deterministic
// (stable ranks by sorting, each search in a fixed order). One workgroup
// walks the layers in order, since each placement renames the next layer's
// operands.
constexpr int kPlaceThreads = 1024;
constexpr int kPlaceMax = 1 << 14;   // outputs per layer (14-bit slots)
struct PlaceNet {
  const uint32_t* in[kMaxLayers];    // compact codes, W[l] each
  uint32_t* out[kMaxLayers];         // placed codes: S[l] = round up(W[l], 32) slots, last W[l]
  int32_t* perm[kMaxLayers];         // output -> slot, layers 0 .. L-2
  int W[kMaxLayers];
  int L;
};

__device__ inline uint32_t remap_code(const PlaceNet& n, int l, int o) {
  const uint32_t c = n.in[l][o];
  uint32_t a = (c >> 14) & 0x3FFFu, b = c & 0x3FFFu;
  if (l > 0) {   // the prep clamps operands below the input width; kept in range here too
    const uint32_t lim = (uint32_t)n.W[l - 1] - 1u;
    a = (uint32_t)n.perm[l - 1][min(a, lim)];
    b = (uint32_t)n.perm[l - 1][min(b, lim)];
  }
  return b | (a << 14) | (c & 0xF0000000u);
}

__global__ void __launch_bounds__(kPlaceThreads) fc_hard_place_kernel(PlaceNet n) {
  __shared__ uint32_t keys[kPlaceMax];            // cell << 14 | output, sorted
  __shared__ int start[1024];                      // first sorted position of each cell
  __shared__ uint32_t taken[kPlaceMax / 32];       // slot occupied, one bit per lane
  __shared__ uint32_t bmask[kPlaceMax / 32];       // b-classes of each group's Latin part
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int l = 0; l + 1 < n.L; ++l) {
    const int W = n.W[l], NG = (W + 31) >> 5, S = NG * 32;
    int P = 32;
    while (P < W) P <<= 1;
    for (int i = tid; i < 1024; i += kPlaceThreads) start[i] = 0;
    for (int i = tid; i < NG; i += kPlaceThreads) taken[i] = bmask[i] = 0u;
    for (int s = tid; s < S; s += kPlaceThreads) n.out[l][s] = 0u;   // unused slots: code 0
    __syncthreads();
    for (int i = tid; i < P; i += kPlaceThreads) {
      uint32_t key = 0xFFFFFFFFu;
      if (i < W) {
        const uint32_t c = remap_code(n, l, i);
        const uint32_t cell = (((c >> 14) & 31u) << 5) | (c & 31u);
        key = (cell << 14) | (uint32_t)i;
        atomicAdd(&start[cell], 1);
      }
      keys[i] = key;
    }
    __syncthreads();
    // bitonic sort of the P keys (ascending: by cell, then by output)
    for (int k = 2; k <= P; k <<= 1) {
      for (int j = k >> 1; j > 0; j >>= 1) {
        for (int i = tid; i < P; i += kPlaceThreads) {
          const int ixj = i ^ j;
          if (ixj > i) {
            const uint32_t x = keys[i], y = keys[ixj];
            if ((x > y) == ((i & k) == 0)) {
              keys[i] = y;
              keys[ixj] = x;
            }
          }
        }
        __syncthreads();
      }
    }
    // cell counts -> exclusive starts (one thread per cell, Hillis-Steele)
    {
      const int cnt = start[tid];
      __syncthreads();
      int v = cnt;
      start[tid] = v;
      __syncthreads();
      for (int off = 1; off < 1024; off <<= 1) {
        const int add = tid >= off ? start[tid - off] : 0;
        __syncthreads();
        v += add;
        start[tid] = v;
        __syncthreads();
      }
      start[tid] = v - cnt;
      __syncthreads();
    }
    // Latin part
    for (int p = tid; p < W; p += kPlaceThreads) {
      const uint32_t key = keys[p];
      const int o = (int)(key & 0x3FFFu), cell = (int)(key >> 14);
      const int ca = cell >> 5, cb = cell & 31;
      const int k = p - start[cell], r = (cb - ca) & 31;
      const int navail = (NG - r + 31) >> 5;
      if (k < navail) {
        const int g = r + 32 * k, slot = 32 * g + ca;
        n.perm[l][o] = slot;
        n.out[l][slot] = remap_code(n, l, o);
        atomicOr(&taken[g], 1u << ca);
        atomicOr(&bmask[g], 1u << cb);
      } else {
        n.perm[l][o] = -1;
      }
    }
    __syncthreads();
    // the rest of a-class c on free lane-c slots (wave w: classes w, w + 16);
    // only this wave changes lane c's bits of `taken`
    for (int c = wave; c < 32; c += kPlaceThreads / 64) {
      const int p0 = start[c * 32], p1 = c == 31 ? W : start[c * 32 + 32];
      for (int q0 = p0; q0 < p1; q0 += 64) {
        const int p = q0 + lane;
        bool over = false;
        int o = 0, cb = 0;
        if (p < p1) {
          const uint32_t key = keys[p];
          o = (int)(key & 0x3FFFu);
          const int cell = (int)(key >> 14);
          cb = cell & 31;
          const int r = (cb - c) & 31;
          over = (p - start[cell]) >= ((NG - r + 31) >> 5);
        }
        uint64_t m = __ballot(over);
        while (m) {
          const int src = __ffsll((long long)m) - 1;
          m &= m - 1;
          const int oo = __shfl(o, src), bb = __shfl(cb, src);
          int best = -1, any = -1;
          for (int g0 = 0; g0 < NG && best < 0; g0 += 64) {
            const int g = g0 + lane;
            const bool fr = g < NG && !((taken[min(g, NG - 1)] >> c) & 1u);
            const bool nob = fr && !((bmask[min(g, NG - 1)] >> bb) & 1u);
            const uint64_t mb = __ballot(nob), mf = __ballot(fr);
            if (mb) best = g0 + __ffsll((long long)mb) - 1;
            else if (any < 0 && mf) any = g0 + __ffsll((long long)mf) - 1;
          }
          const int g = best >= 0 ? best : any;
          if (g >= 0) {
            if (lane == 0) {
              const int slot = 32 * g + c;
              n.perm[l][oo] = slot;
              n.out[l][slot] = remap_code(n, l, oo);
              atomicOr(&taken[g], 1u << c);
            }
          }
          __builtin_amdgcn_s_waitcnt(0);   // lane 0's LDS update before the next search
          __builtin_amdgcn_wave_barrier();
        }
      }
    }
    __syncthreads();
    // leftovers (index order) onto the free slots (ascending), by wave 0;
    // the sorted keys are no longer needed and hold the list
    if (wave == 0) {
      int cnt = 0;
      for (int o0 = 0; o0 < W; o0 += 64) {
        const int o = o0 + lane;
        const bool left = o < W && n.perm[l][o] < 0;
        const uint64_t m = __ballot(left);
        if (left) keys[cnt + __popcll(m & ((1ull << lane) - 1))] = (uint32_t)o;
        cnt += __popcll(m);
      }
      __builtin_amdgcn_s_waitcnt(0);
      __builtin_amdgcn_wave_barrier();
      int j = 0;
      for (int s0 = 0; s0 < S && j < cnt; s0 += 64) {
        const int s = s0 + lane;
        const bool fr = s < S && !((taken[min(s >> 5, NG - 1)] >> (s & 31)) & 1u);
        const uint64_t m = __ballot(fr);
        const int rk = j + __popcll(m & ((1ull << lane) - 1));
        if (fr && rk < cnt) {
          const int o = (int)keys[rk];
          n.perm[l][o] = s;
          n.out[l][s] = remap_code(n, l, o);
        }
        j += __popcll(m);
      }
    }
    __syncthreads();
    __threadfence_block();
  }
  // last layer: its own order, operands renamed
  const int l = n.L - 1;
  for (int o = tid; o < n.W[l]; o += kPlaceThreads) n.out[l][o] = remap_code(n, l, o);
}

// ---------------------------------------------------------------------------
// type-uniform placement for the fused network on unpacked rows
// ---------------------------------------------------------------------------
// Every layer but the last gets MAXO * 1024 slots, slot s = j * 1024 + tid in
// row j of thread tid (wave w = tid / 64), in groups of 32 (s / 32). A plan
// per layer picks U and gives each type T m[T] waves whose rows 0..U-1 hold
// type-T outputs (64 U per wave, in index order); what does not fit, and the
// types left without a wave, go to the generic rows U..rows-1. The 16 waves
// go one at a time to the type with the most outputs not yet given a wave
// (ties: the lower type); U is the largest value whose overflow fits the
// rows left (U = 0: all rows generic). Within its groups a bin's outputs
// are placed greedily in index order: each goes to the group where it adds
// the fewest repeated operand bank classes (word index mod 32, only for the
// operands its gate reads: the highest count first, then the sum, then the
// lowest group), among groups with a free slot (bins of up to 64 groups keep
// their counts in registers, saturating at 3). The outputs of a wave's own
// rows (the k-th wave of type T takes that type's ranks [64 U k, 64 U
// (k + 1))) are placed in two halves, the first 32 U into the groups of its
// lanes 0-31 and the rest into those of lanes 32-63, all halves at once;
// four more place the generic bin, each every fourth output into every
// fourth group. Uniform
// rows get codes (a << 16) | b with absolute word indices (the read buffer
// of layer l starts at word (l & 1) * MAXO * 1024); generic rows get compact
// codes on the renamed operands; unused slots get codes reading word 0 of
// the read buffer. The last layer keeps its order and compact codes, with
// operands renamed (slots past its width: code 0). Every layer's codes are
// stored thread-major (slot j * 1024 + tid at tid * MAXO + j). The result is
// a relabelling: the logits are the same.
constexpr int kTypeMaxGroups = 512;     // 16 rows x 32 groups
struct TypePlaceNet {
  const uint32_t* in[kMaxLayers];    // compact codes, W[l] each
  uint32_t* out[kMaxLayers];         // MAXO * 1024 slots per layer, stored thread-major
  int32_t* perm[kMaxLayers];         // output -> slot, layers 0 .. L-2
  int32_t* plan;                     // [L][kPlanStride]
  int W[kMaxLayers];
  int L, maxo, in0;
};

__device__ inline void type_operands(const TypePlaceNet& n, int l, int o, uint32_t& a, uint32_t& b,
                                     uint32_t& tt) {
  const uint32_t c = n.in[l][o];
  a = (c >> 14) & 0x3FFFu;
  b = c & 0x3FFFu;
  tt = c >> 28;
  if (l > 0) {   // the prep clamps operands below the input width; kept in range here too
    const uint32_t lim = (uint32_t)n.W[l - 1] - 1u;
    a = (uint32_t)n.perm[l - 1][min(a, lim)];
    b = (uint32_t)n.perm[l - 1][min(b, lim)];
  }
}

// Wave-wide minimum of a 32-bit key, in every lane (every lane active):
// DPP quad_perm [1,0,3,2] and [2,3,0,1], row_half_mirror and row_mirror
// within 16-lane rows, then permlane16/32 swaps across rows.
__device__ __forceinline__ uint32_t wave_min(uint32_t k) {
  k = min(k, (uint32_t)__builtin_amdgcn_mov_dpp((int)k, 0xB1, 0xF, 0xF, false));
  k = min(k, (uint32_t)__builtin_amdgcn_mov_dpp((int)k, 0x4E, 0xF, 0xF, false));
  k = min(k, (uint32_t)__builtin_amdgcn_mov_dpp((int)k, 0x141, 0xF, 0xF, false));
  k = min(k, (uint32_t)__builtin_amdgcn_mov_dpp((int)k, 0x140, 0xF, 0xF, false));
  const auto r16 = __builtin_amdgcn_permlane16_swap(k, k, false, false);
  k = min(r16[0], r16[1]);
  const auto r32 = __builtin_amdgcn_permlane32_swap(k, k, false, false);
  return min(r32[0], r32[1]);
}

// Group of candidate q of a bin: uniform bin of type T (waves w0.., U rows
// each, two groups per row) or the generic bin (rows U.., 32 groups per row).
__device__ __forceinline__ int bin_group(bool generic, int q, int U, int w0) {
  if (generic) return U * 32 + q;
  const int i = q / (2 * U), r = q - i * 2 * U;
  return (r >> 1) * 32 + (w0 + i) * 2 + (r & 1);
}

// Place output o (classes ca, cb) in the best group of a bin of G groups;
// the calling wave owns the bin's groups. Returns the slot.
__device__ int place_greedy(uint8_t (*cnt)[64], int* fill, bool generic, int G, int U, int w0,
                            bool na, bool nb, int ca, int cb, int lane) {
  uint32_t best = 0xFFFFFFFFu;
  for (int q = lane; q < G; q += 64) {
    const int g = bin_group(generic, q, U, w0);
    if (fill[g] >= 32) continue;
    const uint32_t pa = na ? cnt[g][ca] : 0u, pb = nb ? cnt[g][32 + cb] : 0u;
    const uint32_t key = ((max(pa, pb) << 7 | (pa + pb)) << 16) | (uint32_t)q;
    best = min(best, key);
  }
  best = wave_min(best);
  int slot = -1;
  if (best != 0xFFFFFFFFu) {
    const int g = bin_group(generic, (int)(best & 0xFFFFu), U, w0);
    slot = g * 32 + fill[g];
    __builtin_amdgcn_wave_barrier();
    if (lane == 0) {
      fill[g] += 1;
      if (na) cnt[g][ca] += 1;
      if (nb) cnt[g][32 + cb] += 1;
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0): lane 0's LDS updates land first
    __builtin_amdgcn_wave_barrier();
  }
  return slot;
}

// slot s = j * 1024 + tid of a layer's codes is stored at tid * MAXO + j
__device__ __forceinline__ int tm_index(int s, int maxo) { return (s & (kNetThreads - 1)) * maxo + (s >> 10); }

// Greedy state of a bin of at most 64 groups held in registers: lane q owns
// group q (its fill count and, per operand side, the bank classes it reads
// at least once, twice and three times: counts saturate at 3 here). A step
// is then a few VALU operations and the DPP minimum, with no LDS round trip;
// the key and the tie order are those of place_greedy. Every lane of the
// wave must call place() together.
struct RegBin {
  int fill = 0;
  uint32_t a1 = 0, a2 = 0, a3 = 0, b1 = 0, b2 = 0, b3 = 0;

  // group q of the bin: every gs-th group from go, bin_group(false, q * gs +
  // go, U, w0) of a type bin or U * 32 + q * gs + go of the generic bin
  __device__ int place(bool generic, int G, int U, int w0, bool na, bool nb, int ca, int cb,
                       int lane, int gs = 1, int go = 0) {
    const uint32_t ba = 1u << ca, bb = 1u << cb;
    const uint32_t pa = na ? (uint32_t)((a1 & ba) != 0) + ((a2 & ba) != 0) + ((a3 & ba) != 0) : 0u;
    const uint32_t pb = nb ? (uint32_t)((b1 & bb) != 0) + ((b2 & bb) != 0) + ((b3 & bb) != 0) : 0u;
    const bool ok = lane < G && fill < 32;
    const uint32_t key = wave_min(ok ? ((max(pa, pb) << 7 | (pa + pb)) << 16) | (uint32_t)lane
                                     : 0xFFFFFFFFu);
    if (key == 0xFFFFFFFFu) return -1;
    const int q = (int)(key & 0xFFFFu);
    const int f = __builtin_amdgcn_readlane(fill, q);
    if (lane == q) {
      fill += 1;
      if (na) { a3 |= a2 & ba; a2 |= a1 & ba; a1 |= ba; }
      if (nb) { b3 |= b2 & bb; b2 |= b1 & bb; b1 |= bb; }
    }
    return (generic ? U * 32 + q * gs + go : bin_group(false, q * gs + go, U, w0)) * 32 + f;
  }
};

// The placement runs per layer as three launches, so that the greedy
// steps of the bins run on as many CUs as there are bins (one workgroup of
// one wave per bin) instead of sharing one CU's VALU: plan (one
// workgroup), bins (one workgroup per type bin and per generic sub-bin),
// codes (every output and slot). Scratch between them, in the caller's
// workspace after the renaming tables (TypePlaceScratch).
struct TypePlaceScratch {
  uint32_t* info;   // [kPlaceMax] output -> a-class | b-class << 5 | type << 10
  int32_t* olist;   // [kPlaceMax] outputs of the type bins, by type then rank
  int32_t* glist;   // [kPlaceMax] generic outputs in index order
  int32_t* slot;    // [kPlaceMax] output -> slot
  int32_t* fill;    // [kTypeMaxGroups] slots taken in each group
  int32_t* meta;    // U, rows, n_generic, then m, w0, wtt, tstart, tcount (16 each)
};
constexpr int kTypeMetaInts = 128;
constexpr int kTypeScratchInts = 4 * kPlaceMax + kTypeMaxGroups + kTypeMetaInts;
enum { kMetaU = 0, kMetaRows = 1, kMetaNGen = 2, kMetaM = 3, kMetaW0 = 19, kMetaWtt = 35,
       kMetaTStart = 51, kMetaTCount = 67 };

// Plan of layer l: operand classes and types, the plan row (U, rows, a
// type per wave; the planner gives the 16 waves one at a time to the type
// with the most outputs not yet given a wave and takes the largest U whose
// overflow fits the rows left), the type bins' outputs by type in index
// order, and the generic outputs in index order.
__global__ void __launch_bounds__(kPlaceThreads)
fc_hard_type_plan_kernel(TypePlaceNet n, TypePlaceScratch ws, int l) {
  // as ws.info (classes and type in bits 0-13), read back here from LDS; bit
  // 14 marks the generic outputs
  __shared__ uint16_t info[kPlaceMax];
  __shared__ int hist[16], m[16], w0[16], wtt[16], tstart[16];
  __shared__ int plan_u;
  __shared__ int ccount[kPlaceMax / 64][16];   // per chunk and type: count, then prefix
  __shared__ int gcount[kPlaceMax / 64];       // per chunk: generic count, then prefix
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int maxo = n.maxo, W = n.W[l];
  if (tid < 16) hist[tid] = 0;
  for (int i = tid; i < kTypeMaxGroups; i += kPlaceThreads) ws.fill[i] = 0;
  __syncthreads();
  // every output's code, then the renaming of its operands, loaded with all
  // of a thread's outputs in flight (two memory round trips, not two per
  // output); the type histogram by wave ballots (lane T of a wave counts
  // type T), one LDS add per type and wave
  constexpr int PER = kPlaceMax / kPlaceThreads;
  uint32_t cv[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int o = tid + i * kPlaceThreads;
    cv[i] = o < W ? n.in[l][o] : 0u;
  }
  uint32_t av[PER], bv[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    av[i] = (cv[i] >> 14) & 0x3FFFu;
    bv[i] = cv[i] & 0x3FFFu;
  }
  if (l > 0) {   // the prep clamps operands below the input width; kept in range here too
    const uint32_t lim = (uint32_t)n.W[l - 1] - 1u;
    const int32_t* pm = n.perm[l - 1];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      if (tid + i * kPlaceThreads < W) {
        av[i] = (uint32_t)pm[min(av[i], lim)];
        bv[i] = (uint32_t)pm[min(bv[i], lim)];
      }
    }
  }
  int my_count = 0;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int o = tid + i * kPlaceThreads;
    uint32_t tt = 16u;  // past the layer: no type
    if (o < W) {
      tt = cv[i] >> 28;
      const uint32_t v = (av[i] & 31u) | ((bv[i] & 31u) << 5) | (tt << 10);
      info[o] = (uint16_t)v;
      ws.info[o] = v;
    }
#pragma unroll
    for (int T = 0; T < 16; ++T) {
      const int c = (int)__popcll(__ballot(tt == (uint32_t)T));
      if (lane == T) my_count += c;
    }
  }
  if (lane < 16 && my_count) atomicAdd(&hist[lane], my_count);
  __syncthreads();
  if (tid == 0) {
    int U = 0, rows = (W + kNetThreads - 1) / kNetThreads;
    int mm[16];
    for (int T = 0; T < 16; ++T) mm[T] = 0;
    for (int u = maxo - 1; u >= 1; --u) {
      const int cap = 64 * u;
      for (int T = 0; T < 16; ++T) mm[T] = 0;
      for (int waves = 0; waves < 16; ++waves) {
        int bt = -1, br = 0;
        for (int T = 0; T < 16; ++T) {
          const int rem = hist[T] - mm[T] * cap;
          if (rem > br) { br = rem; bt = T; }
        }
        if (bt < 0) break;
        mm[bt] += 1;
      }
      int over = 0;
      for (int T = 0; T < 16; ++T) over += max(0, hist[T] - mm[T] * cap);
      const int rg = (over + kNetThreads - 1) / kNetThreads;
      if (u + rg <= maxo) { U = u; rows = u + rg; break; }
    }
    if (U == 0)
      for (int T = 0; T < 16; ++T) mm[T] = 0;
    int w = 0, ts = 0;
    for (int T = 0; T < 16; ++T) {
      m[T] = mm[T];
      w0[T] = w;
      for (int i = 0; i < mm[T]; ++i) wtt[w++] = T;
      tstart[T] = ts;
      ts += min(hist[T], 64 * U * mm[T]);
    }
    for (; w < 16; ++w) wtt[w] = 0;
    plan_u = U;
    int32_t* pl = n.plan + l * kPlanStride;
    pl[0] = U;
    pl[1] = rows;
    for (int i = 0; i < 16; ++i) pl[2 + i] = wtt[i];
    pl[18] = n.maxo;
    pl[19] = n.in0;
    ws.meta[kMetaU] = U;
    ws.meta[kMetaRows] = rows;
    for (int i = 0; i < 16; ++i) {
      ws.meta[kMetaM + i] = m[i];
      ws.meta[kMetaW0 + i] = w0[i];
      ws.meta[kMetaWtt + i] = wtt[i];
      ws.meta[kMetaTStart + i] = tstart[i];
      ws.meta[kMetaTCount + i] = min(hist[i], 64 * U * m[i]);
    }
  }
  __syncthreads();
  const int U = plan_u;
  // ranks within each type and the generic outputs, from per-chunk counts:
  // chunk c = outputs [64c, 64c + 64); each type's outputs of rank below its
  // waves' capacity go to the type's list in rank order, the rest (and the
  // types without a wave) are generic, listed in index order
  const int nch = (W + 63) >> 6;
  const uint64_t below = (1ull << lane) - 1ull;
  for (int c = wave; c < nch; c += kPlaceThreads / 64) {
    const int o = c * 64 + lane;
    const uint32_t t = o < W ? (uint32_t)(info[o] >> 10) : 16u;
#pragma unroll
    for (int T = 0; T < 16; ++T) {
      const int k = (int)__popcll(__ballot(t == (uint32_t)T));
      if (lane == T) ccount[c][T] = k;
    }
  }
  __syncthreads();
  // exclusive prefix over the chunks, per type: wave T scans type T, lane j
  // holding chunks [4j, 4j + 4)
  if (wave < 16) {
    const int T = wave;
    int v4[4], sum = 0;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int c = 4 * lane + u;
      v4[u] = c < nch ? ccount[c][T] : 0;
      sum += v4[u];
    }
    int incl = sum;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int y = __shfl_up(incl, d);
      if (lane >= d) incl += y;
    }
    int run = incl - sum;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int c = 4 * lane + u;
      if (c < nch) ccount[c][T] = run;
      run += v4[u];
    }
  }
  __syncthreads();
  for (int c = wave; c < nch; c += kPlaceThreads / 64) {
    const int o = c * 64 + lane;
    const uint32_t t = o < W ? (uint32_t)(info[o] >> 10) : 16u;
    int r = 0;
#pragma unroll
    for (int T = 0; T < 16; ++T) {
      const uint64_t mk = __ballot(t == (uint32_t)T);
      if (t == (uint32_t)T) r = ccount[c][T] + (int)__popcll(mk & below);
    }
    bool gen = false;
    if (o < W) {
      const int cap = 64 * U * m[t];
      if (r < cap) ws.olist[tstart[t] + r] = o;
      gen = r >= cap;
    }
    const int k = (int)__popcll(__ballot(gen));
    if (lane == 0) gcount[c] = k;
    if (o < W && gen) info[o] = (uint16_t)(info[o] | 0x4000u);
  }
  __syncthreads();
  // the generic outputs in index order: a prefix over the chunks' counts
  if (wave == 0) {
    int v4[4], sum = 0;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int c = 4 * lane + u;
      v4[u] = c < nch ? gcount[c] : 0;
      sum += v4[u];
    }
    int incl = sum;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int y = __shfl_up(incl, d);
      if (lane >= d) incl += y;
    }
    int run = incl - sum;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int c = 4 * lane + u;
      if (c < nch) gcount[c] = run;
      run += v4[u];
    }
    if (lane == 63) ws.meta[kMetaNGen] = incl;
  }
  __syncthreads();
  for (int c = wave; c < nch; c += kPlaceThreads / 64) {
    const int o = c * 64 + lane;
    const bool left = o < W && (info[o] & 0x4000u);
    const uint64_t ml = __ballot(left);
    if (left) ws.glist[gcount[c] + (int)__popcll(ml & below)] = o;
  }
}

// The bins of layer l: workgroups 2w and 2w + 1 (w < 16) are the two lane
// halves of wave w of the type-uniform rows (the k-th wave of type T holds
// that type's ranks [64 U k, 64 U (k + 1)); half h places the h-th 32 U of
// them into the wave's U groups of lane half h), workgroups 32.. the
// generic sub-bins (up to 256 groups: sub-bin j takes the generic outputs of
// rank j, j + NS, ... into groups j, j + NS, ...; larger bins: one workgroup
// places them all, with the counts in LDS). Each places its outputs
// greedily in index order and writes their slots and its groups' fill.
__global__ void __launch_bounds__(64) fc_hard_type_bins_kernel(TypePlaceNet n, TypePlaceScratch ws) {
  __shared__ uint8_t cnt[kTypeMaxGroups][64];
  __shared__ int fill[kTypeMaxGroups];
  const int lane = threadIdx.x;
  const int U = ws.meta[kMetaU], rows = ws.meta[kMetaRows];
  if (blockIdx.x < 2 * 16) {
    // half h of the type bin of wave w: the wave's groups of lane half h
    // (one per row) and half of the bin's ranks, so that the two halves'
    // greedy steps run side by side
    const int w = blockIdx.x >> 1, h = blockIdx.x & 1;
    const int T = ws.meta[kMetaWtt + w], k = w - ws.meta[kMetaW0 + T];
    const int mT = ws.meta[kMetaM + T];
    if (U == 0 || mT == 0 || k < 0 || k >= mT) return;
    // the type's list holds its first min(count, 64 U m) outputs by rank:
    // this wave's bin takes ranks [64 U k, 64 U (k + 1)) of them, and half
    // h the h-th 32 U of those
    const int start = ws.meta[kMetaTStart + T], count = ws.meta[kMetaTCount + T];
    const int lo = 64 * U * k + 32 * U * h, hi = min(lo + 32 * U, count), G = U;
    const bool na = tt_needs_a(T), nb = tt_needs_b(T);
    RegBin rb;
    for (int r0 = lo; r0 < hi; r0 += 64) {
      const int r = r0 + lane;
      const bool ok = r < hi;
      const int o = ok ? ws.olist[start + r] : -1;
      const uint32_t in = ok ? ws.info[o] : 0u;
      uint64_t mk = __ballot(ok);
      while (mk) {
        const int src = __ffsll((long long)mk) - 1;
        mk &= mk - 1;
        const int ca = __builtin_amdgcn_readlane((int)(in & 31u), src);
        const int cb = __builtin_amdgcn_readlane((int)((in >> 5) & 31u), src);
        const int oo = __builtin_amdgcn_readlane(o, src);
        const int sl = rb.place(false, G, U, w, na, nb, ca, cb, lane, 2, h);
        if (lane == 0) ws.slot[oo] = sl;
      }
    }
    if (lane < G) ws.fill[bin_group(false, 2 * lane + h, U, w)] = rb.fill;
    return;
  }
  const int G = 32 * (rows - U);
  const int NS = G <= 256 ? 4 : 1;
  const int j = blockIdx.x - 2 * 16;
  if (j >= NS || G == 0) return;
  const int Gs = G / NS;
  const bool regs = Gs <= 64;
  if (!regs) {
    for (int i = lane; i < kTypeMaxGroups * 16; i += 64)
      reinterpret_cast<uint32_t*>(&cnt[0][0])[i] = 0u;
    for (int i = lane; i < kTypeMaxGroups; i += 64) fill[i] = 0;
    __syncthreads();
  }
  const int ng = ws.meta[kMetaNGen];
  RegBin rb;
  for (int r0 = 0; r0 < ng; r0 += 64) {
    const int r = r0 + lane;
    const bool ok = r < ng && r % NS == j;
    const int o = ok ? ws.glist[r] : -1;
    const uint32_t in = ok ? ws.info[o] : 0u;
    uint64_t mk = __ballot(ok);
    while (mk) {
      const int src = __ffsll((long long)mk) - 1;
      mk &= mk - 1;
      const int ca = __builtin_amdgcn_readlane((int)(in & 31u), src);
      const int cb = __builtin_amdgcn_readlane((int)((in >> 5) & 31u), src);
      const int oo = __builtin_amdgcn_readlane(o, src);
      const int sl = regs ? rb.place(true, Gs, U, 0, true, true, ca, cb, lane, NS, j)
                          : place_greedy(cnt, fill, true, G, U, 0, true, true, ca, cb, lane);
      if (lane == 0) ws.slot[oo] = sl;
    }
  }
  if (regs) {
    if (lane < Gs) ws.fill[U * 32 + lane * NS + j] = rb.fill;
  } else {
    __syncthreads();
    for (int g = lane; g < G; g += 64) ws.fill[U * 32 + g] = fill[U * 32 + g];
  }
}

// Codes of layer l (every output) and its unused slots (every slot), and
// the renaming table the next layer reads.
__global__ void __launch_bounds__(256) fc_hard_type_codes_kernel(TypePlaceNet n, TypePlaceScratch ws,
                                                                 int l) {
  const int U = ws.meta[kMetaU];
  const int maxo = n.maxo, S = maxo * kNetThreads, W = n.W[l];
  const uint32_t base = (uint32_t)((l & 1) * S);
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < W) {
    uint32_t a, b, tt;
    type_operands(n, l, i, a, b, tt);
    const int s = ws.slot[i];
    n.perm[l][i] = s;
    n.out[l][tm_index(s, maxo)] =
        (s >> 10) < U ? ((a + base) << 16) | (b + base) : (b | (a << 14) | (tt << 28));
  }
  if (i < S) {
    // groups no bin filled were cleared by the plan kernel
    if ((i & 31) >= ws.fill[i >> 5])
      n.out[l][tm_index(i, maxo)] = (i >> 10) < U ? (base << 16) | base : 0u;
  }
}

// The last layer: its own order, compact codes, operands renamed (slots
// past its width: code 0), and its plan row.
__global__ void __launch_bounds__(256) fc_hard_type_last_kernel(TypePlaceNet n) {
  const int l = n.L - 1;
  const int maxo = n.maxo, S = maxo * kNetThreads;
  const int s = blockIdx.x * 256 + threadIdx.x;
  if (s < S) {
    uint32_t a = 0, b = 0, tt = 0;
    if (s < n.W[l]) type_operands(n, l, s, a, b, tt);
    n.out[l][tm_index(s, maxo)] = b | (a << 14) | (tt << 28);
  }
  if (s == 0) {
    int32_t* pl = n.plan + l * kPlanStride;
    pl[0] = 0;
    pl[1] = (n.W[l] + kNetThreads - 1) / kNetThreads;
    for (int i = 0; i < 16; ++i) pl[2 + i] = 0;
    pl[18] = n.maxo;
    pl[19] = n.in0;
  }
}

// ---------------------------------------------------------------------------
// packed GroupSum (layer-wise path): one workgroup per 64-sample word column
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256) groupsum_packed_kernel(const uint64_t* __restrict__ xp, int W,
                                                              int nw, int B, int C,
                                                              float* __restrict__ logits) {
  extern __shared__ int gcnt[];  // [C][64]
  const int w = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
  for (int i = threadIdx.x; i < C * 64; i += blockDim.x) gcnt[i] = 0;
  __syncthreads();
  const int G = W / C;
  const int chunks = (G + 63) / 64;
  for (int task = wave; task < C * chunks; task += nwaves) {
    const int c = task / chunks, j0 = (task % chunks) * 64;
    uint64_t v = (j0 + lane < G) ? xp[(int64_t)(c * G + j0 + lane) * nw + w] : 0ull;
    v = transpose64(v, lane);
    const int pc = __popcll(v);
    if (pc) atomicAdd(&gcnt[c * 64 + lane], pc);
  }
  __syncthreads();
  for (int i = threadIdx.x; i < 64 * C; i += blockDim.x) {
    const int s = i / C, c = i % C;
    const int b = w * 64 + s;
    if (b < B) logits[(int64_t)b * C + c] = (float)gcnt[c * 64 + s];
  }
}


template <int LAYOUT, typename WT, int MAXO>
static int launch_net_packed(const void* xp, int B, const NetDesc& d, size_t lds, int64_t tiles,
                             float* logits, hipStream_t st) {
  auto kern = d.plan ? fc_hard_net_packed_kernel<LAYOUT, WT, MAXO, true>
                     : fc_hard_net_packed_kernel<LAYOUT, WT, MAXO, false>;
  if (int rc = set_lds(kern, lds, "fc_hard_net")) return rc;
  hipLaunchKernelGGL(kern, dim3((unsigned)tiles), dim3(kNetThreads), lds, st, d, xp, B,
                     (int)cdiv(B, 64), logits);
  SLG_LAUNCH_CHECK("fc_hard_net");
  return 0;
}

template <int LAYOUT, typename WT>
static int net_packed_maxo(int maxo, const void* xp, int B, const NetDesc& d, size_t lds,
                           int64_t tiles, float* logits, hipStream_t st) {
  switch (maxo) {
    case 2: return launch_net_packed<LAYOUT, WT, 2>(xp, B, d, lds, tiles, logits, st);
    case 4: return launch_net_packed<LAYOUT, WT, 4>(xp, B, d, lds, tiles, logits, st);
    case 8: return launch_net_packed<LAYOUT, WT, 8>(xp, B, d, lds, tiles, logits, st);
    case 10: return launch_net_packed<LAYOUT, WT, 10>(xp, B, d, lds, tiles, logits, st);
    default: return launch_net_packed<LAYOUT, WT, 16>(xp, B, d, lds, tiles, logits, st);
  }
}

template <typename IT, int MAXO>
static int launch_net_rows(const IT* x, int B, const NetDesc& d, size_t lds, float* logits,
                           hipStream_t st) {
  const int64_t tiles = cdiv(B, 64);
  const int64_t grid = std::min<int64_t>(tiles, device_cus());
  auto kern = d.n_layers <= 4
                  ? (d.plan ? fc_hard_net_rows_kernel<IT, MAXO, true, 16>
                            : fc_hard_net_rows_kernel<IT, MAXO, false, 16>)
                  : (d.plan ? fc_hard_net_rows_kernel<IT, MAXO, true, 11>
                            : fc_hard_net_rows_kernel<IT, MAXO, false, 11>);
  if (int rc = set_lds(kern, lds, "fc_hard_net_rows")) return rc;
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(kNetThreads), lds, st, d, x, B, (int)tiles,
                     logits);
  SLG_LAUNCH_CHECK("fc_hard_net_rows");
  return 0;
}

template <typename IT>
static int net_rows_maxo(int maxo, const IT* x, int B, const NetDesc& d, size_t lds, float* logits,
                         hipStream_t st) {
  switch (maxo) {
    case 2: return launch_net_rows<IT, 2>(x, B, d, lds, logits, st);
    case 4: return launch_net_rows<IT, 4>(x, B, d, lds, logits, st);
    case 8: return launch_net_rows<IT, 8>(x, B, d, lds, logits, st);
    default: return launch_net_rows<IT, 10>(x, B, d, lds, logits, st);
  }
}

// The fused network on any input kind: fp32 / byte rows stream through
// the persistent rows kernel when 64-sample tiles hold at most 1024
// features, else each workgroup packs its own tile's rows (LAYOUT 2, 3);
// packed words by their layout. Rows at small batches (at most one
// 64-sample tile per four CUs: every workgroup holds one tile and the
// stream has nothing to overlap) take 32-sample tiles packed per tile, so
// twice the workgroups each read half the rows (config 1, B = 256: 10.4 ->
// 8.2 us).
static int launch_net_any(const void* x, int in_kind, int B, const NetDesc& d, int spw, int maxo,
                          size_t lds, float* logits, hipStream_t st) {
  if (in_kind <= 1 && spw == 64 && 4 * cdiv(B, 64) <= device_cus()) {
    const int64_t t32 = cdiv(B, 32);
    return in_kind == 0 ? net_packed_maxo<2, uint32_t>(maxo, x, B, d, lds / 2, t32, logits, st)
                        : net_packed_maxo<3, uint32_t>(maxo, x, B, d, lds / 2, t32, logits, st);
  }
  if (in_kind <= 1 && spw == 64 && d.in0 <= kNetThreads) {
    if (in_kind == 0) return net_rows_maxo<float>(maxo, (const float*)x, B, d, lds, logits, st);
    return net_rows_maxo<uint8_t>(maxo, (const uint8_t*)x, B, d, lds, logits, st);
  }
  const int64_t tiles = cdiv(B, spw);
  switch (in_kind) {
    case 0:
      return spw == 64 ? net_packed_maxo<2, uint64_t>(maxo, x, B, d, lds, tiles, logits, st)
                       : net_packed_maxo<2, uint32_t>(maxo, x, B, d, lds, tiles, logits, st);
    case 1:
      return spw == 64 ? net_packed_maxo<3, uint64_t>(maxo, x, B, d, lds, tiles, logits, st)
                       : net_packed_maxo<3, uint32_t>(maxo, x, B, d, lds, tiles, logits, st);
    case 2:
      return spw == 64 ? net_packed_maxo<0, uint64_t>(maxo, x, B, d, lds, tiles, logits, st)
                       : net_packed_maxo<0, uint32_t>(maxo, x, B, d, lds, tiles, logits, st);
    default:
      return spw == 64 ? net_packed_maxo<1, uint64_t>(maxo, x, B, d, lds, tiles, logits, st)
                       : net_packed_maxo<1, uint32_t>(maxo, x, B, d, lds, tiles, logits, st);
  }
}

}  // namespace slg

using namespace slg;

extern "C" {

int slg_pack_bits(const void* x, int32_t dtype, int64_t B, int64_t D, int32_t layout, uint64_t* xp,
                  slg_stream_t stream) {
  SLG_REQUIRE((x && xp) || B == 0, SLG_E_ARG, "pack_bits: null pointer");
  SLG_REQUIRE(dtype == 0 || dtype == 1, SLG_E_ARG, "pack_bits: dtype %d", dtype);
  SLG_REQUIRE(layout == 0 || layout == 1, SLG_E_ARG, "pack_bits: layout %d", layout);
  SLG_REQUIRE(B >= 0 && D > 0 && B < (1LL << 31) && D < (1LL << 31) && B * D < (1LL << 46),
              SLG_E_SHAPE, "pack_bits: bad sizes");
  if (B == 0) return 0;
  const int64_t nw = cdiv(B, 64);
  const size_t esz = dtype == 0 ? 4 : 1;
  const bool vec = D % 4 == 0 && (uintptr_t)x % (4 * esz) == 0;
  const int64_t dtiles = cdiv(D, vec ? 256 : 64);
  SLG_REQUIRE(cdiv(nw, 4) * dtiles < (1LL << 31), SLG_E_SHAPE, "pack_bits: too many tiles");
  dim3 grid((unsigned)(cdiv(nw, 4) * dtiles));
  hipStream_t st = as_stream(stream);
#define SLG_PACK(T, LY, V)                                                                     \
  hipLaunchKernelGGL((pack_kernel<T, LY, V>), grid, dim3(256), 0, st, (const T*)x, (int)B,     \
                     (int)D, (int)nw, (int)dtiles, xp)
#define SLG_PACK_V(T, LY) \
  do { if (vec) SLG_PACK(T, LY, 4); else SLG_PACK(T, LY, 1); } while (0)
  if (dtype == 0 && layout == 0) SLG_PACK_V(float, 0);
  else if (dtype == 0) SLG_PACK_V(float, 1);
  else if (layout == 0) SLG_PACK_V(uint8_t, 0);
  else SLG_PACK_V(uint8_t, 1);
#undef SLG_PACK_V
#undef SLG_PACK
  SLG_LAUNCH_CHECK("pack_bits");
  return 0;
}

int slg_unpack_bits(const uint64_t* xp, int64_t B, int64_t D, uint8_t* out, slg_stream_t stream) {
  SLG_REQUIRE((xp && out) || B == 0, SLG_E_ARG, "unpack_bits: null pointer");
  SLG_REQUIRE(B >= 0 && D > 0 && B < (1LL << 31) && D < (1LL << 31), SLG_E_SHAPE,
              "unpack_bits: bad sizes");
  if (B == 0) return 0;
  const int64_t n = B * D;
  hipLaunchKernelGGL(unpack_kernel, dim3((unsigned)cdiv(n, 256)), dim3(256), 0, as_stream(stream),
                     xp, (int)B, (int)D, (int)cdiv(B, 64), out);
  SLG_LAUNCH_CHECK("unpack_bits");
  return 0;
}

int slg_fc_hard_prep(const int32_t* cand, const float* conn, int64_t OUT, int32_t K, int64_t IN,
                     int32_t node_kind, const float* raw, uint32_t* codes, slg_stream_t stream) {
  SLG_REQUIRE(cand && raw && codes, SLG_E_ARG, "fc_hard_prep: null pointer");
  SLG_REQUIRE(OUT > 0 && OUT < (1LL << 31) && IN > 0 && IN <= (1LL << 28) && K >= 1 && K <= 64,
              SLG_E_SHAPE, "fc_hard_prep: bad sizes");
  SLG_REQUIRE(node_kind >= 0 && node_kind <= 2, SLG_E_ARG, "fc_hard_prep: node_kind %d", node_kind);
  SLG_REQUIRE(((uintptr_t)codes % 8) == 0, SLG_E_ARG, "fc_hard_prep: codes alignment");
  hipLaunchKernelGGL(fc_hard_prep_kernel, dim3((unsigned)cdiv(OUT, 256)), dim3(256), 0,
                     as_stream(stream), cand, conn, (int)OUT, K, (int)IN, node_kind, raw,
                     reinterpret_cast<uint2*>(codes));
  SLG_LAUNCH_CHECK("fc_hard_prep");
  return 0;
}

int slg_fc_hard_prep_net(int32_t n_layers, const int32_t* const* cand, const float* const* conn,
                         const float* const* raw, const int64_t* in_dim, const int64_t* out_dim,
                         const int32_t* K, const int32_t* node_kind, int32_t compact,
                         uint32_t* const* codes, slg_stream_t stream) {
  SLG_REQUIRE(n_layers >= 1 && n_layers <= kMaxPrepLayers, SLG_E_SHAPE,
              "fc_hard_prep_net: n_layers=%d outside 1..%d", n_layers, kMaxPrepLayers);
  SLG_REQUIRE(cand && conn && raw && in_dim && out_dim && K && node_kind && codes, SLG_E_ARG,
              "fc_hard_prep_net: null array");
  HardPrepNet net{};
  net.n = n_layers;
  const int th = 256;
  int64_t blocks = 0;
  for (int l = 0; l < n_layers; ++l) {
    SLG_REQUIRE(cand[l] && raw[l] && codes[l], SLG_E_ARG, "fc_hard_prep_net: null pointer, layer %d", l);
    SLG_REQUIRE(out_dim[l] > 0 && out_dim[l] < (1LL << 28) && in_dim[l] > 0 &&
                    in_dim[l] <= (1LL << 28) && K[l] >= 1 && K[l] <= 64, SLG_E_SHAPE,
                "fc_hard_prep_net: bad sizes, layer %d", l);
    SLG_REQUIRE(node_kind[l] >= 0 && node_kind[l] <= 2, SLG_E_ARG,
                "fc_hard_prep_net: node_kind %d", node_kind[l]);
    SLG_REQUIRE(((uintptr_t)codes[l] % (compact ? 4 : 8)) == 0, SLG_E_ARG,
                "fc_hard_prep_net: codes alignment");
    SLG_REQUIRE(!compact || in_dim[l] <= kMaxCompactIn, SLG_E_SHAPE,
                "fc_hard_prep_net: compact codes need inputs <= %d wide (layer %d)", kMaxCompactIn, l);
    const int vec = (((uintptr_t)cand[l] | (uintptr_t)conn[l] | (uintptr_t)raw[l]) % 16) == 0;
    net.L[l] = HardPrepLayer{cand[l], conn[l], raw[l], reinterpret_cast<uint2*>(codes[l]),
                             (int)in_dim[l], (int)out_dim[l], K[l], node_kind[l], vec};
    net.blk_start[l] = (int)blocks;
    blocks += cdiv(out_dim[l], th);
  }
  net.blk_start[n_layers] = (int)blocks;
  hipLaunchKernelGGL(fc_hard_prep_net_kernel, dim3((unsigned)blocks), dim3(th), 0,
                     as_stream(stream), net, compact ? 1 : 0);
  SLG_LAUNCH_CHECK("fc_hard_prep_net");
  return 0;
}

int slg_fc_hard_layer(const uint64_t* xin, int64_t IN, int64_t nw, const uint32_t* codes,
                      int64_t OUT, uint64_t* xout, slg_stream_t stream) {
  SLG_REQUIRE(codes && ((xin && xout) || nw == 0), SLG_E_ARG, "fc_hard_layer: null pointer");
  SLG_REQUIRE(IN > 0 && nw >= 0 && OUT > 0 && OUT * nw < (1LL << 40) && nw < (1LL << 31),
              SLG_E_SHAPE, "fc_hard_layer: bad sizes");
  if (nw == 0) return 0;
  const int64_t n = OUT * nw;
  hipLaunchKernelGGL(fc_hard_layer_kernel, dim3((unsigned)cdiv(n, 256)), dim3(256), 0,
                     as_stream(stream), xin, (int)nw, reinterpret_cast<const uint2*>(codes),
                     (int)OUT, xout);
  SLG_LAUNCH_CHECK("fc_hard_layer");
  return 0;
}

int slg_fc_hard_place_net(int32_t n_layers, const int64_t* widths, const uint32_t* const* codes,
                          uint32_t* const* placed, int32_t* perm_ws, int64_t perm_ws_len,
                          slg_stream_t stream) {
  SLG_REQUIRE(widths && codes && placed && (perm_ws || n_layers == 1), SLG_E_ARG,
              "fc_hard_place_net: null pointer");
  SLG_REQUIRE(n_layers >= 1 && n_layers <= kMaxLayers, SLG_E_SHAPE,
              "fc_hard_place_net: %d layers", n_layers);
  PlaceNet n{};
  n.L = n_layers;
  int64_t used = 0;
  for (int l = 0; l < n_layers; ++l) {
    SLG_REQUIRE(codes[l] && placed[l] && widths[l] > 0 && widths[l] <= kPlaceMax, SLG_E_SHAPE,
                "fc_hard_place_net: layer %d width %lld outside 1..%d", l, (long long)widths[l],
                kPlaceMax);
    SLG_REQUIRE(codes[l] != placed[l], SLG_E_ARG, "fc_hard_place_net: in place, layer %d", l);
    n.in[l] = codes[l];
    n.out[l] = placed[l];
    n.W[l] = (int)widths[l];
    if (l + 1 < n_layers) {
      n.perm[l] = perm_ws + used;
      used += widths[l];
    }
  }
  SLG_REQUIRE(used <= perm_ws_len, SLG_E_ARG, "fc_hard_place_net: workspace of %lld ints, %lld needed",
              (long long)perm_ws_len, (long long)used);
  hipLaunchKernelGGL(fc_hard_place_kernel, dim3(1), dim3(kPlaceThreads), 0, as_stream(stream), n);
  SLG_LAUNCH_CHECK("fc_hard_place");
  return 0;
}

int64_t slg_fc_hard_type_slots(int64_t IN0, int32_t n_layers, const int64_t* widths) {
  if (!widths || n_layers < 1 || n_layers > kMaxLayers || IN0 < 1 || IN0 > kPlaceMax) return 0;
  int64_t maxw = IN0;
  for (int l = 0; l < n_layers; ++l) {
    if (widths[l] < 1) return 0;
    maxw = std::max<int64_t>(maxw, widths[l]);
  }
  const int maxo = maxw <= kPlaceMax ? pick_maxo(maxw) : 0;
  if (maxo == 0 || net_spw(IN0, n_layers, widths, 1) == 0) return 0;
  return (int64_t)maxo * kNetThreads;
}

int slg_fc_hard_type_place_net(int32_t n_layers, int64_t IN0, const int64_t* widths,
                               const uint32_t* const* codes, uint32_t* const* placed,
                               int32_t* plan, int32_t* perm_ws, int64_t perm_ws_len,
                               slg_stream_t stream) {
  SLG_REQUIRE(widths && codes && placed && plan && perm_ws, SLG_E_ARG,
              "fc_hard_type_place_net: null pointer");
  SLG_REQUIRE(n_layers >= 1 && n_layers <= kMaxLayers, SLG_E_SHAPE,
              "fc_hard_type_place_net: %d layers", n_layers);
  const int64_t S = slg_fc_hard_type_slots(IN0, n_layers, widths);
  SLG_REQUIRE(S > 0, SLG_E_UNSUPPORTED,
              "fc_hard_type_place_net: needs inputs and widths <= %d and a network whose "
              "32-sample column fits LDS", kPlaceMax);
  TypePlaceNet n{};
  n.L = n_layers;
  n.maxo = (int)(S / kNetThreads);
  n.in0 = (int)IN0;
  n.plan = plan;
  int64_t used = 0;
  for (int l = 0; l < n_layers; ++l) {
    SLG_REQUIRE(codes[l] && placed[l], SLG_E_ARG, "fc_hard_type_place_net: null codes, layer %d", l);
    SLG_REQUIRE(codes[l] != placed[l], SLG_E_ARG, "fc_hard_type_place_net: in place, layer %d", l);
    n.in[l] = codes[l];
    n.out[l] = placed[l];
    n.W[l] = (int)widths[l];
    if (l + 1 < n_layers) {
      n.perm[l] = perm_ws + used;
      used += widths[l];
    }
  }
  // the placement's scratch follows the renaming tables
  const int64_t need = slg_fc_hard_type_place_workspace(n_layers, widths);
  SLG_REQUIRE(need > 0 && need <= perm_ws_len && perm_ws, SLG_E_ARG,
              "fc_hard_type_place_net: workspace of %lld ints, %lld needed",
              (long long)perm_ws_len, (long long)need);
  int32_t* sc = perm_ws + used;
  TypePlaceScratch ws{reinterpret_cast<uint32_t*>(sc), sc + kPlaceMax, sc + 2 * kPlaceMax,
                      sc + 3 * kPlaceMax, sc + 4 * kPlaceMax,
                      sc + 4 * kPlaceMax + kTypeMaxGroups};
  hipStream_t st = as_stream(stream);
  const int S_i = (int)S;
  for (int l = 0; l + 1 < n_layers; ++l) {
    hipLaunchKernelGGL(fc_hard_type_plan_kernel, dim3(1), dim3(kPlaceThreads), 0, st, n, ws, l);
    hipLaunchKernelGGL(fc_hard_type_bins_kernel, dim3(2 * 16 + 4), dim3(64), 0, st, n, ws);
    hipLaunchKernelGGL(fc_hard_type_codes_kernel, dim3((unsigned)cdiv(std::max(S_i, n.W[l]), 256)),
                       dim3(256), 0, st, n, ws, l);
  }
  hipLaunchKernelGGL(fc_hard_type_last_kernel, dim3((unsigned)cdiv(S_i, 256)), dim3(256), 0, st, n);
  SLG_LAUNCH_CHECK("fc_hard_type_place");
  return 0;
}

int64_t slg_fc_hard_type_place_workspace(int32_t n_layers, const int64_t* widths) {
  if (!widths || n_layers < 1 || n_layers > kMaxLayers) return -1;
  int64_t perm = 0;
  for (int l = 0; l + 1 < n_layers; ++l) perm += widths[l];
  return perm + kTypeScratchInts;
}

int slg_fc_hard_net_typed(const void* x, int32_t in_kind, int64_t B, int64_t IN0, int32_t n_layers,
                          const int64_t* widths, const uint32_t* const* codes, const int32_t* plan,
                          int32_t C, float* logits, slg_stream_t stream) {
  SLG_REQUIRE(widths && codes && plan && ((x && logits) || B == 0), SLG_E_ARG,
              "fc_hard_net_typed: null pointer");
  SLG_REQUIRE(in_kind >= 0 && in_kind <= 3, SLG_E_ARG, "fc_hard_net_typed: in_kind %d", in_kind);
  SLG_REQUIRE(n_layers >= 1 && n_layers <= kMaxLayers, SLG_E_SHAPE, "fc_hard_net_typed: %d layers",
              n_layers);
  SLG_REQUIRE(B >= 0 && B < (1LL << 31) && IN0 > 0 && IN0 <= kPlaceMax, SLG_E_SHAPE,
              "fc_hard_net_typed: bad sizes");
  const int64_t S = slg_fc_hard_type_slots(IN0, n_layers, widths);
  SLG_REQUIRE(S > 0, SLG_E_UNSUPPORTED, "fc_hard_net_typed: widths do not fit LDS");
  const int spw = net_spw(IN0, n_layers, widths, 1);
  NetDesc d{};
  for (int l = 0; l < n_layers; ++l) {
    SLG_REQUIRE(codes[l], SLG_E_ARG, "fc_hard_net_typed: layer %d", l);
    d.codes[l] = codes[l];
    d.width[l] = (int)widths[l];
  }
  SLG_REQUIRE(C > 0 && C <= 64 && widths[n_layers - 1] % C == 0, SLG_E_SHAPE,
              "fc_hard_net_typed: last width %lld not divisible by %d classes",
              (long long)widths[n_layers - 1], C);
  if (B == 0) return 0;
  d.n_layers = n_layers; d.in0 = (int)IN0; d.C = C; d.wire_r = 0;
  d.maxw = (int)S;
  d.plan = plan;
  const int maxo = (int)(S / kNetThreads);
  const size_t lds = (size_t)2 * d.maxw * (spw / 8);
  hipStream_t st = as_stream(stream);
  // one layer at a small batch: per (word, class) workgroups
  if (use_head(n_layers, 0, in_kind, B, widths[0], C))
    return launch_head((const uint64_t*)x, in_kind, B, IN0, widths[0], C, codes[0], maxo, plan,
                       logits, st);
  return launch_net_any(x, in_kind, (int)B, d, spw, maxo, lds, logits, st);
}

int slg_fc_hard_net_supported(int64_t IN0, int32_t n_layers, const int64_t* widths, int32_t C) {
  if (!widths || n_layers < 1 || n_layers > kMaxLayers || C < 1) return 0;
  if (widths[n_layers - 1] % C != 0) return 0;
  return net_spw(IN0, n_layers, widths, C);
}

int slg_fc_hard_net(const void* x, int32_t in_kind, int64_t B, int64_t IN0, int32_t n_layers,
                    const int64_t* widths, const uint32_t* const* codes, int32_t C, int64_t wire_r,
                    float* logits, slg_stream_t stream) {
  SLG_REQUIRE(widths && codes && ((x && logits) || B == 0), SLG_E_ARG, "fc_hard_net: null pointer");
  SLG_REQUIRE(in_kind >= 0 && in_kind <= 3, SLG_E_ARG, "fc_hard_net: in_kind %d", in_kind);
  SLG_REQUIRE(n_layers >= 1 && n_layers <= kMaxLayers, SLG_E_SHAPE, "fc_hard_net: %d layers", n_layers);
  SLG_REQUIRE(B >= 0 && B < (1LL << 31) && IN0 > 0 && IN0 < (1LL << 28), SLG_E_SHAPE,
              "fc_hard_net: bad sizes");
  NetDesc d{};
  for (int l = 0; l < n_layers; ++l) {
    SLG_REQUIRE(codes[l] && widths[l] > 0 && widths[l] < (1LL << 28), SLG_E_ARG,
                "fc_hard_net: layer %d", l);
    d.codes[l] = codes[l];
    d.width[l] = (int)widths[l];
  }
  SLG_REQUIRE(C > 0 && widths[n_layers - 1] % C == 0, SLG_E_SHAPE,
              "fc_hard_net: last width %lld not divisible by %d classes",
              (long long)widths[n_layers - 1], C);
  const int spw = net_spw(IN0, n_layers, widths, C);
  SLG_REQUIRE(spw > 0, SLG_E_UNSUPPORTED, "fc_hard_net: widths do not fit LDS");
  if (B == 0) return 0;
  d.n_layers = n_layers; d.in0 = (int)IN0; d.C = C; d.wire_r = (int)std::max<int64_t>(0, wire_r);
  int64_t maxw = IN0;
  for (int l = 0; l < n_layers; ++l) maxw = std::max<int64_t>(maxw, widths[l]);
  const int maxo = pick_maxo(maxw);
  SLG_REQUIRE(maxo > 0, SLG_E_UNSUPPORTED, "fc_hard_net: width too large");
  d.maxw = maxo * kNetThreads;
  const size_t lds = (size_t)2 * d.maxw * (spw / 8);
  hipStream_t st = as_stream(stream);
  // one layer at a small batch: per (word, class) workgroups
  if (use_head(n_layers, wire_r, in_kind, B, widths[0], C))
    return launch_head((const uint64_t*)x, in_kind, B, IN0, widths[0], C, codes[0], 0, nullptr,
                       logits, st);
  return launch_net_any(x, in_kind, (int)B, d, spw, maxo, lds, logits, st);
}

int slg_groupsum_packed(const uint64_t* xp, int64_t W, int64_t B, int32_t C, float* logits,
                        slg_stream_t stream) {
  SLG_REQUIRE((xp && logits) || B == 0, SLG_E_ARG, "groupsum_packed: null pointer");
  SLG_REQUIRE(C > 0 && C <= 64 && W > 0 && W % C == 0 && W < (1LL << 31) && B >= 0 &&
                  B < (1LL << 31),
              SLG_E_SHAPE, "groupsum_packed: bad sizes");
  if (B == 0) return 0;
  const int64_t nw = cdiv(B, 64);
  hipLaunchKernelGGL(groupsum_packed_kernel, dim3((unsigned)nw), dim3(256), (size_t)C * 256,
                     as_stream(stream), xp, (int)W, (int)nw, (int)B, C, logits);
  SLG_LAUNCH_CHECK("groupsum_packed");
  return 0;
}

}  // extern "C"
