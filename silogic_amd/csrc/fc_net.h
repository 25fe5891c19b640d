// The depth-fused hard FC network's device code (layer steps, type-uniform
// rows, GroupSum) and its host-side shape rules, shared by the network
// kernels of fc_hard.hip and the conv-block-and-head kernels of
// conv_net.hip.
#pragma once
#include <algorithm>

#include "slg_common.h"

namespace slg {

// ---------------------------------------------------------------------------
// depth-fused FC network + GroupSum
// ---------------------------------------------------------------------------
// One workgroup of 1024 threads owns a column of SPW samples (a 64- or 32-bit
// word per feature) and keeps the whole activation column in LDS, ping-
// ponging between two buffers of max-width words, through every layer. Per
// layer each thread owns outputs tid, tid+1024, ...: it holds their codes in
// registers (prefetched one layer ahead: codes do not depend on the data),
// reads its two operand words from LDS and writes the result word. The
// GroupSum counts are bit-sliced sums (carry-save adders and lane
// butterflies) per class.
constexpr int kMaxLayers = 16;
constexpr int kNetThreads = 1024;
struct NetDesc {
  const uint32_t* codes[kMaxLayers];  // compact codes, one word per output
  int width[kMaxLayers];
  int n_layers, in0, C, wire_r;
  int maxw;  // words per activation buffer: MAXO * 1024 (every row of every layer)
  const int32_t* plan;  // type-uniform layout ([n_layers][kPlanStride]), or null
};
// The network kernels take the descriptor as their first argument and read
// it through the kernel-argument segment (constant memory): its per-layer
// arrays are indexed by the layer number, and read that way the loads stay
// scalar instead of going through a private copy of the struct.
typedef __attribute__((address_space(4))) const NetDesc const_netdesc_t;

// Codes of this thread's outputs o = tid + j*1024 of a W-wide layer, read
// through a raw buffer resource of W codes: offsets past it read 0 (a valid
// code), so the loads need no clamp.
template <int MAXO>
__device__ inline void load_codes(uint32_t (&cb)[MAXO], const uint32_t* __restrict__ codes, int W) {
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint32_t*>(codes), (short)0, W * 4, kBufferWord3);
  const int v = threadIdx.x * 4;
#pragma unroll
  for (int j = 0; j < MAXO; ++j) cb[j] = __builtin_amdgcn_raw_buffer_load_b32(r, v + j * kNetThreads * 4, 0, 0);
}

// Codes of a placed (type-uniform) layer, stored thread-major: the MAXO
// codes of thread tid are contiguous at tid * MAXO, so one address register
// and immediate offsets read them (the wave's loads stay contiguous).
template <int MAXO>
__device__ inline void load_codes_tm(uint32_t (&cb)[MAXO], const uint32_t* __restrict__ codes) {
  const uint32_t* p = codes + threadIdx.x * MAXO;
#pragma unroll
  for (int j = 0; j < MAXO; ++j) cb[j] = p[j];
}

__device__ inline uint32_t bfi32(uint32_t m, uint32_t x, uint32_t y) { return (m & x) | (~m & y); }

// gate16 on words from a compact code: T_g = all-ones iff tt bit g, read by
// a sign-extending 1-bit field extract; out = a ? (b ? T3 : T2) : (b ? T1 : T0).
template <typename WT>
__device__ inline WT gate_compact(WT a, WT b, uint32_t c) {
  const uint32_t t0 = (uint32_t)__builtin_amdgcn_sbfe((int)c, 28, 1);
  const uint32_t t1 = (uint32_t)__builtin_amdgcn_sbfe((int)c, 29, 1);
  const uint32_t t2 = (uint32_t)__builtin_amdgcn_sbfe((int)c, 30, 1);
  const uint32_t t3 = (uint32_t)__builtin_amdgcn_sbfe((int)c, 31, 1);
  if constexpr (sizeof(WT) == 8) {
    const uint32_t al = (uint32_t)a, ah = (uint32_t)(a >> 32);
    const uint32_t bl = (uint32_t)b, bh = (uint32_t)(b >> 32);
    const uint32_t lo = bfi32(al, bfi32(bl, t3, t2), bfi32(bl, t1, t0));
    const uint32_t hi = bfi32(ah, bfi32(bh, t3, t2), bfi32(bh, t1, t0));
    return ((uint64_t)hi << 32) | lo;
  } else {
    return bfi32(a, bfi32(b, t3, t2), bfi32(b, t1, t0));
  }
}

// Operand reads are issued at raised wave priority. Every wave of the
// workgroup is in the same phase of a layer (a barrier ends each one), so
// the waves that still have LDS reads to issue would otherwise wait behind
// those already computing gates; with the reads first, the LDS queue fills
// sooner and the gate math overlaps it (config 2's fused network 63.2 ->
// 61.4 us, the same bits).
__device__ __forceinline__ void reads_begin() { __builtin_amdgcn_s_setprio(1); }
__device__ __forceinline__ void reads_end() { __builtin_amdgcn_s_setprio(0); }

// One layer on the LDS column: lds[nxt + o] = gate_o(lds[cur + a_o], lds[cur + b_o])
// for this thread's outputs o = tid + j*1024, in groups of GRP outputs: all
// operand reads of a group are issued before its results are computed, so
// the LDS latency of a thread's gates overlaps; the group's gate math runs
// between its reads and its writes, with no LDS access in between. Each
// buffer holds MAXO*1024 words, so every row of a group is computed and
// written without a mask: rows past the layer have code 0 (read past the
// codes' buffer resource) and write their word into the buffer's unused
// tail. Operand indices are below the layer's input width by construction
// (the prep kernel clamps them). Groups wholly past the layer are skipped.
template <typename WT, int MAXO, int GRP>
__device__ __forceinline__ void layer_step(WT* lds, int cur, int nxt, int W,
                                           const uint32_t (&cb)[MAXO]) {
  static_assert(MAXO % GRP == 0, "groups must tile MAXO");
  const int rows = (W + kNetThreads - 1) / kNetThreads;
  const WT* src = lds + cur;
  WT* dst = lds + nxt + threadIdx.x;
#pragma unroll
  for (int g0 = 0; g0 < MAXO; g0 += GRP) {
    if (g0 >= rows) break;                               // wave-uniform
    WT va[GRP], vb[GRP];
    reads_begin();
#pragma unroll
    for (int u = 0; u < GRP; ++u) {
      const uint32_t c = cb[g0 + u];
      va[u] = src[(c >> 14) & 0x3FFFu];
      vb[u] = src[c & 0x3FFFu];
    }
    reads_end();
    // all gate math, then all writes: no LDS access between the computes
    WT r[GRP];
#pragma unroll
    for (int u = 0; u < GRP; ++u) r[u] = gate_compact<WT>(va[u], vb[u], cb[g0 + u]);
#pragma unroll
    for (int u = 0; u < GRP; ++u) dst[(g0 + u) * kNetThreads] = r[u];
  }
}

// ---------------------------------------------------------------------------
// type-uniform rows
// ---------------------------------------------------------------------------
// With a placement plan (slg_fc_hard_type_place_net) the first U rows of a
// layer hold, in each wave, outputs of one gate type: wave w computes gate
// tt[w] in rows 0..U-1 and generic gates (compact codes) in rows U..rows-1.
// A wave then branches once per layer to code specialised for its gate, where
// a 32-bit half of an output word is one v_bitop3 with the truth table as
// immediate (or nothing: constants and pass-throughs), and gates that ignore
// an operand do not read it. A uniform row's code is (a << 16) | b with a, b
// word indices counted from the start of the first activation buffer (the
// read buffer's offset included), so an operand's LDS byte address is one
// v_mad_u32_u16 (16-bit field x word size + LDS base).
// per layer: U, rows, truth table of waves 0..15, then the slots per thread
// (MAXO) and the input width the layout was placed for
constexpr int kPlanStride = 20;

// tt bit k = output for address k = (a << 1) | b (compact-code order)
__host__ __device__ constexpr bool tt_needs_a(int tt) { return (tt & 3) != (tt >> 2); }
__host__ __device__ constexpr bool tt_needs_b(int tt) { return (tt & 5) != ((tt >> 1) & 5); }
// v_bitop3 truth table of (a, b, 0): entry (a << 2 | b << 1 | c) = tt bit (a << 1 | b)
__host__ __device__ constexpr uint32_t tt_bitop3(int tt) {
  return ((tt & 1) ? 0x03u : 0u) | ((tt & 2) ? 0x0Cu : 0u) | ((tt & 4) ? 0x30u : 0u) |
         ((tt & 8) ? 0xC0u : 0u);
}

template <int TT>
__device__ __forceinline__ uint32_t gate_tt32(uint32_t a, uint32_t b) {
  if constexpr (TT == 0) return 0u;
  else if constexpr (TT == 15) return 0xFFFFFFFFu;
  else if constexpr (TT == 12) return a;
  else if constexpr (TT == 10) return b;
  else if constexpr (TT == 3) return ~a;
  else if constexpr (TT == 5) return ~b;
  else return __builtin_amdgcn_bitop3_b32(a, b, 0u, (unsigned char)tt_bitop3(TT));
}

template <int TT, typename WT>
__device__ __forceinline__ WT gate_tt(WT a, WT b) {
  if constexpr (sizeof(WT) == 8) {
    const uint32_t lo = gate_tt32<TT>((uint32_t)a, (uint32_t)b);
    const uint32_t hi = gate_tt32<TT>((uint32_t)(a >> 32), (uint32_t)(b >> 32));
    return ((uint64_t)hi << 32) | lo;
  } else {
    return gate_tt32<TT>(a, b);
  }
}

typedef __attribute__((address_space(3))) uint32_t lds_u32_t;
typedef __attribute__((address_space(3))) uint64_t lds_u64_t;

// LDS byte address of word (c >> 16) (HI) or (c & 0xFFFF) of words of SZ bytes
// counted from LDS byte `base`
template <int SZ, bool HI>
__device__ __forceinline__ uint32_t field_addr(uint32_t c, uint32_t base) {
  uint32_t r;
  if constexpr (SZ == 8 && HI) asm("v_mad_u32_u16 %0, %1, 8, %2 op_sel:[1,0,0,0]" : "=v"(r) : "v"(c), "s"(base));
  else if constexpr (SZ == 8) asm("v_mad_u32_u16 %0, %1, 8, %2" : "=v"(r) : "v"(c), "s"(base));
  else if constexpr (HI) asm("v_mad_u32_u16 %0, %1, 4, %2 op_sel:[1,0,0,0]" : "=v"(r) : "v"(c), "s"(base));
  else asm("v_mad_u32_u16 %0, %1, 4, %2" : "=v"(r) : "v"(c), "s"(base));
  return r;
}

template <typename WT>
__device__ __forceinline__ WT lds_word(uint32_t addr) {
  if constexpr (sizeof(WT) == 8) return *(const lds_u64_t*)(uintptr_t)addr;
  else return *(const lds_u32_t*)(uintptr_t)addr;
}

// Rows [g0, g0 + N) of gate TT: every operand read first, then `between`
// (work that overlaps the reads), then the gates, then the writes.
struct NoWork {
  __device__ void operator()() const {}
};

template <typename WT, int MAXO, int TT, int N, typename F = NoWork>
__device__ __forceinline__ void uniform_group(uint32_t base, WT* dst, int g0,
                                              const uint32_t (&cb)[MAXO], F&& between = F()) {
  constexpr int SZ = (int)sizeof(WT);
  WT va[N], vb[N];
  reads_begin();
#pragma unroll
  for (int u = 0; u < N; ++u) {
    va[u] = vb[u] = (WT)0;
    if constexpr (tt_needs_a(TT)) va[u] = lds_word<WT>(field_addr<SZ, true>(cb[g0 + u], base));
    if constexpr (tt_needs_b(TT)) vb[u] = lds_word<WT>(field_addr<SZ, false>(cb[g0 + u], base));
  }
  reads_end();
  between();
  WT r[N];
#pragma unroll
  for (int u = 0; u < N; ++u) r[u] = gate_tt<TT, WT>(va[u], vb[u]);
#pragma unroll
  for (int u = 0; u < N; ++u) dst[(g0 + u) * kNetThreads] = r[u];
}

// A group of N = 1..GRP-1 rows at g0 (N wave-uniform), as one batch.
template <typename WT, int MAXO, int TT, int G0, int N>
__device__ __forceinline__ void uniform_tail(uint32_t base, WT* dst, int n,
                                             const uint32_t (&cb)[MAXO]) {
  if constexpr (N >= 1 && G0 + N <= MAXO) {
    if (n == N) uniform_group<WT, MAXO, TT, N>(base, dst, G0, cb);
    else uniform_tail<WT, MAXO, TT, G0, N - 1>(base, dst, n, cb);
  }
}

// Rows 0..U-1 of a wave of gate TT (U wave-uniform), in groups of GRP rows
// and one shorter group for the rest.
template <typename WT, int MAXO, int GRP, int TT, int G0 = 0>
__device__ __forceinline__ void uniform_rows(uint32_t base, WT* dst, int U,
                                             const uint32_t (&cb)[MAXO]) {
  if constexpr (G0 < MAXO) {
    if (G0 + GRP <= U) {
      uniform_group<WT, MAXO, TT, GRP>(base, dst, G0, cb);
      uniform_rows<WT, MAXO, GRP, TT, G0 + GRP>(base, dst, U, cb);
    } else if (U > G0) {
      uniform_tail<WT, MAXO, TT, G0, GRP - 1>(base, dst, U - G0, cb);
    }
  }
}

// Generic rows J..rows-1 (U == J) from compact codes, one at a time; the
// compile-time start keeps the register indexing static.
template <typename WT, int MAXO, int J>
__device__ __forceinline__ void generic_rows(const WT* src, WT* dst, int U, int rows,
                                             const uint32_t (&cb)[MAXO]) {
  if constexpr (J <= MAXO) {
    if (U != J) {
      generic_rows<WT, MAXO, J + 1>(src, dst, U, rows, cb);
      return;
    }
#pragma unroll
    for (int j = J; j < MAXO; ++j) {
      if (j >= rows) break;                              // wave-uniform
      const uint32_t c = cb[j];
      reads_begin();
      const WT a = src[(c >> 14) & 0x3FFFu], b = src[c & 0x3FFFu];
      reads_end();
      dst[j * kNetThreads] = gate_compact<WT>(a, b, c);
    }
  }
}

// The usual plan, U = MAXO - 1 and rows = MAXO: uniform rows in groups of
// GRP, the last group read and computed in one batch with the generic row
// MAXO - 1. No branch inside. `filler` (the layer's input-row work) runs
// while the first group's reads are in flight.
template <typename WT, int MAXO, int GRP, int TT, typename F>
__device__ __forceinline__ void typed_rows_full(uint32_t base, const WT* src, WT* dst,
                                                const uint32_t (&cb)[MAXO], F&& filler) {
  constexpr int SZ = (int)sizeof(WT);
  constexpr int LG = ((MAXO - 2) / GRP) * GRP;       // first row of the last group
  constexpr int N = MAXO - 1 - LG;                   // its uniform rows (>= 1)
  if constexpr (LG >= GRP) uniform_group<WT, MAXO, TT, GRP>(base, dst, 0, cb, filler);
  else filler();
#pragma unroll
  for (int g0 = GRP; g0 < LG; g0 += GRP) uniform_group<WT, MAXO, TT, GRP>(base, dst, g0, cb);
  WT va[N], vb[N];
  reads_begin();
#pragma unroll
  for (int u = 0; u < N; ++u) {
    va[u] = vb[u] = (WT)0;
    if constexpr (tt_needs_a(TT)) va[u] = lds_word<WT>(field_addr<SZ, true>(cb[LG + u], base));
    if constexpr (tt_needs_b(TT)) vb[u] = lds_word<WT>(field_addr<SZ, false>(cb[LG + u], base));
  }
  const uint32_t c = cb[MAXO - 1];
  const WT ga = src[(c >> 14) & 0x3FFFu], gb = src[c & 0x3FFFu];
  reads_end();
  WT r[N];
#pragma unroll
  for (int u = 0; u < N; ++u) r[u] = gate_tt<TT, WT>(va[u], vb[u]);
#pragma unroll
  for (int u = 0; u < N; ++u) dst[(LG + u) * kNetThreads] = r[u];
  dst[(MAXO - 1) * kNetThreads] = gate_compact<WT>(ga, gb, c);
}

// A layer's plan as the wave reads it: U, the rows computed, its truth
// table. The plan is read as constant memory, so its loads are scalar: a
// vector load would retire in order behind the layer's input-row loads and
// wait for them.
typedef __attribute__((address_space(4))) const int32_t const_i32_t;

struct PlanRow {
  int U, rows, tt;
};

// The codes of a placed layout are read at a stride of MAXO slots, which
// follows the input width it was placed for: a plan placed for another
// width or slot count would index past its codes, so the network kernels
// check the plan's own record first and write NaN logits instead.
__device__ __forceinline__ bool plan_fits(const int32_t* plan, int maxo, int in0) {
  const const_i32_t* pl = (const const_i32_t*)plan;
  return __builtin_amdgcn_readfirstlane(pl[18]) == maxo &&
         __builtin_amdgcn_readfirstlane(pl[19]) == in0;
}

__device__ inline void nan_logits(float* __restrict__ logits, int B, int C) {
  const int64_t n = (int64_t)B * C, step = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += step)
    logits[i] = __int_as_float(0x7FC00000);
}

__device__ __forceinline__ PlanRow plan_row(const int32_t* plan, int l) {
  const const_i32_t* pl = (const const_i32_t*)(plan + l * kPlanStride);
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  return {__builtin_amdgcn_readfirstlane(pl[0]), __builtin_amdgcn_readfirstlane(pl[1]),
          __builtin_amdgcn_readfirstlane(pl[2 + wave])};
}

// One layer of a planned network: the wave's uniform rows, then rows
// U..rows-1 from compact codes (as layer_step).
template <typename WT, int MAXO, int GRP, typename F>
__device__ __forceinline__ void typed_step(WT* lds, int cur, int nxt, PlanRow pr,
                                           const uint32_t (&cb)[MAXO], F&& filler) {
  const int U = pr.U, rows = pr.rows, tt = pr.tt;
  const uint32_t base = (uint32_t)(uintptr_t)lds;
  const WT* src = lds + cur;
  WT* dst = lds + nxt + threadIdx.x;
  if (MAXO > 1 && U == MAXO - 1 && rows == MAXO) {
    switch (tt & 15) {
#define SLG_TT_CASE(T) \
      case T: typed_rows_full<WT, MAXO, GRP, T>(base, src, dst, cb, filler); break;
      SLG_TT_CASE(0) SLG_TT_CASE(1) SLG_TT_CASE(2) SLG_TT_CASE(3)
      SLG_TT_CASE(4) SLG_TT_CASE(5) SLG_TT_CASE(6) SLG_TT_CASE(7)
      SLG_TT_CASE(8) SLG_TT_CASE(9) SLG_TT_CASE(10) SLG_TT_CASE(11)
      SLG_TT_CASE(12) SLG_TT_CASE(13) SLG_TT_CASE(14) SLG_TT_CASE(15)
#undef SLG_TT_CASE
    }
    return;
  }
  filler();
  switch (tt & 15) {
#define SLG_TT_CASE(T) \
    case T: uniform_rows<WT, MAXO, GRP, T>(base, dst, U, cb); break;
    SLG_TT_CASE(0) SLG_TT_CASE(1) SLG_TT_CASE(2) SLG_TT_CASE(3)
    SLG_TT_CASE(4) SLG_TT_CASE(5) SLG_TT_CASE(6) SLG_TT_CASE(7)
    SLG_TT_CASE(8) SLG_TT_CASE(9) SLG_TT_CASE(10) SLG_TT_CASE(11)
    SLG_TT_CASE(12) SLG_TT_CASE(13) SLG_TT_CASE(14) SLG_TT_CASE(15)
#undef SLG_TT_CASE
  }
  generic_rows<WT, MAXO, 0>(src, dst, U, rows, cb);
}

// wire residual (models.py:88-94): the first `keep` outputs copy the inputs
template <typename WT, int MAXO>
__device__ inline void keep_inputs(WT* lds, int cur, int nxt, int keep) {
#pragma unroll
  for (int j = 0; j < MAXO; ++j) {
    const int o = threadIdx.x + j * kNetThreads;
    if (o < keep) lds[nxt + o] = lds[cur + o];
  }
}

// Per-class sample counts without a bit transpose. One wave takes a class:
// for 64-bit words lanes 0..31 count the low 32 samples and lanes 32..63 the
// high 32, each lane carry-save adding (Harley-Seal) the half-words of 32
// words into a bit-sliced 6-bit count per sample (slice k holds bit k of
// every sample's count); five butterfly rounds inside each 32-lane group
// then add the lanes' bit-sliced counts (ripple-carry adders on the slices),
// after which every lane of a group holds its 32 samples' class totals in
// 11 slices and lane s reads its own bits. 32-bit words take 16 words per
// lane over all 64 lanes and a sixth round across the two groups. The
// exchanges are DPP moves and permlane swaps, no LDS; words past the class
// read 0; every lane of the wave must be active.
// Majority and 3-input xor as one v_bitop3 each (truth tables 0xE8 and
// 0x96, both symmetric in their inputs).
__device__ __forceinline__ uint32_t maj3(uint32_t a, uint32_t b, uint32_t c) {
  return __builtin_amdgcn_bitop3_b32(a, b, c, 0xE8);
}
__device__ __forceinline__ uint32_t xor3(uint32_t a, uint32_t b, uint32_t c) {
  return __builtin_amdgcn_bitop3_b32(a, b, c, 0x96);
}

__device__ __forceinline__ void csa(uint32_t& h, uint32_t& l, uint32_t a, uint32_t b, uint32_t c) {
  h = maj3(a, b, c);
  l = xor3(a, b, c);
}

constexpr int kGsSlices = 12;   // bit slices of a lane's counts (at most 2048)

// Harley-Seal step over 16 words: ones..eights carry across calls, the
// 16s word of this block is returned.
__device__ __forceinline__ uint32_t hs16(uint32_t& ones, uint32_t& twos, uint32_t& fours,
                                         uint32_t& eights, const uint32_t* w) {
  uint32_t twosA, twosB, foursA, foursB, eightsA, eightsB, sixteens;
  csa(twosA, ones, ones, w[0], w[1]);
  csa(twosB, ones, ones, w[2], w[3]);
  csa(foursA, twos, twos, twosA, twosB);
  csa(twosA, ones, ones, w[4], w[5]);
  csa(twosB, ones, ones, w[6], w[7]);
  csa(foursB, twos, twos, twosA, twosB);
  csa(eightsA, fours, fours, foursA, foursB);
  csa(twosA, ones, ones, w[8], w[9]);
  csa(twosB, ones, ones, w[10], w[11]);
  csa(foursA, twos, twos, twosA, twosB);
  csa(twosA, ones, ones, w[12], w[13]);
  csa(twosB, ones, ones, w[14], w[15]);
  csa(foursB, twos, twos, twosA, twosB);
  csa(eightsB, fours, fours, foursA, foursB);
  csa(sixteens, eights, eights, eightsA, eightsB);
  return sixteens;
}

// Bit-sliced add x += y of NB-bit counts (x[NB] is 0 on entry and takes the
// carry out): a ripple of full adders, slice by slice.
template <int NB>
__device__ __forceinline__ void add_slices(uint32_t (&x)[kGsSlices], const uint32_t (&y)[kGsSlices]) {
  uint32_t carry = 0;
#pragma unroll
  for (int k = 0; k < NB; ++k) {
    const uint32_t t = xor3(x[k], y[k], carry);
    carry = maj3(x[k], y[k], carry);
    x[k] = t;
  }
  x[NB] = carry;
}

// Butterfly step within 16-lane rows by a DPP lane pattern: quad_perm
// [1,0,3,2] (lane ^ 1), [2,3,0,1] (lane ^ 2), then row_half_mirror (lane i of
// 8 with 7 - i: joins the two quads' totals) and row_mirror (i of 16 with
// 15 - i: joins the two 8-lane totals).
template <int NB, int CTRL>
__device__ __forceinline__ void add_dpp(uint32_t (&x)[kGsSlices]) {
  uint32_t y[kGsSlices];
#pragma unroll
  for (int k = 0; k < NB; ++k) y[k] = (uint32_t)__builtin_amdgcn_mov_dpp((int)x[k], CTRL, 0xF, 0xF, false);
  add_slices<NB>(x, y);
}

// Butterfly step across 16- or 32-lane halves: v_permlane16/32_swap of a
// value with itself returns, in every lane, the lane's own value and that of
// lane ^ 16 (^ 32) as the pair (a, b), so the sum is a + b.
template <int NB, bool P32>
__device__ __forceinline__ void add_swap(uint32_t (&x)[kGsSlices]) {
  uint32_t a[kGsSlices], b[kGsSlices];
#pragma unroll
  for (int k = 0; k < NB; ++k) {
    if constexpr (P32) {
      const auto r = __builtin_amdgcn_permlane32_swap(x[k], x[k], false, false);
      a[k] = r[0];
      b[k] = r[1];
    } else {
      const auto r = __builtin_amdgcn_permlane16_swap(x[k], x[k], false, false);
      a[k] = r[0];
      b[k] = r[1];
    }
  }
#pragma unroll
  for (int k = 0; k < NB; ++k) x[k] = a[k];
  x[NB] = 0;
  add_slices<NB>(x, b);
}

// Class total of this lane's sample over the class's G words `cls32`
// (32-bit halves, NH per word): sample lane for NH == 2, lane & 31 for
// NH == 1. A pass takes WPL words per lane: 32 for 64-bit words (1024 words
// per pass); 16 or 32 for 32-bit words (1024 or 2048 words per pass: one
// butterfly for classes of up to 2048 words, where 1024-word passes would
// take two).
template <int NH, int WPL1 = 16>
__device__ __forceinline__ int class_count(const uint32_t* cls32, int G, int lane) {
  constexpr int WPL = NH == 2 ? 32 : WPL1;               // words per lane per pass
  constexpr int LSTRIDE = NH == 2 ? 32 : 64;             // word stride between them
  constexpr int CHUNK = WPL * LSTRIDE;                   // words per pass
  constexpr int NBITS = (NH == 1 && WPL == 32) ? 12 : 11;  // slices of the pass's total
  static_assert(WPL == 16 || WPL == 32, "16 or 32 words per lane");
  const int l = NH == 2 ? (lane & 31) : lane;
  const int h = NH == 2 ? (lane >> 5) : 0;
  int total = 0;
  for (int q0 = 0; q0 < G; q0 += CHUNK) {
    // rows of the pass wholly inside the class load without a lane guard
    // (a wave-uniform test); only the class's last partial row is guarded
    const int nvalid = G - q0;
    const uint32_t* p = cls32 + (q0 + l) * NH + h;
    uint32_t w[WPL];
    reads_begin();
#pragma unroll
    for (int j = 0; j < WPL; ++j) {
      if (j * LSTRIDE + LSTRIDE <= nvalid) w[j] = p[j * LSTRIDE * NH];
      else w[j] = j * LSTRIDE + l < nvalid ? p[j * LSTRIDE * NH] : 0u;
    }
    reads_end();
    uint32_t x[kGsSlices];
#pragma unroll
    for (int k = 0; k < kGsSlices; ++k) x[k] = 0;
    if constexpr (WPL == 32) {
      const uint32_t s16a = hs16(x[0], x[1], x[2], x[3], w);
      const uint32_t s16b = hs16(x[0], x[1], x[2], x[3], w + 16);
      x[4] = s16a ^ s16b;
      x[5] = s16a & s16b;
      // 6 bits (<= 32) grow one bit per round: 11 (<= 1024) after five
      // rounds inside each 32-lane group, 12 (<= 2048) after the sixth
      add_dpp<6, 0xB1>(x);    // quad_perm [1,0,3,2]
      add_dpp<7, 0x4E>(x);    // quad_perm [2,3,0,1]
      add_dpp<8, 0x141>(x);   // row_half_mirror
      add_dpp<9, 0x140>(x);   // row_mirror
      add_swap<10, false>(x);  // lane ^ 16
      if constexpr (NH == 1) add_swap<11, true>(x);  // lane ^ 32
    } else {
      x[4] = hs16(x[0], x[1], x[2], x[3], w);
      add_dpp<5, 0xB1>(x);
      add_dpp<6, 0x4E>(x);
      add_dpp<7, 0x141>(x);
      add_dpp<8, 0x140>(x);
      add_swap<9, false>(x);
      add_swap<10, true>(x);  // lane ^ 32
    }
    const int sh = lane & 31;
    int cnt = 0;
#pragma unroll
    for (int k = 0; k < NBITS; ++k) cnt |= (int)((x[k] >> sh) & 1u) << k;
    total += cnt;
  }
  return total;
}

// Per-class popcounts of a tile written as logits: one wave per class.
template <typename WT>
__device__ __forceinline__ void groupsum_tile(const WT* cur, int W, int C, int b0, int B,
                                              float* __restrict__ logits) {
  constexpr int NH = (int)sizeof(WT) / 4;                // 32-sample halves per word
  constexpr int SPW = NH * 32;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nwaves = kNetThreads >> 6;
  const int G = W / C;
  for (int c = wave; c < C; c += nwaves) {
    const uint32_t* cls = reinterpret_cast<const uint32_t*>(cur + c * G);
    const int n = (NH == 1 && G > 1024) ? class_count<NH, 32>(cls, G, lane)
                                        : class_count<NH>(cls, G, lane);
    const int b = b0 + lane;
    if (lane < SPW && b < B) logits[(int64_t)b * C + c] = (float)n;
  }
}


// The layers and the GroupSum of one tile whose input words are in LDS
// (buffer 0, after a barrier): per layer the next layer's codes (and plan
// row) load while this one computes, a barrier ends each layer, and the
// last layer's buffer is counted per class into the logits of samples
// tile * SPW ... `cb` holds layer 0's codes.
template <typename WT, int MAXO, bool TYPED>
__device__ __forceinline__ void net_tile_layers(const_netdesc_t& d, WT* lds, uint32_t (&cb)[MAXO],
                                                int tile, int B, float* __restrict__ logits) {
  constexpr int SPW = (int)sizeof(WT) * 8;
  int cur = 0, nxt = d.maxw, cur_w = d.in0;
  const int L = d.n_layers;
  // typed: plan row and next codes pointer scalar-loaded a layer ahead
  PlanRow pc{};
  const uint32_t* cn = nullptr;
  if constexpr (TYPED) {
    pc = plan_row(d.plan, 0);
    cn = d.codes[L > 1 ? 1 : 0];
  }
  for (int l = 0; l < L; ++l) {
    const int W = d.width[l];
    uint32_t nb[MAXO];
    const int ln = (l + 1 < L) ? l + 1 : l;
    if constexpr (TYPED) {
      load_codes_tm(nb, cn);
      const PlanRow pn = plan_row(d.plan, ln);
      const uint32_t* cnn = d.codes[(ln + 1 < L) ? ln + 1 : ln];
      typed_step<WT, MAXO, (MAXO % 2 == 0 && MAXO > 4) ? MAXO / 2 : MAXO>(
          lds, cur, nxt, pc, cb, NoWork());
      pc = pn;
      cn = cnn;
    } else {
      load_codes(nb, d.codes[ln], d.width[ln]);
      layer_step<WT, MAXO, MAXO>(lds, cur, nxt, W, cb);
      if (d.wire_r > 0 && cur_w == W) keep_inputs<WT, MAXO>(lds, cur, nxt, min(d.wire_r, W));
    }
    __syncthreads();
    const int t = cur; cur = nxt; nxt = t;
    cur_w = W;
#pragma unroll
    for (int j = 0; j < MAXO; ++j) cb[j] = nb[j];
  }
  groupsum_tile<WT>(lds + cur, cur_w, d.C, tile * SPW, B, logits);
}

// One-layer heads at small batches take a workgroup per (word, class)
// (fc_hard_head_kernel, conv_head_kernel).
constexpr int kHeadThreads = 256;
constexpr int kHeadMaxG = 8192;   // a class's gate words in 64 KiB of LDS

// Whether a one-layer network on packed words takes fc_hard_head_kernel:
// fewer sample words than half the CUs (the fused kernel's workgroups), no
// wire residual, a class in LDS.
inline bool use_head(int n_layers, int64_t wire_r, int in_kind, int64_t B, int64_t width, int C) {
  return n_layers == 1 && wire_r <= 0 && in_kind >= 2 && B > 0 &&
         2 * cdiv(B, 64) < device_cus() && width / C <= kHeadMaxG;
}

inline int pick_maxo(int64_t maxw) {
  const int64_t m = cdiv(maxw, kNetThreads);
  for (int c : {2, 4, 8, 10, 16})
    if (m <= c) return c;
  return 0;
}

inline int net_spw(int64_t IN0, int n_layers, const int64_t* widths, int C) {
  if (!widths || n_layers < 1 || n_layers > kMaxLayers || C < 1 || C > 64) return 0;
  int64_t maxw = IN0;
  for (int l = 0; l < n_layers; ++l) maxw = std::max<int64_t>(maxw, widths[l]);
  if (maxw > 16 * kNetThreads) return 0;
  const int64_t words = (int64_t)pick_maxo(maxw) * kNetThreads;  // per activation buffer
  const int64_t lds = device_lds_bytes();
  if (2 * words * 8 <= lds) return 64;
  if (2 * words * 4 <= lds) return 32;
  return 0;
}


template <typename K>
inline int set_lds(K kern, size_t lds, const char* what) {
  hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                     (int)lds);
  if (e != hipSuccess) {
    set_error("%s: LDS %zu: %s", what, lds, hipGetErrorString(e));
    return (int)e;
  }
  return 0;
}

}  // namespace slg
