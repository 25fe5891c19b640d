// Hard conv blocks (ConvLogicTree.forward_hard + OrPool(2), fused) on
// word-major, zero-bordered packed images, for gfx950: the layout of
// LogicConvNet.forward_hard's launch sequence.
//
// Layout: word-major [nw][C][H + 2p][W + 2p] uint64 (word w holds samples
// 64w .. 64w+63, sample b at bit b % 64), the border of width p (the next
// conv's padding) zero. A block writes only the interior of its output, so
// a buffer whose border was cleared once keeps it; with the padding stored,
// every leaf read is unconditional.
//
// One thread per (pooled position, word) of one output channel (the grid's
// y index, so leaf taps and truth tables are uniform). A leaf read is one
// buffer load whose per-thread offset (the position's window corner) is
// fixed and whose uniform offset (the leaf's channel, row, column) goes in
// the instruction's scalar offset: no address arithmetic per leaf.
//
// Node evaluation (silogic/nodes.py:183-189, layers.py:515-527), per 32-bit
// half of a word: gate16 trees and arity-2 LUTs as v_bitop3 multiplexers
// with masks from the table (an arity-k LUT, address sum_j v_j << j, is a
// Shannon tree of 2^k - 1 muxes; a gate16 node is the arity-2 case of its
// 4-bit table, address (a << 1) | b, nodes in table order, level by level).
// LUTs of arity 3-6 are evaluated "typed": the table splits into 2^(k-3)
// bytes, each the 3-input function of leaves 0-2 for one value of the other
// leaves; the wave branches once per byte (uniform: the channel's table) to
// the v_bitop3 whose immediate is that byte, and the bytes' results are
// combined by multiplexers on leaves 3..k-1: 2^(k-3) + 2^(k-3) - 1
// instructions per 32 samples instead of 2^k - 1 (15 instead of 63 at arity
// 6), the same bits.
#include <algorithm>

#include "conv_hard_tree.h"
#include "slg_common.h"

namespace slg {

// Four 3-input functions r[i] = f(a[i], b[i], c[i]), the truth table f the
// wave-uniform byte `type` (entry (a << 2) | (b << 1) | c, the v_bitop3
// operand order): a jump into a table of 256 entries, entry t being the four
// v_bitop3 with immediate t and a branch to the end. An entry is 36 bytes
// (four 8-byte VOP3 instructions and a 4-byte s_branch), so the target is
// table + 36 * type, from s_getpc_b64 (the address of the instruction after
// it). The table is one asm block (.rept over a counter symbol): the
// compiler neither hoists nor duplicates it, and a branch costs a few
// scalar instructions instead of a compare tree. s[40:41] hold the target
// (declared clobbered).
__device__ __forceinline__ void bitop3_dispatch4(uint32_t type, const uint32_t (&a)[4],
                                                 const uint32_t (&b)[4], const uint32_t (&c)[4],
                                                 uint32_t (&r)[4]) {
  uint32_t off;
  asm volatile(
      "s_getpc_b64 s[40:41]\n"
      "slg_base%=:\n"
      "s_mul_i32 %[off], %[type], 36\n"
      "s_add_u32 %[off], %[off], slg_table%= - slg_base%=\n"
      "s_add_u32 s40, s40, %[off]\n"
      "s_addc_u32 s41, s41, 0\n"
      "s_setpc_b64 s[40:41]\n"
      "slg_table%=:\n"
      ".set slg_t%=, 0\n"
      ".rept 256\n"
      "v_bitop3_b32 %[r0], %[a0], %[b0], %[c0] bitop3:slg_t%=\n"
      "v_bitop3_b32 %[r1], %[a1], %[b1], %[c1] bitop3:slg_t%=\n"
      "v_bitop3_b32 %[r2], %[a2], %[b2], %[c2] bitop3:slg_t%=\n"
      "v_bitop3_b32 %[r3], %[a3], %[b3], %[c3] bitop3:slg_t%=\n"
      "s_branch slg_end%=\n"
      ".set slg_t%=, slg_t%= + 1\n"
      ".endr\n"
      "slg_end%=:\n"
      : [r0] "=&v"(r[0]), [r1] "=&v"(r[1]), [r2] "=&v"(r[2]), [r3] "=&v"(r[3]), [off] "=&s"(off)
      : [type] "s"(type & 255u), [a0] "v"(a[0]), [b0] "v"(b[0]), [c0] "v"(c[0]), [a1] "v"(a[1]),
        [b1] "v"(b[1]), [c1] "v"(c[1]), [a2] "v"(a[2]), [b2] "v"(b[2]), [c2] "v"(c[2]),
        [a3] "v"(a[3]), [b3] "v"(b[3]), [c3] "v"(c[3])
      : "scc", "s40", "s41");
}

// An arity-A LUT (3 <= A <= 6) per evaluation, table T (uniform): byte m of
// T is the 3-input function of leaves 2, 1, 0 where leaves 3.. spell m. The
// bytes are taken in order and combined as a binary counter with one pending
// value per level: leaf 3 + j selects between two results whose m differ in
// bit j (the upper one is the current result).
template <int NV, int A>
__device__ __forceinline__ void lut_typed(uint64_t T, const uint32_t (&v)[NV][A],
                                          uint32_t (&res)[NV]) {
  static_assert(NV % 4 == 0, "evaluations go in fours");
  constexpr int NB = 1 << (A - 3);
  uint32_t S[A > 3 ? A - 3 : 1][NV];
#pragma unroll 1
  for (int m = 0; m < NB; ++m) {
    const uint32_t type = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(T >> (8 * m)));
    uint32_t r[NV];
#pragma unroll
    for (int g = 0; g < NV / 4; ++g) {
      uint32_t a[4], b[4], c[4], o[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        a[i] = v[4 * g + i][2];
        b[i] = v[4 * g + i][1];
        c[i] = v[4 * g + i][0];
      }
      bitop3_dispatch4(type, a, b, c, o);
#pragma unroll
      for (int i = 0; i < 4; ++i) r[4 * g + i] = o[i];
    }
    bool carry = true;
#pragma unroll
    for (int j = 0; j < A - 3; ++j) {
      if (carry) {
        if ((m >> j) & 1) {
#pragma unroll
          for (int i = 0; i < NV; ++i) r[i] = mux32(v[i][3 + j], r[i], S[j][i]);
        } else {
#pragma unroll
          for (int i = 0; i < NV; ++i) S[j][i] = r[i];
          carry = false;
        }
      }
    }
    if (carry) {
#pragma unroll
      for (int i = 0; i < NV; ++i) res[i] = r[i];
    }
  }
}

template <int NODE, int NLEAF>
constexpr bool typed_lut() {
  return NODE != SLG_NODE_GATE16 && NLEAF >= 3;
}

template <int NODE, int NLEAF>
__global__ void __launch_bounds__(256)
conv_hard_wm_kernel(const uint64_t* __restrict__ xp, int C, int H, int W, int nw, int N,
                    const int* __restrict__ leaf, const uint64_t* __restrict__ tt, int kernel,
                    int pad, uint64_t* __restrict__ out, int Ho, int Wo, int opad) {
  constexpr int NM = n_mux_masks<NODE, NLEAF>();
  constexpr bool TYPED = typed_lut<NODE, NLEAF>();
  const int n = blockIdx.y;
  const int P = Ho * Wo;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const bool active = i < (int64_t)P * nw;
  const int w = active ? (int)(i / P) : 0, p = active ? (int)(i - (int64_t)w * P) : 0;
  const int oy = p / Wo, ox = p - oy * Wo;
  const int Hp = H + 2 * pad, Wp = W + 2 * pad;
  const int64_t CHWp = (int64_t)C * Hp * Wp;
  // the input as one buffer: byte offsets fit 32 bits (checked on the host)
  const __amdgpu_buffer_rsrc_t rs = uniform_rsrc(xp, (int)(nw * CHWp * 8));
  // the window corner of the pooled output, padded coordinates (2 oy, 2 ox)
  int vq[4];
#pragma unroll
  for (int q = 0; q < 4; ++q)
    vq[q] = (int)(((int64_t)w * CHWp + (int64_t)(2 * oy + (q >> 1)) * Wp + 2 * ox + (q & 1)) * 8);
  uint32_t lo[4][NLEAF], hi[4][NLEAF];
#pragma unroll
  for (int l = 0; l < NLEAF; ++l) {
    const int code = __builtin_amdgcn_readfirstlane(leaf[(int64_t)n * NLEAF + l]);
    const int lc = min(max(code >> 8, 0), C - 1);
    const int lh = min((code >> 4) & 15, kernel - 1), lw = min(code & 15, kernel - 1);
    const int so = ((lc * Hp + lh) * Wp + lw) * 8;   // uniform: the instruction's scalar offset
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const auto v = __builtin_amdgcn_raw_buffer_load_b64(rs, vq[q], so, 0);
      lo[q][l] = v[0];
      hi[q][l] = v[1];
    }
  }
  const uint32_t tlo = __builtin_amdgcn_readfirstlane((uint32_t)tt[n]);
  const uint32_t thi = __builtin_amdgcn_readfirstlane((uint32_t)(tt[n] >> 32));
  uint32_t rlo[4], rhi[4];
  if constexpr (TYPED) {
    uint32_t v[8][NLEAF], r[8];
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int l = 0; l < NLEAF; ++l) {
        v[q][l] = lo[q][l];
        v[4 + q][l] = hi[q][l];
      }
    lut_typed<8, NLEAF>(((uint64_t)thi << 32) | tlo, v, r);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      rlo[q] = r[q];
      rhi[q] = r[4 + q];
    }
  } else {
    uint32_t ev[NM], es[NM];
    tree_masks<NODE, NLEAF>(tlo, thi, ev, es);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      rlo[q] = tree_eval32<NODE, NLEAF>(lo[q], ev, es);
      rhi[q] = tree_eval32<NODE, NLEAF>(hi[q], ev, es);
    }
  }
  const uint64_t acc = ((uint64_t)(rhi[0] | rhi[1] | rhi[2] | rhi[3]) << 32) |
                       (rlo[0] | rlo[1] | rlo[2] | rlo[3]);
  if (active) {
    const int Hq = Ho + 2 * opad, Wq = Wo + 2 * opad;
    out[((int64_t)w * N + n) * Hq * Wq + (int64_t)(oy + opad) * Wq + ox + opad] = acc;
  }
}

// Packing of [B, C, H, W] images (fp32: x >= 1, bytes: x != 0; the
// pack_bits rule) into the zero-bordered word-major layout: the interior of
// [nw][C][H + 2p][W + 2p] (the border is left as it is). A workgroup takes
// one word and 64 V pixels; its four waves take the word's four 16-sample
// quarters, a lane V consecutive pixels of one row (V = 4: W % 4 == 0, read
// as one vector per sample), and each lane writes its 16 bits of each word
// as one 2-byte store. (A lane taking all 64 samples of its pixels gave a
// quarter of the workgroups: config 3's 24 MB packed at 3.3 TB/s.)
template <typename T, int V>
__global__ void __launch_bounds__(256)
pack_image_kernel(const T* __restrict__ x, int B, int C, int H, int W, int pad, int nw, int dtiles,
                  uint64_t* __restrict__ xp) {
  const int lane = threadIdx.x & 63;
  const int D = C * H * W;
  const int w = (int)(blockIdx.x / (uint32_t)dtiles);
  const int q = (int)(threadIdx.x >> 6);                 // quarter of the word
  const int d0 = (int)(blockIdx.x % (uint32_t)dtiles) * 64 * V + lane * V;
  if (w >= nw || d0 >= D) return;                        // no barriers below
  const int nr = min(64, B - w * 64);                    // samples of the word
  const int r0 = 16 * q;
  int src[V];
#pragma unroll
  for (int v = 0; v < V; ++v) src[v] = min(d0 + v, D - 1);  // tail lanes: stores are guarded
  auto bit = [](T v) {
    if constexpr (sizeof(T) == 1) return v != 0;
    else return v >= (T)1;
  };
  const T* xr = x + (int64_t)w * 64 * D;
  uint32_t m[V];
#pragma unroll
  for (int v = 0; v < V; ++v) m[v] = 0;
  // rows past the word's samples read its last row; their bits are cleared
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const T* row = xr + (int64_t)min(r0 + i, nr - 1) * D;
    if constexpr (V == 4) {
      if constexpr (sizeof(T) == 1) {
        const uint32_t v4 = *reinterpret_cast<const uint32_t*>(row + src[0]);
#pragma unroll
        for (int v = 0; v < 4; ++v) m[v] |= (bit((T)(v4 >> (8 * v))) ? 1u : 0u) << i;
      } else {
        const float4 v4 = *reinterpret_cast<const float4*>(row + src[0]);
        const float qv[4] = {v4.x, v4.y, v4.z, v4.w};
#pragma unroll
        for (int v = 0; v < 4; ++v) m[v] |= (bit(qv[v]) ? 1u : 0u) << i;
      }
    } else {
#pragma unroll
      for (int v = 0; v < V; ++v) m[v] |= (bit(row[src[v]]) ? 1u : 0u) << i;
    }
  }
  const int valid = max(0, min(16, nr - r0));
  const uint32_t keep = valid == 16 ? 0xFFFFu : (1u << valid) - 1u;
  const int Hp = H + 2 * pad, Wp = W + 2 * pad;
  uint16_t* dst = reinterpret_cast<uint16_t*>(xp + (int64_t)w * C * Hp * Wp);
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const int d = d0 + v;
    if (d < D) {
      const int c = d / (H * W), r = d - c * H * W, y = r / W, xx = r - y * W;
      dst[(((int64_t)c * Hp + y + pad) * Wp + xx + pad) * 4 + q] = (uint16_t)(m[v] & keep);
    }
  }
}

template <int NODE, int NLEAF>
static int launch_conv_hard_wm(const uint64_t* xp, int64_t nw, int64_t C, int64_t H, int64_t W,
                               int64_t N, const int* leaf, const uint64_t* tt, int kernel, int pad,
                               uint64_t* out, int64_t Ho, int64_t Wo, int opad, hipStream_t st) {
  const int64_t n = Ho * Wo * nw;
  hipLaunchKernelGGL((conv_hard_wm_kernel<NODE, NLEAF>), dim3((unsigned)cdiv(n, 256), (unsigned)N),
                     dim3(256), 0, st, xp, (int)C, (int)H, (int)W, (int)nw, (int)N, leaf, tt, kernel,
                     pad, out, (int)Ho, (int)Wo, opad);
  SLG_LAUNCH_CHECK("conv_hard_wm");
  return 0;
}

}  // namespace slg

using namespace slg;

extern "C" {

int slg_conv_hard_fwd_wm(const uint64_t* xp, int64_t B, int64_t C, int64_t H, int64_t W, int64_t N,
                         int32_t node_kind, int32_t depth, int32_t arity, const int32_t* leaf,
                         const uint64_t* tt, int32_t kernel, int32_t pad, uint64_t* out,
                         int32_t out_pad, slg_stream_t stream) {
  SLG_REQUIRE(leaf && tt && ((xp && out) || B == 0), SLG_E_ARG, "conv_hard_wm: null pointer");
  SLG_REQUIRE(C > 0 && H > 0 && W > 0 && B >= 0 && B < (1LL << 31) && N > 0 && N < 65536 &&
                  kernel >= 1 && kernel <= 15 && pad >= 0 && pad <= 7 && out_pad >= 0 &&
                  out_pad <= 7 && H < 4096 && W < 4096 && C < (1LL << 23),
              SLG_E_SHAPE, "conv_hard_wm: bad sizes");
  const int64_t Hf = H + 2 * pad - kernel + 1, Wf = W + 2 * pad - kernel + 1;
  SLG_REQUIRE(Hf > 1 && Wf > 1, SLG_E_SHAPE, "conv_hard_wm: empty pooled output");
  const int64_t Ho = Hf / 2, Wo = Wf / 2, nw = cdiv(B, 64);
  // the input is one buffer resource with 32-bit byte offsets
  SLG_REQUIRE(nw * C * (H + 2 * pad) * (W + 2 * pad) * 8 < (1LL << 31) &&
                  nw * N * (Ho + 2 * out_pad) * (Wo + 2 * out_pad) < (1LL << 40),
              SLG_E_SHAPE, "conv_hard_wm: maps too large");
  if (B == 0) return 0;
  hipStream_t st = as_stream(stream);
#define SLG_CHW(ND, NL)                                                                    \
  return launch_conv_hard_wm<ND, NL>(xp, nw, C, H, W, N, leaf, tt, kernel, pad, out, Ho, Wo, \
                                     out_pad, st)
  if (node_kind == SLG_NODE_GATE16) {
    switch (depth) {
      case 1: SLG_CHW(SLG_NODE_GATE16, 2);
      case 2: SLG_CHW(SLG_NODE_GATE16, 4);
      case 3: SLG_CHW(SLG_NODE_GATE16, 8);
      case 4: SLG_CHW(SLG_NODE_GATE16, 16);
      default: break;
    }
  } else if ((node_kind == SLG_NODE_MULTILINEAR2 || node_kind == SLG_NODE_HYBRID) && depth == 1) {
    switch (arity) {
      case 2: SLG_CHW(SLG_NODE_MULTILINEAR2, 2);
      case 3: SLG_CHW(SLG_NODE_MULTILINEAR2, 3);
      case 4: SLG_CHW(SLG_NODE_MULTILINEAR2, 4);
      case 5: SLG_CHW(SLG_NODE_MULTILINEAR2, 5);
      case 6: SLG_CHW(SLG_NODE_MULTILINEAR2, 6);
      default: break;
    }
  }
#undef SLG_CHW
  set_error("conv_hard_wm: node %d depth %d / arity %d", node_kind, depth, arity);
  return SLG_E_UNSUPPORTED;
}

int slg_pack_image_wm(const void* x, int32_t dtype, int64_t B, int64_t C, int64_t H, int64_t W,
                      int32_t pad, uint64_t* xp, slg_stream_t stream) {
  SLG_REQUIRE((x && xp) || B == 0, SLG_E_ARG, "pack_image_wm: null pointer");
  SLG_REQUIRE(dtype == 0 || dtype == 1, SLG_E_ARG, "pack_image_wm: dtype %d", dtype);
  SLG_REQUIRE(B >= 0 && B < (1LL << 31) && C > 0 && H > 0 && W > 0 && pad >= 0 && pad <= 7 &&
                  C * H * W < (1LL << 31) && cdiv(B, 64) * C * (H + 2 * pad) * (W + 2 * pad) < (1LL << 40),
              SLG_E_SHAPE, "pack_image_wm: bad sizes");
  if (B == 0) return 0;
  const int64_t nw = cdiv(B, 64), D = C * H * W;
  const size_t esz = dtype == 0 ? 4 : 1;
  const bool vec = W % 4 == 0 && (uintptr_t)x % (4 * esz) == 0;
  const int64_t dtiles = cdiv(D, vec ? 256 : 64);
  SLG_REQUIRE(nw * dtiles < (1LL << 31), SLG_E_SHAPE, "pack_image_wm: too many tiles");
  dim3 grid((unsigned)(nw * dtiles));
  hipStream_t st = as_stream(stream);
#define SLG_PI(T, V)                                                                          \
  hipLaunchKernelGGL((pack_image_kernel<T, V>), grid, dim3(256), 0, st, (const T*)x, (int)B,  \
                     (int)C, (int)H, (int)W, (int)pad, (int)nw, (int)dtiles, xp)
  if (dtype == 0) {
    if (vec) SLG_PI(float, 4); else SLG_PI(float, 1);
  } else {
    if (vec) SLG_PI(uint8_t, 4); else SLG_PI(uint8_t, 1);
  }
#undef SLG_PI
  SLG_LAUNCH_CHECK("pack_image_wm");
  return 0;
}

}  // extern "C"
