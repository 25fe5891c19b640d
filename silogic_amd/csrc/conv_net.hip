// The last pooled conv block of a conv network evaluated inside its head,
// on word-major zero-bordered packed images, for gfx950: a one-layer head at
// a small batch (a workgroup per (word, class), only the conv outputs its
// gates read) or the depth-fused head network (a workgroup per word, every
// conv output of the word into LDS, then the layers and the GroupSum).
// Either replaces a conv block launch that writes every output and a head
// launch that reads them back (LogicConvNet.forward_hard, silogic/
// models.py:283-293, heads.py:41-45), with the same logits.
#include "conv_hard_tree.h"
#include "fc_net.h"
#include "slg_common.h"

namespace slg {

constexpr int kConvHeadMaxIn = 1 << 14;   // operand indices of compact codes: 14 bits

// Nodes the kernels here evaluate: gate16 trees of depth 1-3 and LUTs of
// arity 2 to max_arity (the conv block kernel's nodes, gate16 depth 4
// aside): 6 in the head kernel; 4 in the network kernel, whose 1024-thread
// workgroups leave a thread 128 VGPRs, fewer than a LUT5 or LUT6 tree with
// per-lane masks holds.
inline bool conv_node_fuses(int kind, int depth, int arity, int max_arity = 6) {
  return (kind == SLG_NODE_GATE16 && depth >= 1 && depth <= 3) ||
         ((kind == SLG_NODE_MULTILINEAR2 || kind == SLG_NODE_HYBRID) && depth == 1 &&
          arity >= 2 && arity <= max_arity);
}
constexpr int kNetMaxArity = 4;

// The last pooled conv block of a conv network evaluated inside its
// one-layer head (LogicConvNet.forward_hard's last ConvLogicTree + OrPool
// and the head layer + GroupSum, models.py:283-293, heads.py:41-45):
// workgroup (w, c) evaluates the G gates of class c on word w as
// fc_hard_head_kernel does, each operand being the conv block's output
// feature f = n * Ho * Wo + oy * Wo + ox (channel n, pooled position) of
// word w, computed here from the block's input words instead of read from
// the block's output, one operand per lane. Only the 2G conv outputs the
// class reads are evaluated (config 5: 2560 of the block's 16384 per word),
// an operand the gate ignores not at all. A conv output is the same bits as
// conv_hard_wm_kernel's: the same leaf taps of the zero-bordered input
// [nw][C][Hp][Wp], the same tree, the OR of the 2x2 pool window; the
// channel's table is held per lane (lanes take different channels), so LUTs
// take the multiplexer tree, not the block kernel's wave-uniform typed
// branches.
struct ConvTap {
  const uint64_t* xp;        // block input, word-major [nw][C][Hp][Wp], border zero
  const int32_t* leaf;       // [N][NLEAF] leaf codes c << 8 | h << 4 | w
  const uint64_t* tt;        // [N] truth tables
  int C, Hp, Wp, Ho, Wo, kernel;
};

template <int NODE, int NLEAF>
__device__ __forceinline__ uint64_t conv_word_lane(const ConvTap& cv, __amdgpu_buffer_rsrc_t rs,
                                                   int w, int f) {
  constexpr int NM = n_mux_masks<NODE, NLEAF>();
  const int P = cv.Ho * cv.Wo;
  const int n = f / P, p = f - n * P;
  const int oy = p / cv.Wo, ox = p - oy * cv.Wo;
  const int base = (int)(((int64_t)w * cv.C * cv.Hp * cv.Wp + (int64_t)(2 * oy) * cv.Wp + 2 * ox) * 8);
  uint32_t lo[4][NLEAF], hi[4][NLEAF];
#pragma unroll
  for (int l = 0; l < NLEAF; ++l) {
    const int code = cv.leaf[n * NLEAF + l];
    const int lc = min(max(code >> 8, 0), cv.C - 1);
    const int lh = min((code >> 4) & 15, cv.kernel - 1), lw = min(code & 15, cv.kernel - 1);
    const int o = base + ((lc * cv.Hp + lh) * cv.Wp + lw) * 8;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const auto v = __builtin_amdgcn_raw_buffer_load_b64(rs, o + ((q >> 1) * cv.Wp + (q & 1)) * 8, 0, 0);
      lo[q][l] = v[0];
      hi[q][l] = v[1];
    }
  }
  const uint64_t t = cv.tt[n];
  uint32_t ev[NM], es[NM];
  tree_masks_lane<NODE, NLEAF>((uint32_t)t, (uint32_t)(t >> 32), ev, es);
  uint32_t rl = 0, rh = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    rl |= tree_eval32<NODE, NLEAF>(lo[q], ev, es);
    rh |= tree_eval32<NODE, NLEAF>(hi[q], ev, es);
  }
  return ((uint64_t)rh << 32) | rl;
}

template <int NODE, int NLEAF>
__global__ void __launch_bounds__(kHeadThreads)
conv_head_kernel(ConvTap cv, int B, int nw, int in0, int G, int C,
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
  // the block input as one buffer: byte offsets fit 32 bits (checked on the host)
  const __amdgpu_buffer_rsrc_t rs =
      uniform_rsrc(cv.xp, (int)((int64_t)nw * cv.C * cv.Hp * cv.Wp * 8));
  // a pair of lanes per gate: the even lane evaluates operand a, the odd
  // one operand b, and the odd lane's word joins the even lane's by a DPP
  // swap of neighbouring lanes (quad_perm [1,0,3,2])
  const int e = threadIdx.x;
  for (int g0 = 0; g0 < G; g0 += kHeadThreads / 2) {
    const int i = g0 + (e >> 1);
    uint32_t code = 0;
    uint64_t v = 0;
    if (i < G) {
      const int o = c * G + i;
      code = codes[tm ? (o & (kNetThreads - 1)) * tm + (o >> 10) : o];
      const int t4 = (int)(code >> 28);
      const bool second = e & 1;
      if (second ? tt_needs_b(t4) : tt_needs_a(t4)) {
        const int f = second ? (int)(code & 0x3FFFu) : (int)((code >> 14) & 0x3FFFu);
        v = conv_word_lane<NODE, NLEAF>(cv, rs, w, min(f, in0 - 1));
      }
    }
    const uint32_t ol = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)v, 0xB1, 0xF, 0xF, false);
    const uint32_t oh = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)(v >> 32), 0xB1, 0xF, 0xF, false);
    if (!(e & 1) && i < G) cls[i] = gate_compact<uint64_t>(v, ((uint64_t)oh << 32) | ol, code);
  }
  __syncthreads();
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    const int n = class_count<2>(reinterpret_cast<const uint32_t*>(cls), G, lane);
    const int b = w * 64 + lane;
    if (b < B) logits[(int64_t)b * C + c] = (float)n;
  }
}

template <int NODE, int NLEAF>
static int launch_conv_head(const ConvTap& cv, int64_t B, int64_t in0, int64_t width, int C,
                            const uint32_t* codes, int tm, const int32_t* plan, float* logits,
                            hipStream_t st) {
  const int64_t nw = cdiv(B, 64);
  const int G = (int)(width / C);
  hipLaunchKernelGGL((conv_head_kernel<NODE, NLEAF>), dim3((unsigned)nw, (unsigned)C),
                     dim3(kHeadThreads), (size_t)G * 8, st, cv, (int)B, (int)nw, (int)in0, G, C,
                     codes, tm, plan, logits);
  SLG_LAUNCH_CHECK("conv_head");
  return 0;
}

// A conv output of the word whose block input [C][Hp][Wp] is staged in LDS
// at `img`, with the block's leaf codes and tables at `leaf`, `tt`:
// conv_word_lane's taps, tree and pool, read from LDS.
template <int NODE, int NLEAF>
__device__ __forceinline__ uint64_t conv_word_staged(const ConvTap& cv, const uint64_t* img,
                                                     const int32_t* leaf, const uint64_t* tt,
                                                     int f) {
  constexpr int NM = n_mux_masks<NODE, NLEAF>();
  const int P = cv.Ho * cv.Wo;
  const int n = f / P, p = f - n * P;
  const int oy = p / cv.Wo, ox = p - oy * cv.Wo;
  const int base = 2 * oy * cv.Wp + 2 * ox;
  uint32_t lo[4][NLEAF], hi[4][NLEAF];
#pragma unroll
  for (int l = 0; l < NLEAF; ++l) {
    const int code = leaf[n * NLEAF + l];
    const int lc = min(max(code >> 8, 0), cv.C - 1);
    const int lh = min((code >> 4) & 15, cv.kernel - 1), lw = min(code & 15, cv.kernel - 1);
    const uint64_t* q0 = img + base + (lc * cv.Hp + lh) * cv.Wp + lw;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint64_t v = q0[(q >> 1) * cv.Wp + (q & 1)];
      lo[q][l] = (uint32_t)v;
      hi[q][l] = (uint32_t)(v >> 32);
    }
  }
  const uint64_t t = tt[n];
  uint32_t ev[NM], es[NM];
  tree_masks_lane<NODE, NLEAF>((uint32_t)t, (uint32_t)(t >> 32), ev, es);
  uint32_t rl = 0, rh = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    rl |= tree_eval32<NODE, NLEAF>(lo[q], ev, es);
    rh |= tree_eval32<NODE, NLEAF>(hi[q], ev, es);
  }
  return ((uint64_t)rh << 32) | rl;
}

// LDS words behind the activation buffers: one word's block input, the
// block's truth tables and its leaf codes (two to a word).
__host__ __device__ inline int64_t conv_stage_words(int64_t C, int64_t Hp, int64_t Wp, int64_t N,
                                                    int nleaf) {
  return C * Hp * Wp + N + (N * nleaf + 1) / 2;
}

// The fused head network with the last conv block as its input: the
// workgroup of word w stages the word's block input [C][Hp][Wp] and the
// block's tables and leaf codes in LDS behind the two activation buffers
// (one coalesced pass, eight loads in flight per thread), evaluates every
// conv output of the word from them (thread f, f + 1024, ...: the block
// kernel's bits) into activation buffer 0, then runs the layers and the
// GroupSum of fc_hard_net_packed_kernel.
template <int NODE, int NLEAF, int MAXO, bool TYPED>
__global__ void __launch_bounds__(kNetThreads)
conv_net_kernel(NetDesc desc, ConvTap cv, int B, int nw, float* __restrict__ logits) {
  const_netdesc_t& d = *(const_netdesc_t*)__builtin_amdgcn_kernarg_segment_ptr();
  if constexpr (TYPED) {
    if (!plan_fits(d.plan, MAXO, d.in0)) {
      nan_logits(logits, B, d.C);
      return;
    }
  }
  extern __shared__ __align__(16) unsigned char smem[];
  uint64_t* lds = reinterpret_cast<uint64_t*>(smem);
  uint64_t* img = lds + 2 * d.maxw;
  const int tile = blockIdx.x;
  uint32_t cb[MAXO];
  if constexpr (TYPED) load_codes_tm(cb, d.codes[0]);
  else load_codes(cb, d.codes[0], d.width[0]);
  const int n_img = cv.C * cv.Hp * cv.Wp, N = d.in0 / (cv.Ho * cv.Wo);
  uint64_t* s_tt = img + n_img;
  int32_t* s_leaf = reinterpret_cast<int32_t*>(s_tt + N);
  for (int i = threadIdx.x; i < N; i += kNetThreads) s_tt[i] = cv.tt[i];
  for (int i = threadIdx.x; i < N * NLEAF; i += kNetThreads) s_leaf[i] = cv.leaf[i];
  const uint64_t* src = cv.xp + (int64_t)tile * n_img;
  constexpr int U = 8;
  for (int i0 = 0; i0 < n_img; i0 += U * kNetThreads) {
    uint64_t v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = i0 + u * kNetThreads + (int)threadIdx.x;
      v[u] = i < n_img ? src[i] : 0ull;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = i0 + u * kNetThreads + (int)threadIdx.x;
      if (i < n_img) img[i] = v[u];
    }
  }
  __syncthreads();
  for (int f = threadIdx.x; f < d.in0; f += kNetThreads)
    lds[f] = conv_word_staged<NODE, NLEAF>(cv, img, s_leaf, s_tt, f);
  __syncthreads();
  net_tile_layers<uint64_t, MAXO, TYPED>(d, lds, cb, tile, B, logits);
}

// Slots per thread of the fused head network on conv outputs (2 or 4: the
// kernels instantiated here; type-placed codes: their layout's), or 0 where
// it does not apply (64-sample words only, the two activation buffers and
// the staged block input of img_words words in LDS).
inline int conv_net_maxo(int64_t in0, int n_layers, const int64_t* widths, const int32_t* plan,
                         int C, int64_t img_words) {
  if (in0 < 1 || in0 > kConvHeadMaxIn || net_spw(in0, n_layers, widths, C) != 64) return 0;
  int maxo;
  if (plan) {
    maxo = (int)(slg_fc_hard_type_slots(in0, n_layers, widths) / kNetThreads);
  } else {
    int64_t maxw = in0;
    for (int l = 0; l < n_layers; ++l) maxw = std::max<int64_t>(maxw, widths[l]);
    maxo = pick_maxo(maxw);
  }
  if (maxo != 2 && maxo != 4) return 0;
  return (2 * (int64_t)maxo * kNetThreads + img_words) * 8 <= device_lds_bytes() ? maxo : 0;
}

template <int NODE, int NLEAF, int MAXO>
static int launch_conv_net(const ConvTap& cv, int64_t B, const NetDesc& d, float* logits,
                           hipStream_t st) {
  const int64_t nw = cdiv(B, 64);
  const size_t lds =
      ((size_t)2 * d.maxw + (size_t)conv_stage_words(cv.C, cv.Hp, cv.Wp, d.in0 / (cv.Ho * cv.Wo),
                                                      NLEAF)) * 8;
  auto kern = d.plan ? conv_net_kernel<NODE, NLEAF, MAXO, true>
                     : conv_net_kernel<NODE, NLEAF, MAXO, false>;
  if (int rc = set_lds(kern, lds, "conv_hard_net")) return rc;
  hipLaunchKernelGGL(kern, dim3((unsigned)nw), dim3(kNetThreads), lds, st, d, cv, (int)B, (int)nw,
                     logits);
  SLG_LAUNCH_CHECK("conv_hard_net");
  return 0;
}

}  // namespace slg

using namespace slg;

extern "C" {

int slg_conv_hard_head_wm(const uint64_t* xp, int64_t B, int64_t C, int64_t H, int64_t W,
                          int64_t N, int32_t node_kind, int32_t depth, int32_t arity,
                          const int32_t* leaf, const uint64_t* tt, int32_t kernel, int32_t pad,
                          int64_t width, const uint32_t* codes, const int32_t* plan,
                          int32_t n_classes, float* logits, slg_stream_t stream) {
  SLG_REQUIRE(leaf && tt && codes && ((xp && logits) || B == 0), SLG_E_ARG,
              "conv_hard_head_wm: null pointer");
  SLG_REQUIRE(C > 0 && H > 0 && W > 0 && B >= 0 && B < (1LL << 31) && N > 0 && N < 65536 &&
                  kernel >= 1 && kernel <= 15 && pad >= 0 && pad <= 7 && H < 4096 && W < 4096 &&
                  C < (1LL << 23),
              SLG_E_SHAPE, "conv_hard_head_wm: bad conv sizes");
  const int64_t Hf = H + 2 * pad - kernel + 1, Wf = W + 2 * pad - kernel + 1;
  SLG_REQUIRE(Hf > 1 && Wf > 1, SLG_E_SHAPE, "conv_hard_head_wm: empty pooled output");
  const int64_t Ho = Hf / 2, Wo = Wf / 2, nw = cdiv(B, 64);
  const int64_t Hp = H + 2 * pad, Wp = W + 2 * pad, in0 = N * Ho * Wo;
  SLG_REQUIRE(nw * C * Hp * Wp * 8 < (1LL << 31), SLG_E_SHAPE, "conv_hard_head_wm: maps too large");
  SLG_REQUIRE(in0 <= kConvHeadMaxIn, SLG_E_SHAPE,
              "conv_hard_head_wm: %lld conv outputs, compact codes take at most %d",
              (long long)in0, kConvHeadMaxIn);
  SLG_REQUIRE(n_classes > 0 && n_classes <= 64 && width > 0 && width % n_classes == 0 &&
                  width / n_classes <= kHeadMaxG && nw * n_classes < (1LL << 31),
              SLG_E_SHAPE, "conv_hard_head_wm: head width %lld, %d classes", (long long)width,
              n_classes);
  int tm = 0;
  if (plan) {
    const int64_t S = slg_fc_hard_type_slots(in0, 1, &width);
    SLG_REQUIRE(S > 0, SLG_E_UNSUPPORTED, "conv_hard_head_wm: no type-uniform layout here");
    tm = (int)(S / kNetThreads);
  }
  if (B == 0) return 0;
  const ConvTap cv{xp, leaf, tt, (int)C, (int)Hp, (int)Wp, (int)Ho, (int)Wo, kernel};
  hipStream_t st = as_stream(stream);
#define SLG_CH(ND, NL) \
  return launch_conv_head<ND, NL>(cv, B, in0, width, n_classes, codes, tm, plan, logits, st)
  if (node_kind == SLG_NODE_GATE16) {
    switch (depth) {
      case 1: SLG_CH(SLG_NODE_GATE16, 2);
      case 2: SLG_CH(SLG_NODE_GATE16, 4);
      case 3: SLG_CH(SLG_NODE_GATE16, 8);
      default: break;
    }
  } else if ((node_kind == SLG_NODE_MULTILINEAR2 || node_kind == SLG_NODE_HYBRID) && depth == 1) {
    switch (arity) {
      case 2: SLG_CH(SLG_NODE_MULTILINEAR2, 2);
      case 3: SLG_CH(SLG_NODE_MULTILINEAR2, 3);
      case 4: SLG_CH(SLG_NODE_MULTILINEAR2, 4);
      case 5: SLG_CH(SLG_NODE_MULTILINEAR2, 5);
      case 6: SLG_CH(SLG_NODE_MULTILINEAR2, 6);
      default: break;
    }
  }
#undef SLG_CH
  set_error("conv_hard_head_wm: node %d depth %d / arity %d", node_kind, depth, arity);
  return SLG_E_UNSUPPORTED;
}

int slg_hard_step_fuses_head(const slg_hard_step_t* step) {
  if (!step || step->n_conv < 1 || step->n_conv > SLG_STEP_MAX_CONV) return 0;
  const slg_hard_step_t& s = *step;
  const slg_step_conv_t& c = s.conv[s.n_conv - 1];
  if (!conv_node_fuses(c.node_kind, c.depth, c.arity) || s.n_layers < 1 ||
      s.n_layers > kMaxLayers || !s.widths || s.n_classes < 1 || s.head_in != c.out ||
      s.head_in_kind != 3 || c.out_pad != 0 || s.wire_r > 0 || c.kernel < 1 || s.B < 1)
    return 0;
  const int64_t Ho = (c.H + 2 * c.pad - c.kernel + 1) / 2, Wo = (c.W + 2 * c.pad - c.kernel + 1) / 2;
  if (s.head_in_dim != c.N * Ho * Wo) return 0;
  if (use_head(s.n_layers, 0, 3, s.B, s.widths[0], s.n_classes)) return 1;
  const int nleaf = c.node_kind == SLG_NODE_GATE16 ? 1 << c.depth : c.arity;
  const int64_t img = conv_stage_words(c.C, c.H + 2 * c.pad, c.W + 2 * c.pad, c.N, nleaf);
  return conv_node_fuses(c.node_kind, c.depth, c.arity, kNetMaxArity) &&
                 cdiv(s.B, 64) <= device_cus() &&
                 conv_net_maxo(s.head_in_dim, s.n_layers, s.widths, s.plan, s.n_classes, img) > 0
             ? 2
             : 0;
}

int slg_conv_hard_net_wm(const uint64_t* xp, int64_t B, int64_t C, int64_t H, int64_t W,
                         int64_t N, int32_t node_kind, int32_t depth, int32_t arity,
                         const int32_t* leaf, const uint64_t* tt, int32_t kernel, int32_t pad,
                         int32_t n_layers, const int64_t* widths, const uint32_t* const* codes,
                         const int32_t* plan, int32_t n_classes, float* logits,
                         slg_stream_t stream) {
  SLG_REQUIRE(leaf && tt && widths && codes && ((xp && logits) || B == 0), SLG_E_ARG,
              "conv_hard_net_wm: null pointer");
  SLG_REQUIRE(C > 0 && H > 0 && W > 0 && B >= 0 && B < (1LL << 31) && N > 0 && N < 65536 &&
                  kernel >= 1 && kernel <= 15 && pad >= 0 && pad <= 7 && H < 4096 && W < 4096 &&
                  C < (1LL << 23) && n_layers >= 1 && n_layers <= kMaxLayers,
              SLG_E_SHAPE, "conv_hard_net_wm: bad sizes");
  const int64_t Hf = H + 2 * pad - kernel + 1, Wf = W + 2 * pad - kernel + 1;
  SLG_REQUIRE(Hf > 1 && Wf > 1, SLG_E_SHAPE, "conv_hard_net_wm: empty pooled output");
  const int64_t Ho = Hf / 2, Wo = Wf / 2, nw = cdiv(B, 64);
  const int64_t Hp = H + 2 * pad, Wp = W + 2 * pad, in0 = N * Ho * Wo;
  SLG_REQUIRE(nw * C * Hp * Wp * 8 < (1LL << 31), SLG_E_SHAPE, "conv_hard_net_wm: maps too large");
  NetDesc d{};
  for (int l = 0; l < n_layers; ++l) {
    SLG_REQUIRE(codes[l] && widths[l] > 0 && widths[l] <= kConvHeadMaxIn, SLG_E_ARG,
                "conv_hard_net_wm: layer %d", l);
    d.codes[l] = codes[l];
    d.width[l] = (int)widths[l];
  }
  SLG_REQUIRE(n_classes > 0 && n_classes <= 64 && widths[n_layers - 1] % n_classes == 0,
              SLG_E_SHAPE, "conv_hard_net_wm: last width %lld, %d classes",
              (long long)widths[n_layers - 1], n_classes);
  SLG_REQUIRE(conv_node_fuses(node_kind, depth, arity, kNetMaxArity), SLG_E_UNSUPPORTED,
              "conv_hard_net_wm: node %d depth %d / arity %d", node_kind, depth, arity);
  const int nleaf = node_kind == SLG_NODE_GATE16 ? 1 << depth : arity;
  const int maxo = conv_net_maxo(in0, n_layers, widths, plan, n_classes,
                                 conv_stage_words(C, Hp, Wp, N, nleaf));
  SLG_REQUIRE(maxo > 0, SLG_E_UNSUPPORTED,
              "conv_hard_net_wm: needs 64-sample words, %lld conv outputs <= %d, activation "
              "buffers of at most 4096 words and room in LDS for them, the %lld-word block "
              "input and the block's tables", (long long)in0, kConvHeadMaxIn,
              (long long)(C * Hp * Wp));
  if (B == 0) return 0;
  d.n_layers = n_layers; d.in0 = (int)in0; d.C = n_classes; d.wire_r = 0;
  d.maxw = maxo * kNetThreads;
  d.plan = plan;
  const ConvTap cv{xp, leaf, tt, (int)C, (int)Hp, (int)Wp, (int)Ho, (int)Wo, kernel};
  hipStream_t st = as_stream(stream);
#define SLG_CN(ND, NL)                                                          \
  return maxo == 2 ? launch_conv_net<ND, NL, 2>(cv, B, d, logits, st)    \
                   : launch_conv_net<ND, NL, 4>(cv, B, d, logits, st)
  if (node_kind == SLG_NODE_GATE16) {
    switch (depth) {
      case 1: SLG_CN(SLG_NODE_GATE16, 2);
      case 2: SLG_CN(SLG_NODE_GATE16, 4);
      default: SLG_CN(SLG_NODE_GATE16, 8);
    }
  }
  switch (arity) {
    case 2: SLG_CN(SLG_NODE_MULTILINEAR2, 2);
    case 3: SLG_CN(SLG_NODE_MULTILINEAR2, 3);
    default: SLG_CN(SLG_NODE_MULTILINEAR2, 4);
  }
#undef SLG_CN
}

}  // extern "C"
