/*
 * silogic_hip.h — C ABI of the MI355X (gfx950) gate-layer library
 * (libsilogic_hip.so).
 *
 * Conventions for every entry point:
 *   - All array pointers are DEVICE pointers owned by the caller, dense
 *     row-major (C order) unless stated. Sizes are int64_t.
 *   - `stream` is a hipStream_t passed as void* (0 = the null stream). Entry
 *     points enqueue work on it and return without host synchronisation.
 *   - Return 0 on success, a negative SLG_E_* code for a rejected argument or
 *     shape (nothing is launched), or a positive hipError_t from the launch.
 *     slg_last_error() returns a thread-local message for the last failure.
 *   - No entry point allocates device memory. Intermediates live in
 *     registers or LDS, or in arrays the caller passes: outputs, and for the
 *     soft backward a workspace whose size slg_fc_soft_bwd_workspace gives.
 *   - Floating-point math is IEEE fp32 (no fast-math); hard paths are exact.
 *
 * Bit-packed layout ("packed"): a [D, nw] array of uint64 words,
 * nw = ceil(B / 64); sample b of feature d is bit (b % 64) of word
 * [d, b / 64]. Byte-identical to the reference's int64 layout
 * (silogic/bitpacking/ops.py:1-49). Conv activations are [C, H, W, nw]
 * (the reference's B-packed [C, H*W, nw], packed_layer.py:184-214).
 *
 * Per-output hard FC code ("slg_code2", 8 bytes): x = index of input a,
 * y = (index of input b) | (tt << 28), where bit g of the 4-bit tt is the
 * gate output at address g = (a << 1) | b (silogic/nodes.py:100-106).
 */
#ifndef SILOGIC_HIP_H
#define SILOGIC_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* slg_stream_t;

enum {
  SLG_OK = 0,
  SLG_E_ARG = -1,        /* null pointer / invalid enum */
  SLG_E_SHAPE = -2,      /* size out of the supported range */
  SLG_E_UNSUPPORTED = -3 /* valid but not implemented combination */
};

/* node kinds of the FC soft kernel */
enum {
  SLG_NODE_GATE16 = 0,      /* y = c0 + c1 a + c2 b + c3 ab, param = coef [OUT,4] */
  SLG_NODE_WALSH = 1,       /* y = sigmoid((c0 + c1 a + c2 b + c3 ab) * inv_tau)  */
  SLG_NODE_MULTILINEAR2 = 2, /* y = sum_P s_P prod_j(...), param = sigmoid(l) [OUT,4] */
  SLG_NODE_HYBRID = 3        /* conv LUT trees: y = s[addr of leaves >= 0.5], gradient of the
                                multilinear form (nodes.py:198-206) */
};

const char* slg_last_error(void);
int slg_version(void);
/* number of compute units of the current device (for launch sizing) */
int slg_device_cus(void);

/* ---------------------------------------------------------------------- */
/* FC soft forward                                                          */
/* ---------------------------------------------------------------------- */

/* Replaces silogic/kernels/dense.py:123-125 `dense_logic(x, ca, cb, wa, wb,
 * coef)` (called at silogic/layers.py:121-122): x [B,IN] fp32, ca/cb [OUT,K]
 * int32, wa/wb [OUT,K] fp32 post-softmax weights, coef [OUT,4]; out [B,OUT]
 * = c0 + c1 a + c2 b + c3 ab with a = sum_k wa[o,k] x[b, ca[o,k]]. */
int slg_dense_logic_fwd(const float* x, int64_t B, int64_t IN, int64_t OUT, int32_t K,
                        const int32_t* ca, const int32_t* cb, const float* wa,
                        const float* wb, const float* coef, float* out,
                        slg_stream_t stream);

/* Replaces silogic/kernels/warp.py:104-105 `warp_logic(x, ca, cb, wa, wb,
 * coef, inv_tau)` (called at silogic/layers.py:123): as dense_logic, then
 * out = sigmoid(z * inv_tau). */
int slg_warp_logic_fwd(const float* x, int64_t B, int64_t IN, int64_t OUT, int32_t K,
                       const int32_t* ca, const int32_t* cb, const float* wa,
                       const float* wb, const float* coef, float inv_tau, float* out,
                       slg_stream_t stream);

/* General FC soft layer on the module's native layouts (replaces the
 * LogicLayer._fused dispatch, silogic/layers.py:111-123, for gate16, walsh
 * and multilinear arity 2): cand [OUT,2,K] int32, w [OUT,2,K] fp32,
 * node_param [OUT,4] (coef for gate16/walsh, sigmoid(logits) for
 * multilinear2). tile_samples / threads: 0 = automatic. */
int slg_fc_soft_fwd(const float* x, int64_t B, int64_t IN, int64_t OUT, int32_t K,
                    const int32_t* cand, const float* w, int32_t node_kind,
                    const float* node_param, float inv_tau, float* out,
                    int32_t tile_samples, int32_t threads, slg_stream_t stream);

/* Soft parameter preparation for one FC layer (replaces the torch ops of
 * TopKConnectome.weights, connectomes.py:114-119, and Gate16Node.coef /
 * WalshNode.coef, nodes.py:82-84,138-143; sigmoid(logits), nodes.py:178):
 *   conn [OUT,2,K] -> w = softmax over K;
 *   gate16: raw [OUT,16] -> coef = softmax(raw) @ BASIS;
 *   walsh:  raw [OUT,4] theta -> coef (change of variables);
 *   multilinear2: raw [OUT,4] logits -> sigmoid(raw).
 * conn may be NULL (K=1 fixed wiring: w = 1). */
int slg_fc_soft_prep(const float* conn, int64_t OUT, int32_t K, int32_t node_kind,
                     const float* raw, float* w, float* node_param, slg_stream_t stream);

/* The soft parameters of n_layers (<= 16) FC layers in one launch, as one
 * record per output of RQ = (3K+3)/4 + 1 quads of 32-bit words: K words
 * idx_a[k] | idx_b[k] << 16 (clamped into [0, in_dim), in_dim <= 65536),
 * w_a[K], w_b[K] (fp32 softmax over K), zeros up to quad RQ-1, then
 * node_param[4] (fp32, as slg_fc_soft_prep) in quad RQ-1, in a chunk-major
 * layout: quad q of output o at quad index ((o / 64) * RQ + q) * 64 + o % 64.
 * rec[l] holds ceil(out_dim/64)*64
 * records (the padding repeats the last output). The inputs of layer l are
 * cand[l] [out_dim,2,K] int32, conn[l] [out_dim,2,K] (NULL = fixed wiring)
 * and raw[l] as in slg_fc_soft_prep; order (may be NULL, or hold NULLs) gives
 * per layer a gather order [out_dim,2,K] uint8 from slg_fc_soft_schedule:
 * step t of slot s reads candidate order[o][s][t]. Host arrays of device
 * pointers, as slg_fc_hard_net's codes. Replaces, for a whole LogicNet, the
 * per-forward torch ops of TopKConnectome.weights (connectomes.py:114-119)
 * and the node coefficients (nodes.py:82-84, 138-143, 178). */
int slg_fc_soft_records(int32_t n_layers, const int32_t* const* cand, const float* const* conn,
                        const float* const* raw, const int64_t* in_dim, const int64_t* out_dim,
                        int32_t K, const int32_t* node_kind, const uint8_t* const* order,
                        float* const* rec, slg_stream_t stream);

/* Bank-aware gather order for one layer's candidates cand [OUT,2,K] int32
 * (K <= 16) read from an IN-wide input: order [OUT,2,K] uint8, a
 * permutation of 0..K-1 per (output, slot) that spreads the LDS reads of
 * each step over distinct banks. Depends only on cand and IN, so a caller
 * computes it once per candidate table. No counterpart in the reference
 * (its kernels read candidates in index order); results change only by the
 * fp32 summation order. */
int slg_fc_soft_schedule(const int32_t* cand, int64_t OUT, int32_t K, int64_t IN, uint8_t* order,
                         slg_stream_t stream);

/* slg_fc_soft_fwd on records from slg_fc_soft_records (the forward of
 * LogicLayer, layers.py:107-123, without gradients). rec_in_dim is the
 * in_dim the records were built for; x [B, IN] must have IN >= rec_in_dim
 * (else SLG_E_SHAPE: the reference's x[:, cand] raises there). */
int slg_fc_soft_fwd_records(const float* x, int64_t B, int64_t IN, int64_t OUT, int32_t K,
                            const float* rec, int64_t rec_in_dim, int32_t node_kind,
                            float inv_tau, float* out, int32_t tile_samples, int32_t threads,
                            slg_stream_t stream);

/* The last LogicLayer of a LogicNet fused with its GroupSum head with the
 * feature STE (layers.py:107-123 then heads.py:34-39, as models.py:96-97
 * runs them): logits [B,C] = per-class count of (y > 0.5) / tau; the layer
 * output y is not written. Exact: the counts are integers. Returns
 * SLG_E_UNSUPPORTED when slg_fc_soft_groupsum_supported says 0. */
int slg_fc_soft_fwd_groupsum(const float* x, int64_t B, int64_t IN, int64_t OUT, int32_t K,
                             const float* rec, int64_t rec_in_dim, int32_t node_kind,
                             float inv_tau, int32_t C, float tau, float* logits,
                             slg_stream_t stream);
/* A network of soft FC layers on records in one launch (the soft forward of
 * LogicNet / WARPNet, models.py:96-101): rec[l] from slg_fc_soft_records
 * for in_dim[l] inputs, layer l with out_dim[l] outputs, all layers of one
 * node kind, K candidates and inv_tau. x [B, IN] fp32 (IN >= in_dim[0]). A
 * workgroup takes a tile of samples through every layer with the
 * activations in LDS, so only x and the result touch HBM: narrow layers and
 * small batches keep two buffers of 4-sample slots; wide layers (K = 8) and
 * batches that give every CU a tile keep one buffer of 4 or 2 samples and
 * hold a layer's outputs in registers until every wave has read its input.
 * Each layer computes as slg_fc_soft_fwd_records does (the same bits). C > 0:
 * the last layer feeds the STE GroupSum head and out = logits [B, C] (counts
 * of y > 0.5 / tau); C = 0: out = the last layer's activations
 * [B, out_dim[n_layers-1]]. SLG_E_UNSUPPORTED when neither kernel takes the
 * shapes (slg_fc_soft_net_supported says 0). */
int slg_fc_soft_net_records(const float* x, int64_t B, int64_t IN, int32_t n_layers,
                            const float* const* rec, const int64_t* in_dim,
                            const int64_t* out_dim, int32_t K, int32_t node_kind, float inv_tau,
                            int32_t C, float tau, float* out, slg_stream_t stream);
/* Which kernel slg_fc_soft_net_records runs for these shapes, where it is
 * the faster path: 1 = two LDS buffers (every activation buffer fits LDS
 * twice, batches below two 8-sample tiles per CU), 2 = one LDS buffer (K =
 * 8, widths whose 4- or 2-sample tile fits LDS, at least one tile per CU);
 * 0 = a launch per layer (slg_fc_soft_fwd_records). */
int slg_fc_soft_net_supported(int64_t B, int64_t IN, int32_t n_layers, const int64_t* out_dim,
                              int32_t K, int32_t C);
/* 1 if slg_fc_soft_fwd_groupsum runs this shape (one workgroup holds every
 * output of its sample tile), else 0. */
int slg_fc_soft_groupsum_supported(int64_t B, int64_t IN, int64_t OUT, int32_t C);

/* Soft FC backward (replaces DenseLogicFn.backward and WarpLogicFn.backward,
 * kernels/dense.py:46-75, 107-120 and warp.py:33-64, plus the arity-2
 * multilinear node of nodes.py:174-178): for the layer of slg_fc_soft_fwd
 * (cand [OUT,2,K] int32, w [OUT,2,K], node_param [OUT,4]) and dL/dy = gy
 * [B,OUT], writes dL/dx into gx [B,IN], dL/dw into gw [OUT,2,K] and
 * dL/dnode_param into gnp [OUT,4]; any of the three may be NULL (not
 * computed). No atomics on values: every sum runs in a fixed order, so the
 * three gradients are the same bits on every call (the reference adds gx
 * with atomics). workspace: caller-owned device memory of at least
 * slg_fc_soft_bwd_workspace(B, IN, OUT, K) floats; that function returns
 * -1 for shapes the kernels do not take (IN beyond what LDS holds). */
int64_t slg_fc_soft_bwd_workspace(int64_t B, int64_t IN, int64_t OUT, int32_t K);
int slg_fc_soft_bwd(const float* x, int64_t B, int64_t IN, int64_t OUT, int32_t K,
                    const int32_t* cand, const float* w, int32_t node_kind,
                    const float* node_param, float inv_tau, const float* gy, float* gx,
                    float* gw, float* gnp, float* workspace, int64_t workspace_floats,
                    slg_stream_t stream);

/* FC layers of n-input LUT nodes, arity 2..6, Top-K (K <= 8) or fixed (K = 1)
 * wiring: the multilinear node (nodes.py:165-189, arity != 2 or any arity)
 * and the DWN-style hybrid node (nodes.py:198-206; replaces the fused op
 * multilinear_logic, kernels/multilinear.py:123-160). cand/w [OUT,n,K]
 * (w: softmax of the connection logits; 1 for fixed wiring), s [OUT,2^n]
 * (sigmoid of the node logits), leaf j = address bit j.
 * Forward: y [B,OUT] = multilinear interpolation of s at the operands, or
 * (hybrid) s at the address of the operands thresholded at 0.5. workspace:
 * slg_fc_lut_soft_workspace(OUT, n, K) floats. */
int64_t slg_fc_lut_soft_workspace(int64_t OUT, int32_t arity, int32_t K);
int slg_fc_lut_soft_fwd(const float* x, int64_t B, int64_t IN, int64_t OUT, int32_t arity,
                        int32_t K, const int32_t* cand, const float* w, const float* s,
                        int32_t hybrid, float* y, float* workspace, int64_t workspace_floats,
                        slg_stream_t stream);
/* slg_fc_lut_soft_fwd without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops,
 * harnesses that forbid hipMalloc); no counterpart in the reference. The
 * records live in a static device array of the library (16 MiB per GPU,
 * held until the process ends): layers needing more than 4 Mi record floats
 * (slg_fc_lut_soft_workspace; about 26 000 outputs at arity 6, K = 8) are
 * rejected with SLG_E_SHAPE. Every call on one GPU uses that GPU's one
 * array, so calls that overlap on a GPU (different streams or threads) race;
 * calls in one stream are ordered and safe. Allocates nothing. */
int slg_fc_lut_soft_fwd_noalloc(const float* x, int64_t B, int64_t IN, int64_t OUT,
                                int32_t arity, int32_t K, const int32_t* cand, const float* w,
                                const float* s, int32_t hybrid, float* y, slg_stream_t stream);
/* Backward of both (the gradient of the multilinear form, the hybrid node's
 * surrogate): gy [B,OUT] -> gx [B,IN], gw [OUT,n,K], gs [OUT,2^n]; any of the
 * three may be NULL. Every sum runs in a fixed order (the reference adds gx
 * with atomics). workspace: slg_fc_lut_soft_bwd_workspace(...) floats, -1 for
 * shapes not taken (IN beyond what LDS holds). */
int64_t slg_fc_lut_soft_bwd_workspace(int64_t B, int64_t IN, int64_t OUT, int32_t arity,
                                      int32_t K);
int slg_fc_lut_soft_bwd(const float* x, int64_t B, int64_t IN, int64_t OUT, int32_t arity,
                        int32_t K, const int32_t* cand, const float* w, const float* s,
                        const float* gy, float* gx, float* gw, float* gs, float* workspace,
                        int64_t workspace_floats, slg_stream_t stream);
/* Hard codes of such a layer for slg_fc_lut_hard (LogicLayer.forward_hard,
 * layers.py:131-135 with nodes.py:180-187): idx [OUT,n] = per slot the first
 * candidate with the largest connection logit (conn NULL: K = 1), tt [OUT]
 * bit p = (logits[o][p] > 0). */
int slg_fc_lut_hard_prep(const int32_t* cand, const float* conn, int64_t OUT, int32_t arity,
                         int32_t K, int64_t IN, const float* logits, int32_t* idx, uint64_t* tt,
                         slg_stream_t stream);

/* Input encoders (the step before the gate layers). Thermometer codes of
 * x [B,D] (dtype 0: fp32; 1: uint8 pixel bytes taken as x / 255 in fp32, the
 * value the reference's loaders compute, data.py:49-57) with T thresholds:
 * learned = 0 is binarize / binarize_spatial
 * (silogic/data.py:23-40, 75-89): feature t*D + d = (x[b][d] >= thr[t]);
 * learned = 1 is LearnedThermometerEncoder.forward_hard (encoders.py:46-49):
 * feature f*T + i = (x[b][f] - thr[f*T + i] > 0). layout 2: uint8 [B, D*T]
 * (the reference's output); 0: packed [D*T, nw] (for images also the conv
 * layout [C*T, H*W, nw]); 1: packed word-major [nw, D*T]. */
int slg_encode_thermometer(const void* x, int32_t dtype, int64_t B, int64_t D, const float* thr,
                           int32_t T, int32_t learned, int32_t layout, void* out,
                           slg_stream_t stream);
/* edge_bits (data.py:102-131): x [N,C,H,W] -> uint8 [N, C*3*2*T, H, W], per
 * colour the 3x3 Sobel-x, Sobel-y and Laplacian responses (zero padding),
 * each thresholded at > t and < -t; channel (ti*2 + s)*3C + c*3 + det. */
int slg_edge_bits(const float* x, int64_t N, int64_t C, int64_t H, int64_t W, const float* thr,
                  int32_t T, uint8_t* out, slg_stream_t stream);
/* Gradient of the learnable thermometer's soft pass (encoders.py:40-44: the
 * hard bits carry the gradient of sigmoid((x - t) * scale)): g [B, F*T] ->
 * gx [B,F], gt [F,T] (either may be NULL; gt summed over samples in a fixed
 * order, workspace slg_learned_thermo_bwd_workspace(B, F, T) floats). */
int64_t slg_learned_thermo_bwd_workspace(int64_t B, int64_t F, int32_t T);
int slg_learned_thermo_bwd(const float* x, int64_t B, int64_t F, int32_t T, const float* thr,
                           float scale, const float* g, float* gx, float* gt, float* workspace,
                           int64_t workspace_floats, slg_stream_t stream);

/* GroupSum.forward (silogic/heads.py:34-39): x [B,W] -> logits [B,C] =
 * sum over class block of (ste ? (x > 0.5) : x), divided by tau. */
int slg_groupsum_soft(const float* x, int64_t B, int64_t W, int32_t C, float tau,
                      int32_t ste, float* logits, slg_stream_t stream);

/* GroupSum.forward_hard (silogic/heads.py:41-45) on unpacked features:
 * x [B,W] (dtype 0 = fp32, 1 = uint8) -> logits [B,C] fp32 block sums. */
int slg_groupsum_hard(const void* x, int32_t dtype, int64_t B, int64_t W, int32_t C,
                      float* logits, slg_stream_t stream);

/* OrPool.forward / forward_hard (silogic/layers.py:548-563): size x size
 * max pool with stride size and floor on x [B,C,H,W] (dtype 0 = fp32,
 * 1 = uint8) -> out [B,C,H/size,W/size]. */
int slg_orpool(const void* x, int32_t dtype, int64_t B, int64_t C, int64_t H, int64_t W,
               int32_t size, void* out, slg_stream_t stream);

/* ---------------------------------------------------------------------- */
/* Hard (bit-packed) path                                                   */
/* ---------------------------------------------------------------------- */

/* LogicLayer.forward_hard input cast (layers.py:133) fused with packing:
 * x [B,D] (dtype 0 = fp32, 1 = uint8) -> packed words, bit set iff
 * uint8(x) != 0 (fp32: x >= 1); padding bits are zero. layout 0 writes the
 * reference layout [D, ceil(B/64)] (replaces silogic/bitpacking/ops.py:32-49
 * pack_bits); layout 1 writes word-major [ceil(B/64), D]. */
int slg_pack_bits(const void* x, int32_t dtype, int64_t B, int64_t D, int32_t layout,
                  uint64_t* xp, slg_stream_t stream);

/* Inverse of slg_pack_bits to uint8 [B,D] (ops.py:52-63 unpack_bits). */
int slg_unpack_bits(const uint64_t* xp, int64_t B, int64_t D, uint8_t* out,
                    slg_stream_t stream);

/* Image packing is slg_pack_bits with D = C*H*W: [B,C,H,W] -> [C,H,W,nw],
 * the reference's B-packed conv layout (packed_layer.py:184-214). */

/* Hard FC codes for one arity-2 layer (convert.py:61-97,126-136 semantics):
 * wiring from cand [OUT,2,K] int32 + conn [OUT,2,K] (argmax, first index on
 * ties), or from idx [OUT,2] int32 when conn == NULL (fixed); truth table
 * from raw: gate16 logits [OUT,16] (argmax), walsh theta [OUT,4] (corner
 * sign of ((t0 +- t1) +- t2) +- t3), multilinear2 logits [OUT,4] (> 0).
 * Indices are clamped into [0, IN). */
int slg_fc_hard_prep(const int32_t* cand, const float* conn, int64_t OUT, int32_t K,
                     int64_t IN, int32_t node_kind, const float* raw, uint32_t* codes,
                     slg_stream_t stream);

/* slg_fc_hard_prep for n_layers (<= 16) layers in one launch: host arrays
 * of length n_layers with the arguments of each layer (conn[l] NULL = fixed
 * wiring, K[l] = 1). compact = 0 writes slg_code2 codes [out_dim, 2];
 * compact = 1 writes the depth-fused network's 4-byte codes [out_dim]
 * (b | a << 14 | tt << 28, inputs at most 16384 wide) for slg_fc_hard_net. */
int slg_fc_hard_prep_net(int32_t n_layers, const int32_t* const* cand, const float* const* conn,
                         const float* const* raw, const int64_t* in_dim, const int64_t* out_dim,
                         const int32_t* K, const int32_t* node_kind, int32_t compact,
                         uint32_t* const* codes, slg_stream_t stream);

/* One packed FC layer (replaces BitpackedFCLayer.forward,
 * packed_layer.py:85-116, and LogicLayer.forward_hard, layers.py:131-135):
 * xin [IN,nw] -> xout [OUT,nw] with xout[o] = tt_o(xin[a_o], xin[b_o]). */
int slg_fc_hard_layer(const uint64_t* xin, int64_t IN, int64_t nw,
                      const uint32_t* codes, int64_t OUT, uint64_t* xout,
                      slg_stream_t stream);

/* Depth-fused packed FC network + GroupSum (replaces LogicNet.forward_hard,
 * models.py:99-101, with GroupSum.forward_hard, heads.py:41-45). codes[l]
 * are compact 4-byte codes [width_l] from slg_fc_hard_prep_net(compact = 1);
 * operand indices are clamped to the layer's input width. Input x:
 * in_kind 0 = fp32 rows [B,IN0] (bit = x >= 1), 1 = uint8 rows [B,IN0]
 * (bit = x != 0), both packed inside the launch (streamed per persistent
 * workgroup for IN0 <= 1024 with 64-sample tiles, else packed per tile in
 * LDS), 2 = packed [IN0, ceil(B/64)] uint64, 3 = packed word-major
 * [ceil(B/64), IN0]. It runs
 * n_layers arity-2 layers whose widths and device code arrays are given
 * by the host arrays widths[n_layers] and codes[n_layers], then writes logits [B,C] fp32 = per-class popcounts of
 * the last layer (no tau). One workgroup keeps a 64-sample (or, for wide
 * layers, 32-sample) column of every activation in LDS across all layers;
 * a one-layer network on packed input with fewer 64-sample words than half
 * the CUs instead takes one workgroup per (word, class), which reads its
 * gates' operand words from memory (same logits).
 * wire_r > 0 replaces the first wire_r outputs of a same-width layer by its
 * inputs (models.py:88-94). Returns SLG_E_UNSUPPORTED when the widths do not
 * fit LDS (see slg_fc_hard_net_supported). */
int slg_fc_hard_net(const void* x, int32_t in_kind, int64_t B, int64_t IN0, int32_t n_layers,
                    const int64_t* widths, const uint32_t* const* codes, int32_t C,
                    int64_t wire_r, float* logits, slg_stream_t stream);
/* Bank-aware placement of a fused network's outputs (no counterpart in the
 * reference: a relabelling of LogicNet.forward_hard's circuit, models.py:
 * 99-101, that leaves the logits unchanged). codes[l] are compact codes
 * [widths[l]] from slg_fc_hard_prep_net (compact = 1); writes placed[l]
 * (distinct buffers): for l < n_layers - 1, round_up(widths[l], 32) slots
 * holding the layer's outputs so that each 32 consecutive slots read
 * operands of distinct LDS bank classes where the counts allow (unused
 * slots hold code 0), with the next layer's operands renamed to the slots;
 * the last layer keeps its order. Pass placed[] with those slot counts as
 * widths to slg_fc_hard_net (wire_r must be 0). perm_ws: int32 workspace of
 * widths[0] + .. + widths[n_layers-2] entries (output -> slot). Widths at
 * most 16384. One workgroup; parameter-sized. */
int slg_fc_hard_place_net(int32_t n_layers, const int64_t* widths, const uint32_t* const* codes,
                          uint32_t* const* placed, int32_t* perm_ws, int64_t perm_ws_len,
                          slg_stream_t stream);
/* 64 or 32 = samples per workgroup slg_fc_hard_net would use, 0 = unsupported. */
int slg_fc_hard_net_supported(int64_t IN0, int32_t n_layers, const int64_t* widths, int32_t C);
/* Slots per layer (MAXO * 1024) of the type-uniform layout below for a
 * network of inputs IN0 and these widths (each at most 16384), or 0 when it
 * does not apply (a 32-sample column must fit LDS). */
int64_t slg_fc_hard_type_slots(int64_t IN0, int32_t n_layers, const int64_t* widths);
/* Type-uniform placement of a fused network's outputs (no counterpart in the
 * reference: a relabelling of LogicNet.forward_hard's circuit, models.py:
 * 99-101, that leaves the logits unchanged). codes[l] are compact codes
 * [widths[l]] from slg_fc_hard_prep_net (compact = 1). Writes, per layer,
 * placed[l] of S = slg_fc_hard_type_slots() slots (slot j*1024 + t stored at
 * t*(S/1024) + j) and a plan row (plan[l*20 ..]: U, rows, a truth table
 * per wave, then S/1024 and IN0): for every layer but the last, rows 0..U-1 hold in each
 * 64-slot wave row outputs of one gate type (codes (a << 16) | b with word
 * indices of the two activation buffers) and the remaining rows compact
 * codes; within that, each 32 consecutive slots read operands of distinct
 * LDS bank classes where the counts allow. The last layer keeps its order
 * (compact codes, operands renamed; plan row U = 0). perm_ws: int32
 * workspace of slg_fc_hard_type_place_workspace() entries (the renaming
 * tables, then the placement's scratch). Per layer three launches: the
 * plan (one workgroup), the greedy bins (one workgroup per bin) and the
 * codes; parameter-sized. */
/* int32 entries of slg_fc_hard_type_place_net's workspace for these widths
 * (widths[0] + .. + widths[n_layers-2] for the renaming tables plus a fixed
 * scratch), or -1. No counterpart in the reference. */
int64_t slg_fc_hard_type_place_workspace(int32_t n_layers, const int64_t* widths);
int slg_fc_hard_type_place_net(int32_t n_layers, int64_t IN0, const int64_t* widths,
                               const uint32_t* const* codes, uint32_t* const* placed,
                               int32_t* plan, int32_t* perm_ws, int64_t perm_ws_len,
                               slg_stream_t stream);
/* slg_fc_hard_net (no wire residual) on the placed codes and plan of
 * slg_fc_hard_type_place_net; widths are the layers' widths, as given to the
 * placement; every input kind of slg_fc_hard_net. Same logits, bit for
 * bit. A plan placed for another IN0 (hence
 * another slot count) is detected on the device from its own record: the
 * logits are then NaN. No counterpart in the reference beyond
 * slg_fc_hard_net's. */
int slg_fc_hard_net_typed(const void* x, int32_t in_kind, int64_t B, int64_t IN0, int32_t n_layers,
                          const int64_t* widths, const uint32_t* const* codes, const int32_t* plan,
                          int32_t C, float* logits, slg_stream_t stream);

/* Packed GroupSum.forward_hard on xp [W,nw] (W % C == 0): logits [B,C] fp32
 * raw counts (ops.py:66-104 without the /tau, as heads.py:41-45). */
int slg_groupsum_packed(const uint64_t* xp, int64_t W, int64_t B, int32_t C,
                        float* logits, slg_stream_t stream);

/* ---------------------------------------------------------------------- */
/* Conv (ConvLogicTree + OrPool)                                            */
/* ---------------------------------------------------------------------- */

/* Replaces silogic/kernels/conv_topk.py:175-189 `tree_conv_topk(x, coef, w,
 * cm, ch, cw, depth, K, stride, pad, Ho, Wo)` (layers.py:458-463) and, with
 * K = 1 and w = NULL, kernels/conv.py:399-400 `tree_conv` (layers.py:453-
 * 457): x [B,C,H,W] fp32; coef [N, 2^depth-1, 4]; w [N, 2^depth, K];
 * cm/ch/cw [N, 2^depth, K] int32; out [B,N,Ho,Wo]. depth in 1..5. */
int slg_tree_conv_fwd(const float* x, int64_t B, int64_t C, int64_t H, int64_t W,
                      int64_t N, int32_t depth, int32_t K, const float* coef,
                      const float* w, const int32_t* cm, const int32_t* ch,
                      const int32_t* cw, int32_t stride, int32_t pad, int64_t Ho,
                      int64_t Wo, float* out, slg_stream_t stream);

/* ConvLogicTree.forward + OrPool.forward fused (layers.py:448-485 and
 * 558-559): as above for stride 1, for every node tree the reference builds
 * (layers.py:388-401, 432-446; node parameters level-major, level 0 being
 * the nodes above the leaves, node m of a level combining values
 * arity*m .. arity*m+arity-1 of the level below):
 *   gate16 (node_kind 0): binary tree of depth 1-5, node_param = BasisProj
 *     coef [N, 2^depth-1, 4];
 *   walsh (node_kind 1): binary tree of depth 1-5 of nodes sigmoid(z / tau)
 *     (nodes.py:145-150), node_param = z's (a, b)-space coefficients times
 *     1/tau [N, 2^depth-1, 4];
 *   multilinear (2) / hybrid (3) LUT trees of `arity` (2-6) and depth with
 *     arity^depth <= 36 leaves, node_param = sigmoid(logits) [N, nodes,
 *     2^arity] (multilinear interpolation, or the LUT at the leaves
 *     thresholded at 0.5).
 * Writes only the 2x2-max-pooled map out [B,N,Ho/2,Wo/2] (floor); pool = 0
 * writes the unpooled [B,N,Ho,Wo] instead. Images whose padded planes do not
 * fit LDS run on kernels that read the image through the caches. */
int slg_conv_soft_fwd(const float* x, int64_t B, int64_t C, int64_t H, int64_t W,
                      int64_t N, int32_t node_kind, int32_t depth, int32_t arity,
                      int32_t K, const float* node_param, const float* w,
                      const int32_t* cm, const int32_t* ch, const int32_t* cw,
                      int32_t pad, int32_t pool, float* out, slg_stream_t stream);

/* Soft conv parameters (replaces ConvLogicTree._topk_w, layers.py:487-497,
 * _basis_coef, 408-417, and sigmoid(logits) of the LUT node, nodes.py:178):
 * conn [N,leaves,K] -> w = softmax over K (conn == NULL: w = 1);
 * gate16: raw [N, 2^depth-1, 16] -> param = softmax(raw) @ BASIS [N,nodes,4];
 * multilinear: raw [N, 2^arity] -> param = sigmoid(raw). */
int slg_conv_soft_prep(const float* conn, int64_t N, int32_t leaves, int32_t K,
                       int32_t node_kind, int32_t depth, int32_t arity, const float* raw,
                       float* w, float* node_param, slg_stream_t stream);

/* Per-channel records for slg_conv_soft_fwd_records: the soft conv
 * parameters of slg_conv_soft_prep together with the tap positions,
 * resolved for one input geometry (C, H, W, pad) and pooling flag (the LDS
 * layout of the pooled kernel differs). conn [N,leaves,K] (NULL: w = 1),
 * taps cm/ch/cw [N,leaves,K] as for slg_conv_soft_fwd, raw as for
 * slg_conv_soft_prep. rec holds N * slg_conv_soft_record_floats(...)
 * floats; the layout is internal to the library. The reference computes
 * these parameters inside every forward (layers.py:487-497, 408-417,
 * nodes.py:178); a caller keeps the records while the parameters and the
 * geometry stay the same. */
/* 1 if the LDS-staged conv kernels (and so the records forward) take images
 * (C, H, W) with this tree, K, pad and pooling flag, else 0; the others run
 * slg_conv_soft_fwd on the kernels that read the image through the caches. */
int slg_conv_soft_lds_fit(int64_t C, int64_t H, int64_t W, int32_t node_kind, int32_t depth,
                          int32_t arity, int32_t K, int32_t pad, int32_t pool);
int64_t slg_conv_soft_record_floats(int32_t node_kind, int32_t depth, int32_t arity,
                                    int32_t K, int32_t pool);
int slg_conv_soft_records(const float* conn, const int32_t* cm, const int32_t* ch,
                          const int32_t* cw, int64_t N, int32_t K, int32_t node_kind,
                          int32_t depth, int32_t arity, const float* raw, int64_t C,
                          int64_t H, int64_t W, int32_t pad, int32_t pool, float* rec,
                          slg_stream_t stream);
/* The same records from slg_conv_soft_fwd's separate arrays (node_param and
 * w as that entry point takes them; gate16, multilinear or hybrid trees):
 * slg_conv_soft_fwd_records on them gives slg_conv_soft_fwd's output bit for
 * bit. For a forward whose parameters change every call (training), where
 * building the records once per call and running the records kernels is
 * faster than the separate-array kernels (no counterpart in the reference:
 * the same computation as layers.py:487-497, 408-417, nodes.py:178). */
int slg_conv_soft_records_arrays(const float* node_param, const float* w, const int32_t* cm,
                                 const int32_t* ch, const int32_t* cw, int64_t N, int32_t K,
                                 int32_t node_kind, int32_t depth, int32_t arity, int64_t C,
                                 int64_t H, int64_t W, int32_t pad, int32_t pool, float* rec,
                                 slg_stream_t stream);

/* slg_conv_soft_fwd with the channel parameters taken from records built for
 * the same (C, H, W, pad, pool, K, node_kind, depth, arity); same output. */
int slg_conv_soft_fwd_records(const float* x, int64_t B, int64_t C, int64_t H, int64_t W,
                              int64_t N, int32_t node_kind, int32_t depth, int32_t arity,
                              int32_t K, const float* rec, int32_t pad, int32_t pool,
                              float* out, slg_stream_t stream);

/* Soft conv backward (replaces the backward of the reference's tree-conv
 * ops, kernels/conv.py:94-145 and kernels/conv_topk.py:84-121, with the
 * following OrPool's F.max_pool2d routing, layers.py:558-559, when pool): for
 * the op of slg_conv_soft_fwd (same arguments; node_param as there: gate16
 * coefficients [N, 2^depth-1, 4] or LUT values [N, 2^arity]) and dL/dout =
 * gy [B,N,Ho,Wo], writes dL/dx into gx [B,C,H,W], dL/dw into gw [N,leaves,K]
 * and dL/dnode_param into gnp; any of the three may be NULL (not computed).
 * A pooled output's gradient goes to the first window position (row-major)
 * that holds the window's maximum. No atomics on values: every sum runs in
 * a fixed order. Supports every tree slg_conv_soft_fwd takes with K <= 8
 * (gate16 trees of depth 1-3 and depth-1 LUTs on an LDS-staged kernel where
 * the image fits, the others on kernels that read it through the caches);
 * slg_conv_soft_bwd_workspace returns the workspace floats, or -1 for
 * shapes the kernels do not take. */
int64_t slg_conv_soft_bwd_workspace(int64_t B, int64_t C, int64_t H, int64_t W, int64_t N,
                                    int32_t node_kind, int32_t depth, int32_t arity, int32_t K,
                                    int32_t pad, int32_t pool);
int slg_conv_soft_bwd(const float* x, int64_t B, int64_t C, int64_t H, int64_t W, int64_t N,
                      int32_t node_kind, int32_t depth, int32_t arity, int32_t K,
                      const float* node_param, const float* w, const int32_t* cm,
                      const int32_t* ch, const int32_t* cw, int32_t pad, int32_t pool,
                      const float* gy, float* gx, float* gw, float* gnp, float* workspace,
                      int64_t workspace_floats, slg_stream_t stream);

/* Hard conv parameters (layers.py:505-527 + nodes.py:183-189 semantics):
 * leaf (cm,ch,cw) by argmax over conn [N,leaves,K] (conn == NULL: K = 1,
 * fixed) -> leaf [N, leaves] int32 packed as cm<<8 | ch<<4 | cw;
 * tt is one uint64 per channel, [N]:
 * gate16: raw = concatenated per-level gate logits [N, 2^depth-1, 16] ->
 * node j's 4-bit truth table (argmax gate) in bits 4j..4j+3 (depth <= 4);
 * multilinear (depth 1): raw [N, 2^arity] logits -> bit p = logits[p] > 0. */
int slg_conv_hard_prep(const int32_t* cm, const int32_t* ch, const int32_t* cw,
                       const float* conn, int64_t N, int32_t leaves, int32_t K,
                       int32_t node_kind, int32_t depth, int32_t arity, const float* raw,
                       int32_t* leaf, uint64_t* tt, slg_stream_t stream);

/* slg_conv_hard_prep for n_blocks (<= 8) conv blocks in one launch (the
 * hard parameters of every ConvLogicTree of LogicConvNet.forward_hard,
 * models.py:273-275). Host arrays of length n_blocks hold each block's
 * arguments (conn[b] NULL = fixed wiring, K[b] = 1); raw holds 4 pointers
 * per block, raw[4b + l]: for gate16, level l's gate logits
 * [N, 2^(depth-1-l), 16] read in place (the per-level gate_logits
 * parameters, layers.py:350-358, walked as layers.py:519-526), slots past
 * depth unused; for multilinear, raw[4b] = logits [N, 2^arity]. */
int slg_conv_hard_prep_net(int32_t n_blocks, const int32_t* const* cm,
                           const int32_t* const* ch, const int32_t* const* cw,
                           const float* const* conn, const float* const* raw, const int64_t* N,
                           const int32_t* K, const int32_t* node_kind, const int32_t* depth,
                           const int32_t* arity, int32_t* const* leaf, uint64_t* const* tt,
                           slg_stream_t stream);

/* Hard parameters of any node tree of slg_conv_soft_fwd (ConvLogicTree.
 * forward_hard, layers.py:505-541 with nodes.py:100-106, 152-156, 183-189):
 * leaf [N, leaves] int32 (argmax tap cm<<8 | ch<<4 | cw over conn
 * [N,leaves,K], conn NULL = fixed) and tables [N, nodes] uint64, one truth
 * table per node, level-major, bit e = the node's output at address
 * e = sum_j child_j << j. raw[i] is tree level i's parameters read in place:
 * gate16 logits [N, m_i, 16], walsh theta [N*m_i, 4], LUT logits
 * [N*m_i, 2^arity] (m_i nodes per channel at level i). */
int slg_conv_tree_hard_prep(const int32_t* cm, const int32_t* ch, const int32_t* cw,
                            const float* conn, int64_t N, int32_t K, int32_t node_kind,
                            int32_t depth, int32_t arity, const float* const* raw, int32_t* leaf,
                            uint64_t* tables, slg_stream_t stream);

/* The packed node tree of slg_conv_tree_hard_prep with the 2x2 OR pool
 * fused (pool = 1): xp [C,H,W,nw] -> out [N,Ho/2,Wo/2,nw] or [N,H,W,nw];
 * stride 1, zero padding pad = (kernel-1)/2. arity is 2 for gate16 / walsh
 * trees. Replaces the reference's packed_unfold + BitpackedConvTreeLayer /
 * BitpackedConvLUTLayer + packed_or_pool (packed_layer.py:224-540) for trees
 * of any depth. */
int slg_conv_tree_hard_fwd(const uint64_t* xp, int64_t C, int64_t H, int64_t W, int64_t nw,
                           int64_t N, int32_t arity, int32_t depth, const int32_t* leaf,
                           const uint64_t* tables, int32_t kernel, int32_t pad, int32_t pool,
                           uint64_t* out, slg_stream_t stream);

/* ConvLogicTree.forward_hard + OrPool.forward_hard fused on packed
 * activations (replaces layers.py:529-541,561-563 and the reference's
 * packed_unfold / BitpackedConvTreeLayer / packed_or_pool,
 * packed_layer.py:224-432): xp [C,H,W,nw] -> out [N,Ho/2,Wo/2,nw]
 * (pool = 1) or [N,H,W,nw] (pool = 0); stride 1, zero padding `pad`. */
int slg_conv_hard_fwd(const uint64_t* xp, int64_t C, int64_t H, int64_t W, int64_t nw,
                      int64_t N, int32_t node_kind, int32_t depth, int32_t arity,
                      const int32_t* leaf, const uint64_t* tt, int32_t kernel, int32_t pad,
                      int32_t pool, uint64_t* out, slg_stream_t stream);
/* slg_conv_hard_fwd (pooled) on word-major, zero-bordered images, the
 * layout of LogicConvNet.forward_hard's launch sequence: xp [nw][C][H+2pad]
 * [W+2pad] uint64 (nw = ceil(B/64); the border, `pad` words wide, must be
 * zero) -> the interior of out [nw][N][Ho/2+2out_pad][Wo/2+2out_pad] (its
 * border is not written: a buffer cleared once keeps it, ready as the next
 * block's input with pad = out_pad; out_pad = 0 gives the head's
 * PACKED_WORD_MAJOR input). The same bits as slg_conv_hard_fwd on the
 * transposed layout. No counterpart in the reference beyond
 * slg_conv_hard_fwd's (a layout of the same computation, layers.py:
 * 529-541,561-563): with the padding stored, every leaf read is
 * unconditional, and LUTs of arity 3-6 are evaluated as 3-input functions. */
int slg_conv_hard_fwd_wm(const uint64_t* xp, int64_t B, int64_t C, int64_t H, int64_t W,
                         int64_t N, int32_t node_kind, int32_t depth, int32_t arity,
                         const int32_t* leaf, const uint64_t* tt, int32_t kernel, int32_t pad,
                         uint64_t* out, int32_t out_pad, slg_stream_t stream);
/* pack_bits for images x [B,C,H,W] (dtype 0 fp32: x >= 1, 1 uint8: x != 0)
 * into the interior of the zero-bordered word-major layout [nw][C][H+2pad]
 * [W+2pad] (the border is not written). No counterpart in the reference
 * (the input of slg_conv_hard_fwd_wm; bitpacking/ops.py:27-49 packs the
 * same bits). */
int slg_pack_image_wm(const void* x, int32_t dtype, int64_t B, int64_t C, int64_t H, int64_t W,
                      int32_t pad, uint64_t* xp, slg_stream_t stream);

/* A network's forward_hard as one call (no counterpart in the reference,
 * whose LogicNet / LogicConvNet.forward_hard run their layers from Python,
 * models.py:99-101 and 283-293): the launches of its packing
 * (slg_pack_image_wm or slg_pack_bits, word-major), of slg_conv_hard_fwd_wm
 * for each conv block and of slg_fc_hard_net_typed (plan set) or
 * slg_fc_hard_net for the head, in that order on one stream, from a
 * descriptor built once per input shape; where slg_hard_step_fuses_head()
 * is 1 or 2, the last conv block and the head run as one launch of
 * slg_conv_hard_head_wm or slg_conv_hard_net_wm (the same logits). Every pointer in it must stay
 * valid while it is used; the intermediate buffers are the descriptor's,
 * so calls that overlap on one descriptor race (serialise them). For
 * callers that run one network many times and would otherwise pay each
 * launch's C-ABI argument conversion per call. Returns the first error of
 * the calls it makes (their checks and codes); B = 0 launches nothing. */
#define SLG_STEP_MAX_CONV 8
typedef struct {
  const uint64_t* in;  /* word-major zero-bordered input images (pad words) */
  uint64_t* out;       /* its pooled output, out_pad words of zero border */
  int64_t C, H, W, N;
  int32_t node_kind, depth, arity, kernel, pad, out_pad;
  const int32_t* leaf;
  const uint64_t* tt;
} slg_step_conv_t;
typedef struct {
  int32_t pack;        /* 0: the head reads x; 1: slg_pack_image_wm; 2: slg_pack_bits */
  int32_t dtype;       /* x: 0 fp32, 1 uint8 */
  int64_t B;
  int64_t C, H, W;     /* pack 1: the image; pack 2: C*H*W features per sample */
  int32_t pack_pad;    /* pack 1: the packed image's zero border */
  uint64_t* packed;    /* the packing's output */
  int32_t n_conv;      /* 0..SLG_STEP_MAX_CONV */
  slg_step_conv_t conv[SLG_STEP_MAX_CONV];
  const void* head_in; /* null: x (pack 0) */
  int32_t head_in_kind;
  int64_t head_in_dim;
  int32_t n_layers;
  const int64_t* widths;
  const uint32_t* const* codes;
  const int32_t* plan; /* type-placed codes' plan, or null */
  int32_t n_classes;
  int64_t wire_r;
} slg_hard_step_t;
int slg_hard_step(const slg_hard_step_t* step, const void* x, float* logits,
                  slg_stream_t stream);
/* Whether slg_hard_step evaluates the descriptor's last conv block inside
 * its head: 1 (slg_conv_hard_head_wm) for a one-layer head at a batch where
 * the head takes a workgroup per (word, class); 2 (slg_conv_hard_net_wm)
 * for other heads at batches of at most one 64-sample word per CU whose
 * fused network has 64-sample words and activation buffers of 2048 or 4096
 * words that fit LDS beside one word's block input; both need a head
 * without wire residual on the block's own output (no border) and a node
 * the fused kernel evaluates (gate16 trees of depth 1-3; LUTs of arity 2-6
 * for 1, 2-4 for 2); else 0. No counterpart in the reference. */
int slg_hard_step_fuses_head(const slg_hard_step_t* step);

/* The last pooled conv block of a conv network and its one-layer head +
 * GroupSum in one launch (replaces the last ConvLogicTree + OrPool of
 * LogicConvNet.forward_hard with its head layer and GroupSum.forward_hard,
 * models.py:283-293, heads.py:41-45; no single counterpart in the
 * reference). xp, B, C, H, W, N, node_kind, depth, arity, leaf, tt, kernel
 * and pad are slg_conv_hard_fwd_wm's (the block's word-major,
 * zero-bordered input); the head is one layer of `width` gates on the
 * block's N*Ho*Wo outputs (feature n*Ho*Wo + oy*Wo + ox, <= 16384) with
 * compact codes, type-placed with `plan` (codes stored thread-major, as
 * slg_fc_hard_type_place_net writes them) or in index order (plan null),
 * and n_classes classes of width/n_classes <= 8192 gates. A workgroup per
 * (64-sample word, class) evaluates only the conv outputs its gates read.
 * logits [B, n_classes] fp32: the class counts of slg_conv_hard_fwd_wm
 * followed by slg_fc_hard_net(_typed) on its output, bit for bit. Gate16
 * trees of depth 1-3 and LUTs of arity 2-6; other nodes return
 * SLG_E_UNSUPPORTED. */
int slg_conv_hard_head_wm(const uint64_t* xp, int64_t B, int64_t C, int64_t H, int64_t W,
                          int64_t N, int32_t node_kind, int32_t depth, int32_t arity,
                          const int32_t* leaf, const uint64_t* tt, int32_t kernel, int32_t pad,
                          int64_t width, const uint32_t* codes, const int32_t* plan,
                          int32_t n_classes, float* logits, slg_stream_t stream);
/* The last pooled conv block of a conv network and its whole head (the
 * depth-fused network of slg_fc_hard_net / slg_fc_hard_net_typed, no wire
 * residual) in one launch (replaces the last ConvLogicTree + OrPool of
 * LogicConvNet.forward_hard with the head layers and GroupSum.forward_hard,
 * models.py:283-293, heads.py:41-45; no single counterpart in the
 * reference): the workgroup of each 64-sample word evaluates every conv
 * output of the word into LDS, then runs the layers and the GroupSum. Conv
 * arguments as slg_conv_hard_head_wm; n_layers, widths, codes, plan and
 * n_classes as slg_fc_hard_net_typed (plan set) or slg_fc_hard_net (plan
 * null) on the block's N*Ho*Wo outputs (<= 16384). logits [B, n_classes]:
 * the class counts of slg_conv_hard_fwd_wm followed by that call, bit for
 * bit. SLG_E_UNSUPPORTED unless the network takes 64-sample words with
 * activation buffers of 2048 or 4096 words, LDS holds them and one word's
 * block input (C*(H+2pad)*(W+2pad) words, staged there), and the node is a
 * gate16 tree of depth 1-3 or a LUT of arity 2-4. */
int slg_conv_hard_net_wm(const uint64_t* xp, int64_t B, int64_t C, int64_t H, int64_t W,
                         int64_t N, int32_t node_kind, int32_t depth, int32_t arity,
                         const int32_t* leaf, const uint64_t* tt, int32_t kernel, int32_t pad,
                         int32_t n_layers, const int64_t* widths, const uint32_t* const* codes,
                         const int32_t* plan, int32_t n_classes, float* logits,
                         slg_stream_t stream);

/* ---------------------------------------------------------------------- */
/* Packed building blocks of the silogic.bitpacking API                      */
/* ---------------------------------------------------------------------- */

/* BitpackedLUTLayer.forward (bitpacking/packed_layer.py:121-178): x [IN,nw]
 * packed -> out [OUT,nw]; output o reads inputs idx[o][0..arity) (clamped)
 * and its truth table tt[o], entry e = sum_j x_j << j at bit e
 * (arity <= 6). */
int slg_fc_lut_hard(const uint64_t* x, int64_t IN, int64_t nw, const int32_t* idx,
                    int32_t arity, const uint64_t* tt, int64_t OUT, uint64_t* out,
                    slg_stream_t stream);

/* packed_unfold (bitpacking/packed_layer.py:224-283): x [C,H*W,nw] ->
 * out [C*kh*kw, Ho*Wo, nw], row c*kh*kw + dy*kw + dx, zero padding. */
int slg_packed_unfold(const uint64_t* x, int64_t C, int64_t H, int64_t W, int64_t nw,
                      int32_t kh, int32_t kw, int32_t stride, int32_t pad, uint64_t* out,
                      slg_stream_t stream);

/* packed_or_pool (bitpacking/packed_layer.py:286-319): x [C,H*W,nw] ->
 * out [C,(H/ps)*(W/ps),nw], OR over ps x ps windows (floor sizes). */
int slg_packed_or_pool(const uint64_t* x, int64_t C, int64_t H, int64_t W, int64_t nw,
                       int32_t ps, uint64_t* out, slg_stream_t stream);

/* BitpackedConvTreeLayer / BitpackedConvLUTLayer.forward_packed
 * (bitpacking/packed_layer.py:324-540) on unfolded input xu [P,L,nw]:
 * output n gathers leaves leaf[n][0..arity^depth) (flat P indices), then
 * evaluates a tree of arity-input LUT nodes; tables [N][nodes] hold the
 * nodes level-major (leaves' level first), node m of a level combining
 * values arity*m .. arity*m+arity-1 of the level below; LUT addressing as
 * slg_fc_lut_hard (a gate16 node is an arity-2 LUT with entry
 * (first child) | (second child) << 1). out [N,L,nw]. */
int slg_lut_tree_hard(const uint64_t* xu, int64_t P, int64_t L, int64_t nw, int64_t N,
                      const int32_t* leaf, int32_t arity, int32_t depth,
                      const uint64_t* tables, uint64_t* out, slg_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* SILOGIC_HIP_H */
