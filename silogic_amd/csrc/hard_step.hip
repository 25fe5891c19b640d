// A network's forward_hard as one C-ABI call: the launch sequence of
// LogicNet / LogicConvNet.forward_hard (silogic/models.py:99-101, 283-293)
// from a descriptor built once per input shape. Host code only: it calls
// the entry points that a launch-per-call caller would.
#include "slg_common.h"

extern "C" {

int slg_hard_step(const slg_hard_step_t* step, const void* x, float* logits,
                  slg_stream_t stream) {
  SLG_REQUIRE(step, SLG_E_ARG, "hard_step: null pointer");
  const slg_hard_step_t& s = *step;
  SLG_REQUIRE(s.n_conv >= 0 && s.n_conv <= SLG_STEP_MAX_CONV && s.pack >= 0 && s.pack <= 2 &&
                  s.B >= 0,
              SLG_E_ARG, "hard_step: pack %d, %d conv blocks, B %lld", s.pack, s.n_conv,
              (long long)s.B);
  if (s.B == 0) return 0;  // an empty batch: no launch (x and logits may be null)
  SLG_REQUIRE(x && logits, SLG_E_ARG, "hard_step: null pointer");
  int rc = 0;
  if (s.pack == 1) {
    rc = slg_pack_image_wm(x, s.dtype, s.B, s.C, s.H, s.W, s.pack_pad, s.packed, stream);
  } else if (s.pack == 2) {
    rc = slg_pack_bits(x, s.dtype, s.B, s.C * s.H * s.W, 1, s.packed, stream);  // word-major
  }
  if (rc) return rc;
  // the head may evaluate the last conv block itself (1: a one-layer head
  // at a small batch, 2: the fused head network)
  const int fused = slg_hard_step_fuses_head(step);
  for (int i = 0; i < s.n_conv - (fused ? 1 : 0); ++i) {
    const slg_step_conv_t& c = s.conv[i];
    rc = slg_conv_hard_fwd_wm(c.in, s.B, c.C, c.H, c.W, c.N, c.node_kind, c.depth, c.arity,
                              c.leaf, c.tt, c.kernel, c.pad, c.out, c.out_pad, stream);
    if (rc) return rc;
  }
  if (fused) {
    const slg_step_conv_t& c = s.conv[s.n_conv - 1];
    if (fused == 1)
      return slg_conv_hard_head_wm(c.in, s.B, c.C, c.H, c.W, c.N, c.node_kind, c.depth, c.arity,
                                   c.leaf, c.tt, c.kernel, c.pad, s.widths[0], s.codes[0], s.plan,
                                   s.n_classes, logits, stream);
    return slg_conv_hard_net_wm(c.in, s.B, c.C, c.H, c.W, c.N, c.node_kind, c.depth, c.arity,
                                c.leaf, c.tt, c.kernel, c.pad, s.n_layers, s.widths, s.codes,
                                s.plan, s.n_classes, logits, stream);
  }
  const void* hin = s.head_in ? s.head_in : x;
  if (s.plan)
    return slg_fc_hard_net_typed(hin, s.head_in_kind, s.B, s.head_in_dim, s.n_layers, s.widths,
                                 s.codes, s.plan, s.n_classes, logits, stream);
  return slg_fc_hard_net(hin, s.head_in_kind, s.B, s.head_in_dim, s.n_layers, s.widths, s.codes,
                         s.n_classes, s.wire_r, logits, stream);
}

}  // extern "C"
