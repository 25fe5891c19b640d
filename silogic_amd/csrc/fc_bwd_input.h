// The input gradient of an FC soft layer with nsides operand slots per
// output (2 for the gate layers, n for LUT layers), shared by both backward
// paths: given the operand gradients gbr [B][nsides*OUT] (row b, column
// side*OUT + o), the candidates cand [OUT,nsides,K] and weights w,
//   gx[b][i] = sum over references (o, side, k) with cand = i of
//              w[o,side,k] * gbr[b][side*OUT + o],
// summed in ascending reference order (the same bits on every call).
#pragma once

#include "slg_common.h"

namespace slg {

// Workspace floats for fc_input_grad.
int64_t fc_input_grad_floats(int64_t B, int64_t IN, int64_t OUT, int nsides, int K);

// Enqueue on st; ws holds fc_input_grad_floats(...) floats (16-byte aligned).
int fc_input_grad(const float* gbr, int64_t B, int64_t IN, int64_t OUT, int nsides, int K,
                  const int32_t* cand, const float* w, float* ws, float* gx, hipStream_t st);

}  // namespace slg
