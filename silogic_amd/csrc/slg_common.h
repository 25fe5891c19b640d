// Shared helpers of the gfx950 gate-layer library: error reporting, launch
// checks, device queries and small device utilities.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <string>

#include "../../include/silogic_hip.h"

namespace slg {

void set_error(const char* fmt, ...);

// Argument / shape rejection: records the message and returns the code.
#define SLG_REQUIRE(cond, code, ...)            \
  do {                                          \
    if (!(cond)) {                              \
      ::slg::set_error(__VA_ARGS__);            \
      return (code);                            \
    }                                           \
  } while (0)

// After a launch: report a launch failure as a positive hipError_t.
#define SLG_LAUNCH_CHECK(what)                                              \
  do {                                                                      \
    hipError_t e_ = hipGetLastError();                                      \
    if (e_ != hipSuccess) {                                                 \
      ::slg::set_error("%s: launch failed: %s", what, hipGetErrorString(e_)); \
      return (int)e_;                                                       \
    }                                                                       \
  } while (0)

inline hipStream_t as_stream(slg_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

// Compute units of the current device (cached per device id).
int device_cus();
// Max dynamic LDS bytes per workgroup of the current device.
int device_lds_bytes();

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Workgroup id remapped so that consecutive logical ids share an XCD.
// The hardware dispatches workgroup i to XCD (i % 8); when the grid is a
// multiple of 8, logical = (i % 8) * (grid / 8) + i / 8 is a bijection that
// keeps runs of consecutive logical ids on one XCD (one L2).
__device__ inline uint32_t xcd_logical_id(uint32_t i, uint32_t grid) {
  if ((grid & 7u) != 0u) return i;
  return (i & 7u) * (grid >> 3) + (i >> 3);
}

// Word 3 of a raw buffer resource on gfx9-family GPUs (32-bit data format).
// Loads through such a resource at offsets past its byte size return 0.
constexpr int kBufferWord3 = 0x00020000;

// A raw buffer resource over `bytes` bytes at `p`, for a wave-uniform p and
// size. The words are passed through readfirstlane so the compiler sees them
// as uniform (a resource it cannot prove uniform costs a waterfall loop
// around every access). readfirstlane returns a signed int: each half is
// taken back as uint32_t before it is widened, or the sign of the low word
// would spill into the high one.
__device__ inline __amdgpu_buffer_rsrc_t uniform_rsrc(const void* p, int bytes) {
  const uint64_t a = (uint64_t)p;
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)a);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
  const int n = __builtin_amdgcn_readfirstlane(bytes);
  return __builtin_amdgcn_make_buffer_rsrc((void*)(((uint64_t)hi << 32) | (uint64_t)lo), (short)0,
                                           n, kBufferWord3);
}

// q = e / d for 0 <= e < 2^24 and 0 < d < 2^24, with inv = 1.0f / d: the
// float quotient is within one of the true one, and the remainder test
// corrects it.
__device__ inline int div_small(int e, int d, float inv) {
  int q = (int)((float)e * inv);
  const int r = e - (int)__umul24(q, d);  // full-rate 24-bit multiply
  q += (r >= d) - (r < 0);
  return q;
}

}  // namespace slg
