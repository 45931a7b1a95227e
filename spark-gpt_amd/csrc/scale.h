// Power-of-two scale rule of the FP8 recipe, exact on the device.
//
// The reference computes  exp2(floor(log2(fmax / max(amax, 1e-30))) - headroom)
// with fp32 torch ops (spark-gpt train.py:942-945 for the delayed activation
// scales, headroom 1; train.py:951 for the just-in-time weight scale,
// headroom 0).  Here the quotient r is formed with the IEEE fp32 divide and
// floor(log2(r)) is taken from r's exponent field, corrected by the band in
// which the correctly rounded fp32 log2 of r rounds up to the next integer:
// if r = 2^K * (1 - n*2^-24) with 1 <= n <= kLog2Band[K], then fl32(log2 r) = K.
#pragma once
#include "common.h"

namespace sfp8 {

// kLog2Band[K + 125], K in [-125, 128]: largest ulp count n below 2^K for which
// the correctly rounded fp32 log2 still equals K.
__device__ __constant__ const uint8_t kLog2Band[254] = {
    44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44,
    44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44,
    44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 22, 22, 22, 22, 22, 22, 22, 22, 22, 22,
    22, 22, 22, 22, 22, 22, 22, 22, 22, 22, 22, 22, 22, 22, 22, 22, 22, 22, 22, 22, 22, 22, 11, 11,
    11, 11, 11, 11, 11, 11, 11, 11, 11, 11, 11, 11, 11, 11, 5, 5, 5, 5, 5, 5, 5, 5, 2, 2,
    2, 2, 1, 1, 0, 0, 0, 0, 1, 1, 2, 2, 2, 2, 5, 5, 5, 5, 5, 5, 5, 5, 11, 11,
    11, 11, 11, 11, 11, 11, 11, 11, 11, 11, 11, 11, 11, 11, 22, 22, 22, 22, 22, 22, 22, 22, 22, 22,
    22, 22, 22, 22, 22, 22, 22, 22, 22, 22, 22, 22, 22, 22, 22, 22, 22, 22, 22, 22, 22, 22, 44, 44,
    44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44,
    44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44,
    44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44, 44,
};

// exp2(floor(log2(r)) - headroom), fp32, for amax >= 0, where
//   r = fmax / max(amax, 1e-30)            (recip_first = false: the scale roll,
//                                           tensor / tensor, train.py:943)
//   r = (1 / max(amax, 1e-30)) * fmax      (recip_first = true: the weight rule
//                                           `448.0 / tensor`, which torch
//                                           evaluates as reciprocal(t) * 448,
//                                           train.py:951)
// each step an IEEE-rounded fp32 operation.
// NaN amax gives NaN; +inf amax gives 0 (log2(0) = -inf, exp2(-inf) = 0).
SFP8_DEV float pow2_scale(float amax, float fmax, int headroom, bool recip_first) {
  if (amax != amax) return amax;
  const float a = fmaxf(amax, 1e-30f);
  const float r = recip_first ? (1.0f / a) * fmax : fmax / a;
  if (r == 0.0f) return 0.0f;
  const uint32_t b = __float_as_uint(r);
  const int e = (int)(b >> 23) - 127;  // r is normal: r >= 448 / 3.4e38
  const uint32_t m = b & 0x7fffffu;
  int k = e;
  const int K = e + 1;
  if (m != 0u && K >= -125 && K <= 128 && (0x800000u - m) <= (uint32_t)kLog2Band[K + 125]) k = K;
  return __builtin_ldexpf(1.0f, k - headroom);
}

}  // namespace sfp8
