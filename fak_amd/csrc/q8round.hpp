// q8round.hpp — the activation/weight int8 rounding rule of fak's Q8 lanes, shared by the
// kernels that must reproduce the CPU reference bit for bit (files built with -ffp-contract=off).
#pragma once

#include <cstdint>

namespace fhip {

// q8round (internal/model/quant.go:89-104, internal/compute/cpuref.go:486-501): truncate toward
// zero, round the fraction half away from zero, clamp to [-127, 127]. On amd64 the Go
// conversion int32(x) of a NaN or of |x| >= 2^31 is the x86 "integer indefinite" 0x80000000, so
// such an input ends at -127 there (or at +127 after the decrement wraps, for x <= -2^31 - 0.5);
// that is reproduced here (the hardware conversion would give 0 or saturate).
__device__ __forceinline__ int q8round(float x) {
  int t = fabsf(x) < 2147483648.f ? (int)x : INT32_MIN;
  const float f = __fsub_rn(x, (float)t);
  if (f >= 0.5f)  // Go's int32 arithmetic wraps: unsigned steps keep that defined here
    t = (int)((unsigned)t + 1u);
  else if (f <= -0.5f)
    t = (int)((unsigned)t - 1u);
  if (t > 127) return 127;
  if (t < -127) return -127;
  return t;
}

// quantizeRowQ8scalar on one 32-value block (internal/model/quant_quantize.go:16-43, the same
// math as quantizeVecQ8 of internal/compute/cpuref.go:505-527): d = amax / 127, codes =
// q8round(x * (1 / d)), an all-zero block when d == 0. Returns d; codes go to q[0..31], and
// *sum receives the int32 sum of the codes.
__device__ __forceinline__ float q8_quant_block32(const float *__restrict__ x, int8_t *__restrict__ q,
                                                  int *sum) {
  float amax = 0.f;
  for (int i = 0; i < 32; ++i) {
    const float a = fabsf(x[i]);
    if (a > amax) amax = a;
  }
  const float d = __fdiv_rn(amax, 127.f);
  int s = 0;
  if (d == 0.f) {
    for (int i = 0; i < 32; ++i) q[i] = 0;
  } else {
    const float inv = __fdiv_rn(1.f, d);
    for (int i = 0; i < 32; ++i) {
      const int c = q8round(__fmul_rn(x[i], inv));
      q[i] = (int8_t)c;
      s += c;
    }
  }
  *sum = s;
  return d;
}

}  // namespace fhip
