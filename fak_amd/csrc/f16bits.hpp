// f16bits.hpp — the exact f16 -> f32 conversion of the reference, shared by the bit-exact
// dequant kernels (files built with -ffp-contract=off).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace fhip {

// F16BitsToF32Bits (internal/model/quantbits.go:15-36) in integer arithmetic, so the result is
// bit-identical for every input (subnormals renormalised, NaN payloads kept unquieted).
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
  const uint32_t sign = (h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t frac = h & 0x3ffu;
  uint32_t bits;
  if (exp == 0) {
    if (frac == 0) {
      bits = sign;
    } else {
      // Shift the leading 1 up to bit 10; each shift lowers the exponent by one from -14.
      const int sh = __clz(frac) - 21;  // frac < 2^10: clz >= 22, sh >= 1
      frac = (frac << sh) & 0x3ffu;
      bits = sign | ((uint32_t)(127 - 14 - sh) << 23) | (frac << 13);
    }
  } else if (exp == 0x1f) {
    bits = sign | 0x7f800000u | (frac << 13);
  } else {
    bits = sign | ((exp - 15 + 127) << 23) | (frac << 13);
  }
  return __uint_as_float(bits);
}

}  // namespace fhip
