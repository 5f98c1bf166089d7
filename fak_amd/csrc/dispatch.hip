// dispatch.hip — the Q4_K matmul entry point: small-M GEMV or MFMA GEMM by batch size.
#include <cstdint>

#include "kernels.hpp"

using namespace fhip;

extern "C" {

int fhip_q4k_matmul_f32(const void *dPacked, const float *dX, float *dY, int out, int in,
                        int P) {
  clear_error();
  if (out <= 0 || in <= 0 || in % 256 != 0)
    return fail(FHIP_EINVAL,
                "fhip_q4k_matmul_f32: need out > 0 and in a positive multiple of 256 (out=%d in=%d)",
                out, in);
  if (P < 0) return fail(FHIP_EINVAL, "fhip_q4k_matmul_f32: P=%d < 0", P);
  if (P == 0) return FHIP_OK;
  if (!dPacked || !dX || !dY) return fail(FHIP_EINVAL, "fhip_q4k_matmul_f32: null pointer");
  if (((uintptr_t)dX & 15) || ((uintptr_t)dPacked & 15))
    return fail(FHIP_EINVAL, "fhip_q4k_matmul_f32: dX and dPacked must be 16-byte aligned");
  int gemv_max = env_int("FAK_HIP_GEMV_MAX_M");
  if (gemv_max <= 0 || gemv_max > 16) gemv_max = 16;
  if (P <= gemv_max) return q4k_gemv(dPacked, dX, dY, out, in, P);
  return q4k_gemm(dPacked, dX, dY, out, in, P);
}

}  // extern "C"
