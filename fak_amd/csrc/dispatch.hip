// dispatch.hip — the Q4_K matmul entry points: small-M GEMV or MFMA GEMM by batch size.
#include <cstdint>

#include "kernels.hpp"

using namespace fhip;

namespace {

// Up to kGemvMaxTokens tokens run the small-M GEMV kernels (decode, speculative verify); up to
// kGemv32MaxTokens the same 32x32 kernel with one f16 operand row per token (small prefill
// chunks, at the GEMM's activation precision); more the prefill GEMM.
constexpr int kGemvMaxTokens = 16;
constexpr int kGemv32MaxTokens = 32;

int check_matmul(const char *who, const void *dPacked, const float *dX, const float *dY, int out,
                 int in, int P) {
  if (out <= 0 || in <= 0 || in % 256 != 0)
    return fail(FHIP_EINVAL, "%s: need out > 0 and in a positive multiple of 256 (out=%d in=%d)",
                who, out, in);
  if (P < 0) return fail(FHIP_EINVAL, "%s: P=%d < 0", who, P);
  if (P == 0) return FHIP_OK;
  if (!dPacked || !dX || !dY) return fail(FHIP_EINVAL, "%s: null pointer", who);
  if (((uintptr_t)dX & 15) || ((uintptr_t)dPacked & 15))
    return fail(FHIP_EINVAL, "%s: dX and dPacked must be 16-byte aligned", who);
  return check_weight(who, dPacked, kWeightQ4K, out, in);
}

}  // namespace

namespace fhip {
int q4k_matmul_run(const void *dPacked, const float *dX, float *dY, int out, int in, int P) {
  if (P <= kGemvMaxTokens) return q4k_gemv(dPacked, dX, dY, out, in, P);
  if (P <= kGemv32MaxTokens) return q4k_gemv32(dPacked, dX, dY, out, in, P);
  return q4k_gemm32(dPacked, dX, dY, out, in, P);
}

size_t q4k_matmul_ws_bytes(int out, int in, int P) {
  if (P <= 0) return 0;
  if (P <= kGemvMaxTokens) return q4k_gemv_ws_bytes(out, in, P);
  if (P <= kGemv32MaxTokens) return gemv16_ws_bytes(0, out, in, P);
  return gemm32_ws_bytes(0, out, in, P);
}
}  // namespace fhip

extern "C" {

int fhip_q4k_matmul_f32(const void *dPacked, const float *dX, float *dY, int out, int in,
                        int P) {
  clear_error();
  if (int rc = check_matmul("fhip_q4k_matmul_f32", dPacked, dX, dY, out, in, P)) return rc;
  if (P == 0) return FHIP_OK;
  untag_range(dY, (size_t)P * out * 4);
  return q4k_matmul_run(dPacked, dX, dY, out, in, P);
}

int fhip_q4k_matmul_group_f32(const void *const *dPacked, float *const *dY, const int *out,
                              int count, const float *dX, int in, int P) {
  clear_error();
  if (count < 1 || count > kMaxGroup)
    return fail(FHIP_EINVAL, "fhip_q4k_matmul_group_f32: count=%d outside 1..%d", count,
                kMaxGroup);
  if (!dPacked || !dY || !out || !dX)
    return fail(FHIP_EINVAL, "fhip_q4k_matmul_group_f32: null pointer");
  if (in <= 0 || in % 256 != 0)
    return fail(FHIP_EINVAL, "fhip_q4k_matmul_group_f32: in=%d not a positive multiple of 256",
                in);
  if (P < 0) return fail(FHIP_EINVAL, "fhip_q4k_matmul_group_f32: P=%d < 0", P);
  if ((uintptr_t)dX & 15)
    return fail(FHIP_EINVAL, "fhip_q4k_matmul_group_f32: dX must be 16-byte aligned");
  GemvGroup g = {};
  g.count = count;
  g.tile0[0] = 0;
  for (int i = 0; i < count; ++i) {
    if (!dPacked[i] || !dY[i] || out[i] <= 0 || ((uintptr_t)dPacked[i] & 15))
      return fail(FHIP_EINVAL, "fhip_q4k_matmul_group_f32: member %d: null or misaligned "
                               "pointer or out=%d", i, out[i]);
    if (int rc = check_weight("fhip_q4k_matmul_group_f32", dPacked[i], kWeightQ4K, out[i], in))
      return rc;
    g.W[i] = (const uint8_t *)dPacked[i];
    g.Y[i] = dY[i];
    g.N[i] = out[i];
    g.tile0[i + 1] = g.tile0[i] + q4k_tiles(out[i]);
  }
  if (P == 0) return FHIP_OK;
  for (int i = 0; i < count; ++i) untag_range(dY[i], (size_t)P * out[i] * 4);
  if (P <= kGemvMaxTokens) return q4k_gemv_group(g, dX, in, P);
  for (int i = 0; i < count; ++i)
    if (int rc = q4k_matmul_run(dPacked[i], dX, dY[i], out[i], in, P)) return rc;
  return FHIP_OK;
}

}  // extern "C"
