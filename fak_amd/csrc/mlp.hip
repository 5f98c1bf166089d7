// mlp.hip — the fused decode MLP: y = down(silu(gate x) * (up x)) for 1..4 tokens in two
// launches on the library stream, with the I-wide intermediate kept on the device.
//
// The replacement for mg_q4k_mlp / mg_q4k_mlp_q6down (internal/metalgemm/q4k.m:458-520,680-740;
// Go side FusedMLP / FusedMLPQ6Down, internal/metalgemm/q4k.go:144-205), which the dense SwiGLU
// FFN calls for a decode token (internal/model/moe.go:111-136, metal_q4k_on.go:189-233):
//   launch 1: gate and up GEMVs over one activation, tiles interleaved so that each workgroup
//             holds both row blocks and writes silu(g) * u directly (stages 1 and 2 of the
//             reference's three encoders);
//   launch 2: the down GEMV over the intermediate (Q4_K on the int8 GEMV, or Q6_K).
// Nothing is synchronized with the host; both launches are graph-capturable.
#include <cstdint>

#include "kernels.hpp"

using namespace fhip;

namespace {

int check_mlp(const char *who, const void *g, const void *u, const void *d, const float *dX,
              float *dY, int hidden, int inter, int P, bool q4_down) {
  if (hidden <= 0 || inter <= 0 || hidden % 256 || inter % 256)
    return fail(FHIP_EINVAL, "%s: hidden=%d and inter=%d must be positive multiples of 256", who,
                hidden, inter);
  if (P < 0 || P > 4) return fail(FHIP_EINVAL, "%s: P=%d outside 0..4", who, P);
  if (!g || !u || !d || !dX || !dY) return fail(FHIP_EINVAL, "%s: null pointer", who);
  if (((uintptr_t)g & 15) || ((uintptr_t)u & 15) || ((uintptr_t)dX & 15) ||
      (q4_down && ((uintptr_t)d & 15)))
    return fail(FHIP_EINVAL, "%s: dX and the Q4_K weights must be 16-byte aligned", who);
  if (P == 0) return FHIP_OK;
  if (int rc = check_weight(who, g, kWeightQ4K, inter, hidden)) return rc;
  if (int rc = check_weight(who, u, kWeightQ4K, inter, hidden)) return rc;
  return check_weight(who, d, q4_down ? kWeightQ4K : kWeightQ6K, hidden, inter);
}

// Workspace: the intermediate [P][inter] (256-byte padded), then the scratch of the two
// launches (stream-ordered, so they may share it). The down GEMV is the plain matmul of the
// intermediate, run inside a ScratchScope over the second region: its own scratch (operands,
// K-range partials) can never land on the intermediate it reads.
int run_mlp(const void *g, const void *u, const void *d, const float *dX, float *dY, int hidden,
            int inter, int P, bool q4_down) {
  const size_t interB = ((size_t)P * inter * 4 + 255) & ~(size_t)255;
  size_t scr = gemv_i8_ws_bytes(2 * q4k_tiles(inter), hidden, P, true);
  const size_t dB =
      q4_down ? q4k_gemv_ws_bytes(hidden, inter, P) : q6k_gemv_ws_bytes(hidden, inter, P);
  if (dB > scr) scr = dB;
  scr = (scr + 255) & ~(size_t)255;
  unsigned char *ws = (unsigned char *)workspace(interB + scr);
  if (!ws) return FHIP_ENOMEM;
  if (int rc = check_disjoint("mlp", dX, (size_t)P * hidden * 4, ws, interB + scr)) return rc;
  float *mid = (float *)ws;
  unsigned char *rest = ws + interB;
  ScratchScope scope(rest, scr);
  if (int rc = q4k_gemv_swiglu(g, u, dX, mid, inter, hidden, P, rest)) return rc;
  if (q4_down) return q4k_gemv(d, mid, dY, hidden, inter, P);
  return q6k_gemv(d, mid, dY, hidden, inter, P);
}

}  // namespace

extern "C" {

int fhip_q4k_mlp_f32(const void *dGate, const void *dUp, const void *dDown, const float *dX,
                     float *dY, int hidden, int inter, int P) {
  clear_error();
  if (int rc = check_mlp("fhip_q4k_mlp_f32", dGate, dUp, dDown, dX, dY, hidden, inter, P, true))
    return rc;
  if (P == 0) return FHIP_OK;
  untag_range(dY, (size_t)P * hidden * 4);
  return run_mlp(dGate, dUp, dDown, dX, dY, hidden, inter, P, true);
}

int fhip_q4k_mlp_q6down_f32(const void *dGate, const void *dUp, const void *dDownQ6,
                            const float *dX, float *dY, int hidden, int inter, int P) {
  clear_error();
  if (int rc = check_mlp("fhip_q4k_mlp_q6down_f32", dGate, dUp, dDownQ6, dX, dY, hidden, inter,
                         P, false))
    return rc;
  if (P == 0) return FHIP_OK;
  untag_range(dY, (size_t)P * hidden * 4);
  return run_mlp(dGate, dUp, dDownQ6, dX, dY, hidden, inter, P, false);
}

}  // extern "C"
