// noalloc.hip — the Q4_K matmul for callers that cannot allocate device memory (code under
// HIP graph capture, tight serving loops, harnesses that forbid hipMalloc):
// fhip_q4k_matmul_noalloc_f32 runs exactly the kernels of fhip_q4k_matmul_f32, but their
// scratch (activation operands, token scales, K-range partial sums) lives in a fixed static
// device array instead of the library's grow-on-demand workspace, so the call never reaches
// hipMalloc, hipFree or any allocating routine.
//
// The array is per device and shared by every call on that device: it keeps the last call's
// contents, and two calls that overlap on one device (two streams, two host threads) race on
// it. Nothing in it has to start at zero: every kernel writes the scratch it reads first.
#include <cstdint>

#include "kernels.hpp"

using namespace fhip;

namespace {

constexpr size_t kScratchBytes = 64u << 20;  // 64 MiB per device
constexpr int kMaxDevices = 16;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

// Device address of `scratch` on each device (the host-side name is only a stand-in).
void *g_scratch_ptr[kMaxDevices] = {};

int scratch_for_current_device(void **out) {
  int dev = 0;
  FHIP_CHECK(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices)
    return fail(FHIP_EINVAL, "fhip_q4k_matmul_noalloc_f32: device %d beyond the %d supported",
                dev, kMaxDevices);
  if (!g_scratch_ptr[dev]) {
    void *p = nullptr;
    FHIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return FHIP_OK;
}

}  // namespace

namespace fhip {
// Called by fhip_init with the device current: resolves the device address of the array once.
int noalloc_setup() {
  void *p = nullptr;
  return scratch_for_current_device(&p);
}
}  // namespace fhip

extern "C" {

int fhip_q4k_matmul_noalloc_f32(const void *dPacked, const float *dX, float *dY, int out, int in,
                                int P) {
  clear_error();
  if (out <= 0 || in <= 0 || in % 256 != 0)
    return fail(FHIP_EINVAL,
                "fhip_q4k_matmul_noalloc_f32: need out > 0 and in a positive multiple of 256 "
                "(out=%d in=%d)", out, in);
  if (P < 0) return fail(FHIP_EINVAL, "fhip_q4k_matmul_noalloc_f32: P=%d < 0", P);
  if (P == 0) return FHIP_OK;
  if (!dPacked || !dX || !dY) return fail(FHIP_EINVAL, "fhip_q4k_matmul_noalloc_f32: null pointer");
  if (((uintptr_t)dX & 15) || ((uintptr_t)dPacked & 15))
    return fail(FHIP_EINVAL, "fhip_q4k_matmul_noalloc_f32: dX and dPacked must be 16-byte aligned");
  if (int rc = check_weight("fhip_q4k_matmul_noalloc_f32", dPacked, kWeightQ4K, out, in)) return rc;
  const size_t need = q4k_matmul_ws_bytes(out, in, P);
  if (need > kScratchBytes)
    return fail(FHIP_EINVAL,
                "fhip_q4k_matmul_noalloc_f32: [%d x %d] at P=%d needs %zu bytes of scratch, more "
                "than the %zu-byte static region; use fhip_q4k_matmul_f32", out, in, P, need,
                kScratchBytes);
  void *base = nullptr;
  if (int rc = scratch_for_current_device(&base)) return rc;
  untag_range(dY, (size_t)P * out * 4);
  ScratchScope scope(base, kScratchBytes);
  return q4k_matmul_run(dPacked, dX, dY, out, in, P);
}

}  // extern "C"
