// xprep.hip — activation operand preparation for the large-M GEMM (layout in kernels.hpp).
//
// The weights never leave their 4-bit form in HBM; the activation side is converted once per
// call into the exact MFMA operand order the GEMM loads with one 16-byte read per lane. A
// single f16 per activation is enough for the GEMM's error bound. (The small-M kernels stage
// their hi/lo f16 activation split in LDS themselves, gemv_common.hpp.)
#include <cstdlib>

#include "kernels.hpp"

namespace fhip {
namespace {

// One thread per (16-token tile mt, slice s, lane l): 8 f16 activations.
__global__ void gemm_xprep_kernel(const float *__restrict__ X, int M, int K, int nslices,
                                  long long total, uint4 *__restrict__ xa) {
  const long long id = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= total) return;
  const int l = (int)(id & 63);
  const long long ms = id >> 6;
  const int mt = (int)(ms / nslices), s = (int)(ms - (long long)mt * nslices);
  const int t = 16 * mt + (l & 15), g = l >> 4;
  f16x8 h;
  if (t < M) {
    const float *x = X + (size_t)t * K + 32 * s + 8 * g;
    const float4 v0 = *reinterpret_cast<const float4 *>(x);
    const float4 v1 = *reinterpret_cast<const float4 *>(x + 4);
    const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
#pragma unroll
    for (int j = 0; j < 8; ++j) h[j] = (_Float16)v[perm8(j)];
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) h[j] = (_Float16)0.f;
  }
  xa[id] = __builtin_bit_cast(uint4, h);
}

}  // namespace

int env_int(const char *name) {
  const char *v = getenv(name);
  return v ? atoi(v) : 0;
}

int launch_gemm_xprep(const float *X, int M, int K, void *xa) {
  const int nslices = K / 32;
  const long long total = (long long)gemm_mt(M) * nslices * 64;
  const int bs = 256;
  gemm_xprep_kernel<<<(unsigned)((total + bs - 1) / bs), bs, 0, stream()>>>(X, M, K, nslices,
                                                                           total, (uint4 *)xa);
  FHIP_CHECK_LAUNCH("gemm_xprep_kernel");
  return FHIP_OK;
}

}  // namespace fhip
