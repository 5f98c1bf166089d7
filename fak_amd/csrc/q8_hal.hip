// q8_hal.hip — the HAL Q8 lane: int8 codes + f32 per-block scales with the activation quantized
// on the device (the semantics of fcuda_q8_matmul_f32, internal/compute/cuda_backend.h:104-111,
// whose CPU reference is cpuBackend.MatMul / BatchedMatMul on Q8_0,
// internal/compute/cpuref.go:113-191).
//
// Every result here is bit-identical to the CPU reference, not just within a tolerance:
//   * quantizeVecQ8 (cpuref.go:505-527): d = amax/127, inv = 1/d, code = q8round(x*inv), with
//     IEEE-rounded single operations and q8round's truncate-then-round-half-away rule
//     (internal/model/quant.go:89-104);
//   * MatMul = qdot8scalar (cpuref.go:532-548): per block the exact int32 dot, then
//     acc = acc + (f32(isum) * dw) * dx in block order. The int32 dot is exact in any order;
//     one lane owns a row's running sum and walks the blocks in order;
//   * BatchedMatMul = qgemm8cell (cpuref.go:553-577, lanes = 16): per block 16 pair products
//     p_k = w[2k]x[2k] + w[2k+1]x[2k+1], acc_k += f32(p_k) * (dw * dx), then the fixed pairwise
//     tree. One thread owns one (row, token) cell and its 16 lane sums.
// The reference is Go on amd64, which never fuses multiply-add, so this file is built with
// -ffp-contract=off (fak_amd/build.py): by default hipcc contracts a*b - c into one fma even when
// written with __fmul_rn/__fsub_rn, which turned q8round of a product that rounds to 43.5 into 43
// instead of 44.
#include "kernels.hpp"
#include "q8round.hpp"

namespace fhip {
namespace {

// One thread per (row, block): quantizeVecQ8 of X[rows][in] into codes [rows][in] and
// scales [rows][in / block].
__global__ void q8_quantize_kernel(const float *__restrict__ X, int8_t *__restrict__ codes,
                                   float *__restrict__ scales, int rows, int in, int block) {
  const int nblk = in / block;
  const long long id = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= (long long)rows * nblk) return;
  const int row = (int)(id / nblk), b = (int)(id - (long long)row * nblk);
  const float *xb = X + (size_t)row * in + (size_t)b * block;
  int8_t *qb = codes + (size_t)row * in + (size_t)b * block;
  float amax = 0.f;
  for (int i = 0; i < block; ++i) {
    const float a = fabsf(xb[i]);
    if (a > amax) amax = a;
  }
  const float d = __fdiv_rn(amax, 127.f);
  scales[id] = d;
  if (d == 0.f) {
    for (int i = 0; i < block; ++i) qb[i] = 0;
    return;
  }
  const float inv = __fdiv_rn(1.f, d);
  for (int i = 0; i < block; ++i) qb[i] = (int8_t)q8round(__fmul_rn(xb[i], inv));
}

// MatMul (one token): a wave owns 16 rows; the 4 lanes of a row each form the int32 dot of 8
// bytes of the current block, the quad sum is exact, and the row's first lane accumulates
// acc = acc + (f32(isum) * dw) * dx in block order.
__global__ __launch_bounds__(256) void q8_hal_gemv_kernel(
    const int8_t *__restrict__ codes, const float *__restrict__ wscale,
    const int8_t *__restrict__ qx, const float *__restrict__ dx, float *__restrict__ Y, int out,
    int in, int block) {
  const int lane = threadIdx.x & 63;
  const int row = (blockIdx.x * 4 + (threadIdx.x >> 6)) * 16 + (lane >> 2);
  const int q = lane & 3;
  const int nblk = in / block;
  const bool valid = row < out;
  const int8_t *wr = codes + (size_t)(valid ? row : 0) * in;
  const float *ws = wscale + (size_t)(valid ? row : 0) * nblk;
  float acc = 0.f;
  for (int b = 0; b < nblk; ++b) {
    int isum = 0;
    // this lane's dwords of the block: 4 * (q + 4 j), j = 0.. (block / 16 of them)
    for (int o = 4 * q; o < block; o += 16) {
      const int w4 = *reinterpret_cast<const int *>(wr + (size_t)b * block + o);
      const int x4 = *reinterpret_cast<const int *>(qx + (size_t)b * block + o);
      isum = __builtin_amdgcn_sdot4(w4, x4, isum, false);
    }
    isum += __shfl_xor(isum, 1);
    isum += __shfl_xor(isum, 2);
    acc = __fadd_rn(acc, __fmul_rn(__fmul_rn((float)isum, ws[b]), dx[b]));
  }
  if (valid && q == 0) Y[row] = acc;
}

// BatchedMatMul: one thread per (row o, token t), t fastest. Pair products come from sdot4 on
// the dword with the other pair's bytes masked to zero.
__global__ __launch_bounds__(256) void q8_hal_gemm_kernel(
    const int8_t *__restrict__ codes, const float *__restrict__ wscale,
    const int8_t *__restrict__ qx, const float *__restrict__ dx, float *__restrict__ Y, int out,
    int in, int P, int block) {
  const long long id = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= (long long)out * P) return;
  const int o = (int)(id / P), t = (int)(id - (long long)o * P);
  const int nblk = in / block;
  const int8_t *wr = codes + (size_t)o * in;
  const int8_t *xr = qx + (size_t)t * in;
  const float *ws = wscale + (size_t)o * nblk;
  const float *xs = dx + (size_t)t * nblk;
  float acc[16];
#pragma unroll
  for (int k = 0; k < 16; ++k) acc[k] = 0.f;
  for (int b = 0; b < nblk; ++b) {
    const int *w4 = reinterpret_cast<const int *>(wr + (size_t)b * block);
    const int *x4 = reinterpret_cast<const int *>(xr + (size_t)b * block);
    const float s = __fmul_rn(ws[b], xs[b]);
#pragma unroll
    for (int j = 0; j < 8; ++j) {  // dword j holds pairs 2j (bytes 0-1) and 2j + 1 (bytes 2-3)
      const int w = w4[j], x = x4[j];
      const int p0 = __builtin_amdgcn_sdot4(w & 0x0000FFFF, x, 0, false);
      const int p1 = __builtin_amdgcn_sdot4(w & (int)0xFFFF0000u, x, 0, false);
      acc[2 * j] = __fadd_rn(acc[2 * j], __fmul_rn((float)p0, s));
      acc[2 * j + 1] = __fadd_rn(acc[2 * j + 1], __fmul_rn((float)p1, s));
    }
  }
#pragma unroll
  for (int k = 0; k < 8; ++k) acc[k] = __fadd_rn(acc[k], acc[k + 8]);
#pragma unroll
  for (int k = 0; k < 4; ++k) acc[k] = __fadd_rn(acc[k], acc[k + 4]);
  acc[0] = __fadd_rn(acc[0], acc[2]);
  acc[1] = __fadd_rn(acc[1], acc[3]);
  Y[(size_t)t * out + o] = __fadd_rn(acc[0], acc[1]);
}

int launch_quantize(const float *X, int8_t *codes, float *scales, int rows, int in, int block) {
  const long long n = (long long)rows * (in / block);
  if (n == 0) return FHIP_OK;
  const int bs = 256;
  q8_quantize_kernel<<<(unsigned)((n + bs - 1) / bs), bs, 0, stream()>>>(X, codes, scales, rows,
                                                                         in, block);
  FHIP_CHECK_LAUNCH("q8_quantize_kernel");
  return FHIP_OK;
}

bool aligned4(const void *p) { return ((uintptr_t)p & 3) == 0; }

}  // namespace
}  // namespace fhip

using namespace fhip;

extern "C" int fhip_q8_quantize_f32(const float *dX, int8_t *dCodes, float *dScales, int rows,
                                    int in, int block) {
  clear_error();
  if (rows < 0 || in < 0 || block <= 0 || in % block)
    return fail(FHIP_EINVAL, "fhip_q8_quantize_f32: need rows >= 0 and in a multiple of block "
                             "(rows=%d in=%d block=%d)", rows, in, block);
  if ((!dX || !dCodes || !dScales) && rows > 0 && in > 0)
    return fail(FHIP_EINVAL, "fhip_q8_quantize_f32: null pointer");
  if (rows > 0 && in > 0) {
    untag_range(dCodes, (size_t)rows * in);
    untag_range(dScales, (size_t)rows * (in / block) * 4);
  }
  return launch_quantize(dX, dCodes, dScales, rows, in, block);
}

extern "C" int fhip_q8_matmul_f32(const int8_t *dCodes, const float *dScales, const float *dX,
                                  float *dY, int out, int in, int P, int block) {
  clear_error();
  if (out < 0 || in <= 0 || P < 0 || block <= 0 || in % block || block % 4)
    return fail(FHIP_EINVAL, "fhip_q8_matmul_f32: need in a positive multiple of block and "
                             "block a multiple of 4 (out=%d in=%d P=%d block=%d)",
                out, in, P, block);
  if (P > 1 && block < 32)
    return fail(FHIP_EINVAL, "fhip_q8_matmul_f32: the batched (P > 1) lane reads 16 pairs per "
                             "block and needs block >= 32 (block=%d)", block);
  if (out == 0 || P == 0) return FHIP_OK;
  if (!dCodes || !dScales || !dX || !dY)
    return fail(FHIP_EINVAL, "fhip_q8_matmul_f32: null pointer");
  if (!aligned4(dCodes)) return fail(FHIP_EINVAL, "fhip_q8_matmul_f32: dCodes must be 4-byte aligned");
  untag_range(dY, (size_t)P * out * 4);
  const int nblk = in / block;
  // activation codes and scales in the library workspace (calls on one library are serialized)
  const size_t qbytes = ((size_t)P * in + 255) & ~(size_t)255;
  unsigned char *ws = (unsigned char *)workspace(qbytes + (size_t)P * nblk * 4);
  if (!ws) return FHIP_ENOMEM;
  int8_t *qx = reinterpret_cast<int8_t *>(ws);
  float *dx = reinterpret_cast<float *>(ws + qbytes);
  if (int rc = launch_quantize(dX, qx, dx, P, in, block)) return rc;
  if (P == 1) {
    const int waves = ceil_div(out, 16);
    q8_hal_gemv_kernel<<<ceil_div(waves, 4), 256, 0, stream()>>>(dCodes, dScales, qx, dx, dY,
                                                                 out, in, block);
    FHIP_CHECK_LAUNCH("q8_hal_gemv_kernel");
    return FHIP_OK;
  }
  const long long n = (long long)out * P;
  q8_hal_gemm_kernel<<<(unsigned)((n + 255) / 256), 256, 0, stream()>>>(dCodes, dScales, qx, dx,
                                                                        dY, out, in, P, block);
  FHIP_CHECK_LAUNCH("q8_hal_gemm_kernel");
  return FHIP_OK;
}
