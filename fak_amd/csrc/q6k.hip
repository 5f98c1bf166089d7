// q6k.hip — GGUF Q6_K weights on the device: upload, the bit-exact dequantizer and the GEMV.
//
// Q6_K super-block (256 weights, 210 bytes; internal/model/quant_kquant.go:45,139-163):
//   [0, 128)    ql: low 4 bits; [128, 192) qh: high 2 bits; [192, 208) 16 int8 scales;
//   [208, 210)  f16 d.
// Weight n + l + 32 i (half n in {0, 128}, l < 32, i < 4) takes the low (i < 2) or high
// (i >= 2) nibble of ql[n/2 + l + 32 (i & 1)], bits 2i..2i+1 of qh[n/4 + l] as bits 4-5, and
// scale sc[n/16 + l/16 + 2i]: w = (d * f32(sc)) * f32(q - 32).
//
// The weights stay in their GGUF bytes on the device (a Q6_K row is not 16-byte aligned in
// general, so the GEMV reads bytes). This is the correctness-first form of the row: one wave
// per output row, lane (half, l) owns weights half*128 + l + 32 i of every super-block, the
// activation slices come from L2, and the f32 partials are reduced across the wave.
#include "f16bits.hpp"
#include "kernels.hpp"

namespace fhip {
namespace {

constexpr int kQ6kBlock = 210;

__device__ __forceinline__ int q6_code(uint32_t ql, uint32_t qh, int i) {
  const uint32_t lo = (i >= 2 ? ql >> 4 : ql) & 0x0fu;
  return (int)(lo | (((qh >> (2 * i)) & 3u) << 4)) - 32;
}

// One thread per super-block: the 256 weights exactly as q6kDequantSuperBlock computes them.
__global__ void q6k_dequant_kernel(float *__restrict__ dw, const uint8_t *__restrict__ raw,
                                   long long nblocks) {
  const long long id = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= nblocks) return;
  const uint8_t *blk = raw + (size_t)id * kQ6kBlock;
  const float d = f16_bits_to_f32(blk[208] | (blk[209] << 8));
  float *o = dw + (size_t)id * 256;
  for (int h = 0; h < 2; ++h) {
    const uint8_t *ql = blk + 64 * h, *qh = blk + 128 + 32 * h;
    const int8_t *sc = reinterpret_cast<const int8_t *>(blk + 192 + 8 * h);
    for (int l = 0; l < 32; ++l) {
      const uint32_t q0 = ql[l], q1 = ql[l + 32], hh = qh[l];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int q = q6_code(i & 1 ? q1 : q0, hh, i);
        o[128 * h + l + 32 * i] = __fmul_rn(__fmul_rn(d, (float)sc[l / 16 + 2 * i]), (float)q);
      }
    }
  }
}

// GEMV for up to 4 tokens per launch slice: wave = one row, lane (h, l) = weights
// 128 h + l + 32 i of each super-block.
template <int MT>
__global__ __launch_bounds__(256) void q6k_gemv_kernel(const uint8_t *__restrict__ W,
                                                       const float *__restrict__ X,
                                                       float *__restrict__ Y, int N, int K,
                                                       int t0) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= N) return;  // whole waves only: no barrier follows
  const int nblk = K / 256;
  const int h = lane >> 5, l = lane & 31;
  const uint8_t *rp = W + (size_t)row * nblk * kQ6kBlock;
  float acc[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) acc[t] = 0.f;
  for (int b = 0; b < nblk; ++b) {
    const uint8_t *blk = rp + (size_t)b * kQ6kBlock;
    const uint32_t q0 = blk[64 * h + l], q1 = blk[64 * h + l + 32], hh = blk[128 + 32 * h + l];
    const int8_t *sc = reinterpret_cast<const int8_t *>(blk + 192 + 8 * h + (l >> 4));
    const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)(blk[208] | (blk[209] << 8)));
    float w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = d * (float)sc[2 * i] * (float)q6_code(i & 1 ? q1 : q0, hh, i);
    const size_t xo = (size_t)b * 256 + 128 * h + l;
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const float *x = X + (size_t)(t0 + t) * K + xo;
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[t] = fmaf(w[i], x[32 * i], acc[t]);
    }
  }
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    float v = acc[t];
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
    if (lane == 0) Y[(size_t)(t0 + t) * N + row] = v;
  }
}

int check_q6k_shape(const char *who, int out, int in) {
  if (out <= 0 || in <= 0 || in % 256 != 0)
    return fail(FHIP_EINVAL, "%s: need out > 0 and in a positive multiple of 256 (out=%d in=%d)",
                who, out, in);
  return FHIP_OK;
}

}  // namespace

// Q6_K GEMV over any number of tokens, four per launch.
int q6k_gemv(const void *dRaw, const float *dX, float *dY, int out, int in, int P) {
  const unsigned grid = (unsigned)ceil_div(out, 4);
  const uint8_t *W = (const uint8_t *)dRaw;
  for (int t0 = 0; t0 < P; t0 += 4) {
    const int mt = P - t0 < 4 ? P - t0 : 4;
    switch (mt) {
      case 1: q6k_gemv_kernel<1><<<grid, 256, 0, stream()>>>(W, dX, dY, out, in, t0); break;
      case 2: q6k_gemv_kernel<2><<<grid, 256, 0, stream()>>>(W, dX, dY, out, in, t0); break;
      case 3: q6k_gemv_kernel<3><<<grid, 256, 0, stream()>>>(W, dX, dY, out, in, t0); break;
      default: q6k_gemv_kernel<4><<<grid, 256, 0, stream()>>>(W, dX, dY, out, in, t0); break;
    }
    FHIP_CHECK_LAUNCH("q6k_gemv_kernel");
  }
  return FHIP_OK;
}

}  // namespace fhip

using namespace fhip;

extern "C" {

size_t fhip_q6k_bytes(int out, int in) {
  if (out <= 0 || in <= 0 || in % 256) return 0;
  return (size_t)out * (in / 256) * kQ6kBlock;
}

void *fhip_q6k_upload(const uint8_t *hRaw, int out, int in) {
  clear_error();
  if (check_q6k_shape("fhip_q6k_upload", out, in)) return nullptr;
  if (!hRaw) { fail(FHIP_EINVAL, "fhip_q6k_upload: null host pointer"); return nullptr; }
  const size_t bytes = fhip_q6k_bytes(out, in);
  void *d = fhip_malloc(bytes);
  if (!d) return nullptr;
  if (fhip_h2d(d, hRaw, bytes) != FHIP_OK) {
    fhip_free(d);
    return nullptr;
  }
  return d;
}

int fhip_q6k_dequant_f32(float *dW, const void *dRaw, int out, int in) {
  clear_error();
  if (int rc = check_q6k_shape("fhip_q6k_dequant_f32", out, in)) return rc;
  if (!dRaw || !dW) return fail(FHIP_EINVAL, "fhip_q6k_dequant_f32: null pointer");
  const long long nb = (long long)out * (in / 256);
  q6k_dequant_kernel<<<(unsigned)((nb + 255) / 256), 256, 0, stream()>>>(
      dW, (const uint8_t *)dRaw, nb);
  FHIP_CHECK_LAUNCH("q6k_dequant_kernel");
  return FHIP_OK;
}

int fhip_q6k_matmul_f32(const void *dRaw, const float *dX, float *dY, int out, int in, int P) {
  clear_error();
  if (int rc = check_q6k_shape("fhip_q6k_matmul_f32", out, in)) return rc;
  if (P < 0) return fail(FHIP_EINVAL, "fhip_q6k_matmul_f32: P=%d < 0", P);
  if (P == 0) return FHIP_OK;
  if (!dRaw || !dX || !dY) return fail(FHIP_EINVAL, "fhip_q6k_matmul_f32: null pointer");
  return q6k_gemv(dRaw, dX, dY, out, in, P);
}

}  // extern "C"
