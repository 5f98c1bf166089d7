// q4k_layout.hip — Q4_K weight upload: raw GGUF super-blocks <-> the tiled device layout
// (described in tiled.hpp), and the bit-exact device dequantizer used to prove the layout and
// the f16/6-bit decoding reproduce q4kDequantSuperBlock (internal/model/quant_q4k.go:90-111).
#include "common.hpp"
#include "f16bits.hpp"
#include "tiled.hpp"

namespace fhip {
namespace {

// One thread per 16-byte unit of the tiled buffer (144 units per record). Units 0..15 are the
// row headers, 16..143 the two 1 KiB lane parts.
__global__ void q4k_repack_kernel(uint8_t *__restrict__ dst, const uint8_t *__restrict__ raw,
                                  int out, int nblk, long long units) {
  const long long u = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (u >= units) return;
  const long long rec = u / 144;
  const int k = (int)(u - rec * 144);
  const int T = (int)(rec / nblk), b = (int)(rec - (long long)T * nblk);
  uint4 v = make_uint4(0, 0, 0, 0);
  if (k < 16) {
    const int row = T * kTileRows + k;
    if (row < out)
      v = *reinterpret_cast<const uint4 *>(raw + ((size_t)row * nblk + b) * kQ4kBlock);
  } else {
    const int idx = k - 16, L = idx >> 6, l = idx & 63, g = l >> 4, r = l & 15;
    const int row = T * kTileRows + r;
    if (row < out) {
      const uint8_t *qs = raw + ((size_t)row * nblk + b) * kQ4kBlock + 16;
      const uint2 a = *reinterpret_cast<const uint2 *>(qs + 64 * L + 8 * g);
      const uint2 c = *reinterpret_cast<const uint2 *>(qs + 64 * L + 32 + 8 * g);
      v = make_uint4(a.x, a.y, c.x, c.y);
    }
  }
  reinterpret_cast<uint4 *>(dst)[u] = v;
}

__global__ void q4k_unpack_kernel(uint8_t *__restrict__ raw, const uint8_t *__restrict__ src,
                                  int out, int nblk, long long units) {
  const long long u = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (u >= units) return;
  const long long rec = u / 144;
  const int k = (int)(u - rec * 144);
  const int T = (int)(rec / nblk), b = (int)(rec - (long long)T * nblk);
  const uint4 v = reinterpret_cast<const uint4 *>(src)[u];
  if (k < 16) {
    const int row = T * kTileRows + k;
    if (row < out) *reinterpret_cast<uint4 *>(raw + ((size_t)row * nblk + b) * kQ4kBlock) = v;
  } else {
    const int idx = k - 16, L = idx >> 6, l = idx & 63, g = l >> 4, r = l & 15;
    const int row = T * kTileRows + r;
    if (row < out) {
      uint8_t *qs = raw + ((size_t)row * nblk + b) * kQ4kBlock + 16;
      *reinterpret_cast<uint2 *>(qs + 64 * L + 8 * g) = make_uint2(v.x, v.y);
      *reinterpret_cast<uint2 *>(qs + 64 * L + 32 + 8 * g) = make_uint2(v.z, v.w);
    }
  }
}

// GetScaleMinK4 (internal/model/quantbits.go:42-47).
__device__ __forceinline__ void scale_min_k4(int j, const uint8_t *q, uint32_t &sc, uint32_t &m) {
  if (j < 4) {
    sc = q[j] & 63u;
    m = q[j + 4] & 63u;
  } else {
    sc = (q[j + 4] & 0x0fu) | ((uint32_t)(q[j - 4] >> 6) << 4);
    m = (uint32_t)(q[j + 4] >> 4) | ((uint32_t)(q[j] >> 6) << 4);
  }
}

// One thread per (row, super-block, 32-weight sub-block). The arithmetic is the reference's:
// d1 = d*f32(sc), m1 = dmin*f32(m), w = d1*f32(nib) - m1, each product rounded on its own.
__global__ void q4k_dequant_kernel(float *__restrict__ dw, const uint8_t *__restrict__ src,
                                   int out, int nblk, long long items) {
#pragma clang fp contract(off)
  const long long it = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (it >= items) return;
  const int s = (int)(it & 7);
  const long long rb = it >> 3;
  const int row = (int)(rb / nblk), b = (int)(rb - (long long)row * nblk);
  const int T = row / kTileRows, r = row % kTileRows;
  const uint8_t *rec = src + ((size_t)T * nblk + b) * kQ4kRecord;
  const uint8_t *hdr = rec + 16 * r;
  const float d = f16_bits_to_f32(hdr[0] | (hdr[1] << 8));
  const float mn = f16_bits_to_f32(hdr[2] | (hdr[3] << 8));
  uint32_t sc, m;
  scale_min_k4(s, hdr + 4, sc, m);
  const float d1 = __fmul_rn(d, (float)sc), m1 = __fmul_rn(mn, (float)m);
  const int c = s >> 1, hi = s & 1;  // nibble chunk and which half of each byte
  const int L = c >> 1, half = c & 1;
  float *o = dw + (size_t)row * nblk * 256 + (size_t)b * 256 + 32 * s;
  for (int l = 0; l < 32; ++l) {
    const int g = l >> 3, i = l & 7;
    const uint8_t byte = rec[kQ4kHdr + 1024 * L + 16 * (16 * g + r) + 8 * half + i];
    const uint32_t nib = hi ? (byte >> 4) : (byte & 0x0fu);
    o[l] = __fsub_rn(__fmul_rn(d1, (float)nib), m1);
  }
}

int check_q4k_shape(const char *who, int out, int in) {
  if (out <= 0 || in <= 0 || in % 256 != 0)
    return fail(FHIP_EINVAL, "%s: need out > 0 and in a positive multiple of 256 (out=%d in=%d)",
                who, out, in);
  return FHIP_OK;
}

}  // namespace
}  // namespace fhip

using namespace fhip;

extern "C" {

size_t fhip_q4k_packed_bytes(int out, int in) {
  if (out <= 0 || in <= 0 || in % 256) return 0;
  return q4k_packed_bytes(out, in);
}

int fhip_q4k_repack(void *dPacked, const uint8_t *dRaw, int out, int in) {
  clear_error();
  if (int rc = check_q4k_shape("fhip_q4k_repack", out, in)) return rc;
  if (!dPacked || !dRaw) return fail(FHIP_EINVAL, "fhip_q4k_repack: null pointer");
  const int nblk = in / 256;
  const long long units = (long long)q4k_tiles(out) * nblk * 144;
  const int bs = 256;
  untag_range(dPacked, q4k_packed_bytes(out, in));
  q4k_repack_kernel<<<(unsigned)((units + bs - 1) / bs), bs, 0, stream()>>>(
      (uint8_t *)dPacked, dRaw, out, nblk, units);
  FHIP_CHECK_LAUNCH("q4k_repack_kernel");
  tag_weight(dPacked, q4k_packed_bytes(out, in), kWeightQ4K, out, in);
  return FHIP_OK;
}

int fhip_q4k_unpack(uint8_t *dRaw, const void *dPacked, int out, int in) {
  clear_error();
  if (int rc = check_q4k_shape("fhip_q4k_unpack", out, in)) return rc;
  if (!dPacked || !dRaw) return fail(FHIP_EINVAL, "fhip_q4k_unpack: null pointer");
  if (int rc = check_weight("fhip_q4k_unpack", dPacked, kWeightQ4K, out, in)) return rc;
  untag_range(dRaw, (size_t)out * (in / 256) * kQ4kBlock);
  const int nblk = in / 256;
  const long long units = (long long)q4k_tiles(out) * nblk * 144;
  const int bs = 256;
  q4k_unpack_kernel<<<(unsigned)((units + bs - 1) / bs), bs, 0, stream()>>>(
      dRaw, (const uint8_t *)dPacked, out, nblk, units);
  FHIP_CHECK_LAUNCH("q4k_unpack_kernel");
  return FHIP_OK;
}

int fhip_q4k_dequant_f32(float *dW, const void *dPacked, int out, int in) {
  clear_error();
  if (int rc = check_q4k_shape("fhip_q4k_dequant_f32", out, in)) return rc;
  if (!dPacked || !dW) return fail(FHIP_EINVAL, "fhip_q4k_dequant_f32: null pointer");
  if (int rc = check_weight("fhip_q4k_dequant_f32", dPacked, kWeightQ4K, out, in)) return rc;
  untag_range(dW, (size_t)out * in * 4);
  const int nblk = in / 256;
  const long long items = (long long)out * nblk * 8;
  const int bs = 256;
  q4k_dequant_kernel<<<(unsigned)((items + bs - 1) / bs), bs, 0, stream()>>>(
      dW, (const uint8_t *)dPacked, out, nblk, items);
  FHIP_CHECK_LAUNCH("q4k_dequant_kernel");
  return FHIP_OK;
}

void *fhip_q4k_upload(const uint8_t *hRaw, int out, int in) {
  clear_error();
  if (check_q4k_shape("fhip_q4k_upload", out, in)) return nullptr;
  if (!hRaw) { fail(FHIP_EINVAL, "fhip_q4k_upload: null host pointer"); return nullptr; }
  const size_t rawBytes = (size_t)out * (in / 256) * kQ4kBlock;
  void *packed = fhip_malloc(q4k_packed_bytes(out, in));
  if (!packed) return nullptr;
  void *staging = fhip_malloc(rawBytes);
  if (!staging) { fhip_free(packed); return nullptr; }
  int rc = fhip_h2d(staging, hRaw, rawBytes);
  if (rc == FHIP_OK) rc = fhip_q4k_repack(packed, (const uint8_t *)staging, out, in);
  if (rc == FHIP_OK) {
    hipError_t e = hipStreamSynchronize(stream());
    if (e != hipSuccess) rc = hip_fail(e, "fhip_q4k_upload: hipStreamSynchronize");
  }
  fhip_free(staging);
  if (rc != FHIP_OK) { fhip_free(packed); return nullptr; }
  return packed;
}

}  // extern "C"
