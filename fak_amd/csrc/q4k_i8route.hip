// q4k_i8route.hip — the int8 Q4_K route (FAK_KQ_INT8): the Q4_K matmul with the activation
// quantized to int8 per 32 values, bit-identical to the CPU reference's int8 decode GEMV
// q4kMatRowsRangeInt8 (internal/model/quant_q4k_int8.go:135-142) and, per token, its batched
// twin q4kGemmRangeInt8 (internal/model/quant_q4k.go:359-372).
//
// The reference computes, per row o and token t:
//   qx, dx = quantizeRowQ8scalar(x_t)             (internal/model/quant_quantize.go:16-43)
//   I_s = sum nibble * qx,  S_s = sum qx           per 32-value sub-block s (int32, exact)
//   acc = 0;  for b, s in order:  acc += (f32(I_s) * (d * f32(sc_s))) * dx_s
//                                 acc -= (f32(S_s) * (dmin * f32(m_s))) * dx_s
// Every float operation is a single IEEE-rounded operation, so this file is built with
// -ffp-contract=off and the only freedom is in the integer sums.
//
// Device plan. A workgroup owns one 16-row tile (tiled.hpp) and a group of up to 16 tokens.
//   * prep kernel: one thread per (token, 32-block) quantizes the activation exactly as the
//     reference does, writing the int8 codes [P][K] and per block {f32(S), dx}.
//   * phase 1 (all KW waves, records split round-robin): the integer sums run on the int8 MFMA
//     v_mfma_i32_16x16x32_i8, whose K = 32 is exactly one sub-block: A = 16 tokens x 32 codes,
//     B = 32 nibbles x 16 rows of the tile, so D[t][row] = I_s. Lane (g, r) feeds the nibbles
//     of row r at positions 8g..8g+7 straight from its tiled 16-byte pieces and the codes of
//     token r at the same positions; result lane (g, r) holds I_s of row r for tokens 4g..4g+3.
//     It forms the two reference terms of every (row, token, sub-block) with the reference's
//     roundings and parks them in LDS.
//   * phase 2: one lane per (row, token) adds the terms in the reference order.
// The terms of a window of records are kept in LDS; long rows (or many tokens) take several
// windows, the chain lanes carrying their sums across them.
#include "kernels.hpp"
#include "q8round.hpp"

namespace fhip {
namespace {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

constexpr int kTokGroup = 16;         // tokens per workgroup (the MFMA's A rows)
constexpr int kTermLds = 64 * 1024;   // LDS budget for one window of terms

// One thread per (token, 32-block): codes to qx[t][K], {f32(S), dx} to sd[t][K/32].
__global__ __launch_bounds__(256) void i8r_prep_kernel(const float *__restrict__ X, int P, int K,
                                                       int8_t *__restrict__ qx,
                                                       float2 *__restrict__ sd) {
  const int nb = K / 32;
  const long long id = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= (long long)P * nb) return;
  const int t = (int)(id / nb), b = (int)(id - (long long)t * nb);
  const size_t off = (size_t)t * K + (size_t)b * 32;
  float x[32];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float4 v = reinterpret_cast<const float4 *>(X + off)[i];
    x[4 * i] = v.x;
    x[4 * i + 1] = v.y;
    x[4 * i + 2] = v.z;
    x[4 * i + 3] = v.w;
  }
  int8_t q[32];
  int s = 0;
  const float d = q8_quant_block32(x, q, &s);
  uint4 *dst = reinterpret_cast<uint4 *>(qx + off);
  dst[0] = *reinterpret_cast<const uint4 *>(q);
  dst[1] = *reinterpret_cast<const uint4 *>(q + 16);
  sd[id] = make_float2((float)s, d);
}

// GetScaleMinK4 (internal/model/quantbits.go:42-47) of sub-block s from the header words
// y = scales[0..3], z = scales[4..7], w = scales[8..11].
__device__ __forceinline__ void scale_min_s(uint32_t y, uint32_t z, uint32_t w, int s,
                                            uint32_t &sc, uint32_t &m) {
  const uint32_t o = 8u * (uint32_t)(s & 3);
  if (s < 4) {
    sc = __builtin_amdgcn_ubfe(y, o, 6);
    m = __builtin_amdgcn_ubfe(z, o, 6);
  } else {
    sc = __builtin_amdgcn_ubfe(w, o, 4) | (__builtin_amdgcn_ubfe(y, o + 6, 2) << 4);
    m = __builtin_amdgcn_ubfe(w, o + 4, 4) | (__builtin_amdgcn_ubfe(z, o + 6, 2) << 4);
  }
}

__global__ __launch_bounds__(256) void q4k_i8route_kernel(
    const uint8_t *__restrict__ W, const int8_t *__restrict__ qx, const float2 *__restrict__ sd,
    float *__restrict__ Y, int N, int K, int nblk, int P, int Wrec, int stride, int KW) {
  extern __shared__ __align__(16) float2 terms[];  // [pg][16 rows][stride]
  const int tile = blockIdx.x;
  const int t0 = blockIdx.y * kTokGroup;
  const int pg = min(kTokGroup, P - t0);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane >> 4, r = lane & 15;
  const int nsb = K / 32;
  const uint8_t *base = W + (size_t)tile * nblk * kQ4kRecord;
  // A operand source: token r's codes (zero for rows past the group's tokens)
  const bool arow = r < pg;
  const int8_t *xrow = qx + (size_t)(t0 + (arow ? r : 0)) * K + 8 * g;

  // chain lane: (token ct, row cj)
  const int c = threadIdx.x;
  const bool chain = c < 16 * pg;
  const int ct = c >> 4, cj = c & 15;
  float acc = 0.f;
  const uint32_t k0F = 0x0F0F0F0Fu;

  for (int wb = 0; wb < nblk; wb += Wrec) {
    const int we = min(nblk, wb + Wrec);
    for (int b = wb + wave; b < we; b += KW) {
      const uint8_t *rec = base + (size_t)b * kQ4kRecord;
      const uint4 h = *reinterpret_cast<const uint4 *>(rec + 16 * r);
      const uint4 qa = *reinterpret_cast<const uint4 *>(rec + kQ4kHdr + 16 * lane);
      const uint4 qb = *reinterpret_cast<const uint4 *>(rec + kQ4kHdr + 1024 + 16 * lane);
      const uint32_t q[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
      long A[8];
#pragma unroll
      for (int s = 0; s < 8; ++s)
        A[s] = arow ? *reinterpret_cast<const long *>(xrow + (size_t)b * 256 + 32 * s) : 0L;
      const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)(h.x & 0xffffu));
      const float dmin = (float)__builtin_bit_cast(_Float16, (uint16_t)(h.x >> 16));
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        // chunk s/2 = words q[2 (s/2)], q[2 (s/2) + 1]: low nibbles for even s, high for odd
        const uint32_t w0 = q[2 * (s >> 1)], w1 = q[2 * (s >> 1) + 1];
        const uint32_t n0 = (s & 1) ? (w0 >> 4) & k0F : w0 & k0F;
        const uint32_t n1 = (s & 1) ? (w1 >> 4) & k0F : w1 & k0F;
        const long B = (long)(((unsigned long)n1 << 32) | n0);
        const i32x4 D = __builtin_amdgcn_mfma_i32_16x16x32_i8(A[s], B, i32x4{0, 0, 0, 0}, 0, 0, 0);
        uint32_t sc, m;
        scale_min_s(h.y, h.z, h.w, s, sc, m);
        const float ws = __fmul_rn(d, (float)sc), wm = __fmul_rn(dmin, (float)m);
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int t = 4 * g + v;
          if (t < pg) {
            const float2 e = sd[(size_t)(t0 + t) * nsb + (size_t)b * 8 + s];  // {f32(S), dx}
            const float T1 = __fmul_rn(__fmul_rn((float)D[v], ws), e.y);
            const float T2 = __fmul_rn(__fmul_rn(e.x, wm), e.y);
            terms[(t * 16 + r) * stride + (b - wb) * 8 + s] = make_float2(T1, T2);
          }
        }
      }
    }
    __syncthreads();
    if (chain) {
      const float4 *tt = reinterpret_cast<const float4 *>(terms + (ct * 16 + cj) * stride);
      const int n2 = (we - wb) * 4;  // pairs of sub-blocks
      for (int k = 0; k < n2; ++k) {
        const float4 v = tt[k];
        acc = __fadd_rn(acc, v.x);
        acc = __fsub_rn(acc, v.y);
        acc = __fadd_rn(acc, v.z);
        acc = __fsub_rn(acc, v.w);
      }
    }
    __syncthreads();
  }
  if (chain) {
    const int row = tile * 16 + cj;
    if (row < N) Y[(size_t)(t0 + ct) * N + row] = acc;
  }
}

}  // namespace
}  // namespace fhip

using namespace fhip;

// The int8 Q4_K route on a tiled Q4_K weight (fhip_q4k_upload): Y[P][out] from X[P][in], every
// value bit-identical to q4kMatRowsRangeInt8 / q4kGemmRangeInt8 on the same GGUF bytes.
extern "C" int fhip_q4k_matmul_int8_f32(const void *dPacked, const float *dX, float *dY, int out,
                                        int in, int P) {
  clear_error();
  if (out < 0 || in <= 0 || P < 0 || in % 256)
    return fail(FHIP_EINVAL, "fhip_q4k_matmul_int8_f32: need in a positive multiple of 256 "
                             "(out=%d in=%d P=%d)", out, in, P);
  if (out == 0 || P == 0) return FHIP_OK;
  if (!dPacked || !dX || !dY) return fail(FHIP_EINVAL, "fhip_q4k_matmul_int8_f32: null pointer");
  if (((uintptr_t)dX & 15) != 0)
    return fail(FHIP_EINVAL, "fhip_q4k_matmul_int8_f32: dX must be 16-byte aligned");
  const int nblk = in / 256, nsb = in / 32;
  const size_t qbytes = ((size_t)P * in + 255) & ~(size_t)255;
  unsigned char *ws = (unsigned char *)workspace(qbytes + (size_t)P * nsb * sizeof(float2));
  if (!ws) return FHIP_ENOMEM;
  int8_t *qx = reinterpret_cast<int8_t *>(ws);
  float2 *sd = reinterpret_cast<float2 *>(ws + qbytes);

  const long long nq = (long long)P * nsb;
  i8r_prep_kernel<<<(unsigned)((nq + 255) / 256), 256, 0, stream()>>>(dX, P, in, qx, sd);
  FHIP_CHECK_LAUNCH("i8r_prep_kernel");

  // Shape: a 16-row tile per workgroup; enough waves for the chain lanes (16 per token) and,
  // for short grids, to spread each tile's records; a window of records whose terms fit in
  // kTermLds (rows padded by 16 bytes so the chain lanes' reads spread over the banks).
  const int ntiles = q4k_tiles(out);
  const int groups = ceil_div(P, kTokGroup);
  const int pg = P < kTokGroup ? P : kTokGroup;
  int KW = 1;
  while (KW * 64 < 16 * pg) KW *= 2;
  while (KW < 4 && (long long)ntiles * groups * KW < 4LL * cu_count() && nblk >= 4 * KW) KW *= 2;
  const int per_rec = pg * 16 * 8 * (int)sizeof(float2);  // bytes of terms per record
  int wmax = (kTermLds - pg * 16 * 16) / per_rec;
  if (wmax < 1) wmax = 1;
  const int nwin = ceil_div(nblk, wmax);
  const int Wrec = ceil_div(nblk, nwin);
  const int stride = Wrec * 8 + 2;  // float2 per (token, row)
  const size_t lds = (size_t)pg * 16 * stride * sizeof(float2);
  if (lds > (size_t)lds_limit())
    return fail(FHIP_EINVAL, "fhip_q4k_matmul_int8_f32: %zu B of LDS exceeds the device limit",
                lds);
  dim3 grid(ntiles, groups);
  q4k_i8route_kernel<<<grid, 64 * KW, lds, stream()>>>(
      reinterpret_cast<const uint8_t *>(dPacked), qx, sd, dY, out, in, nblk, P, Wrec, stride, KW);
  FHIP_CHECK_LAUNCH("q4k_i8route_kernel");
  return FHIP_OK;
}
