// q8_0.hip — GGUF Q8_0 weights (34-byte blocks: f16 d + 32 int8 codes; gguf.go:24): upload
// into the tiled layout (tiled.hpp), bit-exact dequant, and the small-M matmul
//   Y[t][o] = sum_k (f32(int8 code) * d) * X[t][k]
// — the device form of kQuantMatRowsRange(kind Q8_0) (internal/model/quant_kquant.go:210-232
// with q8_0DequantBlock, internal/model/quant_iquant.go:14-19).
//
// Each 32-weight block is one K=32 f16 MFMA step: the codes become exact f16 values through
// the exponent trick ((b ^ 0x80) | 0x6400 = 1152 + b), the activation is the scaled hi/lo f16
// pair of gemv_common.hpp (x = e * (hi + lo), e a power of two per block and token), and after
// the MFMA the block scales are applied on the VALU:
//   y += (d e) * (T - 1152 * S),   T = MFMA sum, S = sum of the block's scaled activations.
#include "gemv_common.hpp"

namespace fhip {
namespace {

constexpr int kUnits = kQ8Record / 16;  // 68 sixteen-byte units per record

// Units 0..3: row scales (rows 4u..4u+3, 4 B each); units 4..67: lanes 0..63.
__global__ void q8_repack_kernel(uint8_t *__restrict__ dst, const uint8_t *__restrict__ raw,
                                 int out, int nb, int npairs, long long units) {
  const long long u = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (u >= units) return;
  const long long rec = u / kUnits;
  const int k = (int)(u - rec * kUnits);
  const int T = (int)(rec / npairs), p = (int)(rec - (long long)T * npairs);
  uint32_t w[4] = {0, 0, 0, 0};
  if (k < 4) {
    for (int e = 0; e < 4; ++e) {
      const int row = T * kTileRows + 4 * k + e;
      if (row >= out) continue;
      uint32_t v = 0;
      for (int h = 0; h < 2; ++h) {
        const int blk = 2 * p + h;
        if (blk >= nb) continue;
        const uint8_t *s = raw + ((size_t)row * nb + blk) * kQ8Block;
        v |= (uint32_t)(s[0] | (s[1] << 8)) << (16 * h);
      }
      w[e] = v;
    }
  } else {
    const int l = k - 4, g = l >> 4, r = l & 15;
    const int row = T * kTileRows + r;
    if (row < out) {
      for (int h = 0; h < 2; ++h) {
        const int blk = 2 * p + h;
        if (blk >= nb) continue;
        const uint8_t *s = raw + ((size_t)row * nb + blk) * kQ8Block + 2 + 8 * g;
        // 34-byte blocks are only 2-byte aligned: assemble the 8 code bytes bytewise.
        uint32_t lo = 0, hi = 0;
        for (int i = 0; i < 4; ++i) {
          lo |= (uint32_t)s[i] << (8 * i);
          hi |= (uint32_t)s[4 + i] << (8 * i);
        }
        w[2 * h] = lo;
        w[2 * h + 1] = hi;
      }
    }
  }
  reinterpret_cast<uint4 *>(dst)[u] = make_uint4(w[0], w[1], w[2], w[3]);
}

__global__ void q8_unpack_kernel(uint8_t *__restrict__ raw, const uint8_t *__restrict__ src,
                                 int out, int nb, int npairs, long long units) {
  const long long u = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (u >= units) return;
  const long long rec = u / kUnits;
  const int k = (int)(u - rec * kUnits);
  const int T = (int)(rec / npairs), p = (int)(rec - (long long)T * npairs);
  const uint4 v4 = reinterpret_cast<const uint4 *>(src)[u];
  const uint32_t w[4] = {v4.x, v4.y, v4.z, v4.w};
  if (k < 4) {
    for (int e = 0; e < 4; ++e) {
      const int row = T * kTileRows + 4 * k + e;
      if (row >= out) continue;
      for (int h = 0; h < 2; ++h) {
        const int blk = 2 * p + h;
        if (blk >= nb) continue;
        uint8_t *s = raw + ((size_t)row * nb + blk) * kQ8Block;
        s[0] = (uint8_t)(w[e] >> (16 * h));
        s[1] = (uint8_t)(w[e] >> (16 * h + 8));
      }
    }
  } else {
    const int l = k - 4, g = l >> 4, r = l & 15;
    const int row = T * kTileRows + r;
    if (row >= out) return;
    for (int h = 0; h < 2; ++h) {
      const int blk = 2 * p + h;
      if (blk >= nb) continue;
      uint8_t *s = raw + ((size_t)row * nb + blk) * kQ8Block + 2 + 8 * g;
      for (int i = 0; i < 4; ++i) {
        s[i] = (uint8_t)(w[2 * h] >> (8 * i));
        s[4 + i] = (uint8_t)(w[2 * h + 1] >> (8 * i));
      }
    }
  }
}

__device__ __forceinline__ float f16_bits_to_f32_exact(uint32_t h) {
  const uint32_t sign = (h & 0x8000u) << 16, exp = (h >> 10) & 0x1fu;
  uint32_t frac = h & 0x3ffu, bits;
  if (exp == 0) {
    if (frac == 0) {
      bits = sign;
    } else {
      const int sh = __clz(frac) - 21;
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

// One thread per (row, block): w = f32(int8(code)) * d (q8_0DequantBlock).
__global__ void q8_dequant_kernel(float *__restrict__ dw, const uint8_t *__restrict__ src,
                                  int out, int nb, int npairs) {
  const long long it = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (it >= (long long)out * nb) return;
  const int row = (int)(it / nb), blk = (int)(it - (long long)row * nb);
  const int T = row / kTileRows, r = row % kTileRows, p = blk >> 1, h = blk & 1;
  const uint8_t *rec = src + ((size_t)T * npairs + p) * kQ8Record;
  const uint8_t *hd = rec + 4 * r + 2 * h;
  const float d = f16_bits_to_f32_exact(hd[0] | (hd[1] << 8));
  float *o = dw + (size_t)row * nb * 32 + 32 * blk;
  for (int l = 0; l < 32; ++l) {
    const int g = l >> 3, i = l & 7;
    const int8_t code = (int8_t)rec[kQ8Hdr + 16 * (16 * g + r) + 8 * h + i];
    o[l] = __fmul_rn((float)code, d);
  }
}

__device__ __forceinline__ uint32_t b02(uint32_t q) { return (q & 0x00FF00FFu) | 0x64006400u; }

// PF: records each wave keeps in flight (8 when its K part is long enough, else 2: a short part
// would fill the ring with repeats of its last record).
template <int M, bool LX, int PF>
__global__ __launch_bounds__((LX && M <= 8) ? 1024 : 512) void q8_gemv_kernel(
    const uint8_t *__restrict__ W, const float *__restrict__ X, const uint4 *__restrict__ xg,
    float *__restrict__ Y, int N, int K, int npairs, int ntiles, int TW, int KW) {
  constexpr int R2 = 2 * M, NSET = (R2 + 15) / 16, J = M < 2 ? M : 2;
  extern __shared__ __align__(16) unsigned char smem[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane >> 4, r = lane & 15;
  const int tile = wave / KW, part = wave - tile * KW;
  const int T = blockIdx.x * TW + tile;
  const bool tvalid = T < ntiles;
  const int p0 = (int)((long long)part * npairs / KW);
  const int p1 = (int)((long long)(part + 1) * npairs / KW);
  const int ns = 2 * npairs, nsv = K / 32;  // staged slices (a padded last block stays zero)
  const uint8_t *base = W + (size_t)(tvalid ? T : 0) * npairs * kQ8Record;
  const uint4 *A;
  const float2 *Ex;
  if (LX) {
    A = reinterpret_cast<const uint4 *>(smem);
    Ex = reinterpret_cast<const float2 *>(smem + xop_a_bytes(M, ns));
  } else {
    A = xg;
    Ex = reinterpret_cast<const float2 *>(reinterpret_cast<const unsigned char *>(xg) +
                                          xop_a_bytes(M, ns));
  }
  float *red = reinterpret_cast<float *>(smem + (LX ? xop_bytes(M, ns) : 0));

  // The activations are staged first (vector loads complete in issue order per CU: behind a
  // burst of records they would land only once the burst had), then each wave keeps PF records
  // (two loads per lane each) in flight.
  if (LX) {
    stage_x<M>(X, K, 0, ns, nsv, reinterpret_cast<uint4 *>(smem),
               reinterpret_cast<float2 *>(smem + xop_a_bytes(M, ns)), threadIdx.x, blockDim.x);
    __syncthreads();
  }
  uint32_t hdr[PF];
  uint4 qr[PF];
  auto load = [&](int p, int u) {
    const uint8_t *rec = base + (size_t)p * kQ8Record;
    hdr[u] = ld_stream32(rec + 4 * r);
    qr[u] = ld_stream(rec + kQ8Hdr + 16 * lane);
  };
  if (p0 < p1)  // uniform; a part shorter than PF repeats its last record (never used)
#pragma unroll
    for (int u = 0; u < PF; ++u) load(min(p0 + u, p1 - 1), u);

  float acc[NSET][J];
#pragma unroll
  for (int k = 0; k < NSET; ++k)
#pragma unroll
    for (int jj = 0; jj < J; ++jj) acc[k][jj] = 0.f;

  for (int pp = p0; pp < p1; pp += PF)
#pragma unroll
  for (int u = 0; u < PF; ++u) {
    const int p = pp + u;
    if (p >= p1) break;
    // This slot's two loads are older than the other slots': the wait leaves those in flight.
    __builtin_amdgcn_s_waitcnt(0x0F70 | (2 * (PF - 1)));
    const uint32_t hc = hdr[u];
    const uint4 qc = qr[u];
    load(min(p + PF, p1 - 1), u);  // unconditional (a repeat at the end is never used): exact waits
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int sl = 2 * p + h;
      const uint32_t x0 = (h ? qc.z : qc.x) ^ 0x80808080u;
      const uint32_t x1 = (h ? qc.w : qc.y) ^ 0x80808080u;
      const f16x8 bw =
          __builtin_bit_cast(f16x8, u32x4{b02(x0), b02(x0 >> 8), b02(x1), b02(x1 >> 8)});
      const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)(hc >> (16 * h)));
      const bool sv = LX || sl < nsv;
#pragma unroll
      for (int k = 0; k < NSET; ++k) {
        // Unconditional loads at clamped indices, the unused values zeroed after: a load under
        // a lane test made the compiler wait for every load in flight after it.
        const int rho = r + 16 * k;
        const bool have = rho < R2 && (LX || sl < nsv);
        const f16x8 araw = __builtin_bit_cast(f16x8, A[(sl * 4 + g) * R2 + min(rho, R2 - 1)]);
        const f16x8 a = have ? araw : f16x8{};
        const f32x4 z = {0.f, 0.f, 0.f, 0.f};
        const f32x4 dd = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bw, z, 0, 0, 0);
#pragma unroll
        for (int jj = 0; jj < J; ++jj) {
          const int t = 8 * k + 2 * g + jj;
          const float2 seraw = Ex[(sl >> 3) * M * 8 + min(t, M - 1) * 8 + (sl & 7)];
          const float2 se = (t < M && sv) ? seraw : make_float2(0.f, 0.f);
          acc[k][jj] = fmaf(d * se.y, fmaf(-1152.f, se.x, dd[2 * jj] + dd[2 * jj + 1]), acc[k][jj]);
        }
      }
    }
  }

  float vals[NSET * J];
#pragma unroll
  for (int k = 0; k < NSET; ++k)
#pragma unroll
    for (int jj = 0; jj < J; ++jj) vals[k * J + jj] = acc[k][jj];
  wg_reduce<NSET * J>(red, tile, part, KW, lane, vals);
  const int row = T * 16 + r;
  if (part != 0 || !tvalid || row >= N) return;
#pragma unroll
  for (int k = 0; k < NSET; ++k)
#pragma unroll
    for (int jj = 0; jj < J; ++jj) {
      const int t = 8 * k + 2 * g + jj;
      if (t < M) Y[(size_t)t * N + row] = vals[k * J + jj];
    }
}

// Global-path operand writer: one thread per (slice, token); slices >= nsv are zero.
template <int M>
__global__ void q8_xprep_kernel(const float *__restrict__ X, int K, int ns, int nsv,
                                uint4 *__restrict__ A) {
  const int id = blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= ns * M) return;
  const int t = id / ns, sl = id - t * ns;
  float2 *E = reinterpret_cast<float2 *>(reinterpret_cast<unsigned char *>(A) + xop_a_bytes(M, ns));
  split_slice<M>(X + (size_t)t * K + 32 * (sl < nsv ? sl : 0), sl < nsv, sl, t, A, E);
}

template <int M>
bool q8_lds_x(int K) {
  constexpr int VALS = ((2 * M + 15) / 16) * (M < 2 ? M : 2);
  const size_t stage = xop_bytes(M, 2 * q8_groups(K));
  return !tuning().gemv_globalx && stage + (size_t)16 * 64 * VALS * 4 <= (size_t)lds_limit();
}

template <int M>
int launch_q8(const uint8_t *W, const float *X, float *Y, int N, int K) {
  const int npairs = q8_groups(K), ntiles = q4k_tiles(N), ns = 2 * npairs;
  constexpr int VALS = ((2 * M + 15) / 16) * (M < 2 ? M : 2);
  const size_t stage = xop_bytes(M, ns);
  const bool lds_x = q8_lds_x<M>(K);
  const int max_waves = (lds_x && M <= 8) ? 16 : 8;
  int TW = tuning().q8_tw, KW = tuning().q8_kw;
  const int cus = cu_count() > 0 ? cu_count() : 256;
  if (KW <= 0 && TW <= 0 && M == 1 && ntiles <= cus) {
    // Up to one tile per CU: one tile per workgroup, split over as many waves as leave each at
    // least one block pair (1536 x 576, 96 tiles: 1 x 8 waves 4.3 us per launch in a graph of
    // 300, 1 x 4 4.5, 4 tiles x 4 waves 5.0).
    TW = 1;
    KW = 1;
    while (2 * KW <= max_waves && npairs >= 2 * KW) KW *= 2;
  }
  if (KW <= 0) {
    const int want_waves = 8 * cus;
    KW = 1;
    while (2 * KW <= max_waves && ntiles * KW < want_waves && npairs / (2 * KW) >= 2) KW *= 2;
  }
  if (KW > npairs) KW = npairs;
  if (KW > max_waves) KW = max_waves;
  if (TW <= 0) TW = max_waves / KW > 4 ? 4 : max_waves / KW;
  if (TW < 1) TW = 1;
  while (TW * KW > max_waves) TW--;
  const int grid = ceil_div(ntiles, TW), threads = 64 * TW * KW;
  const size_t redB = KW > 1 ? (size_t)TW * KW * 64 * VALS * 4 : 0;
  if (lds_x) {
    // Measured (us, ring of 8 / ring of 1 before): 18944 x 3584 one token 21.6 / 23.2, 3584 x
    // 18944 four tokens 53.1 / 57.1; a 1536 x 576 matrix (about two records per wave) is
    // faster with the short ring.
    if (npairs >= 8 * KW)
      q8_gemv_kernel<M, true, 8><<<grid, threads, stage + redB, stream()>>>(W, X, nullptr, Y, N, K,
                                                                            npairs, ntiles, TW, KW);
    else
      q8_gemv_kernel<M, true, 2><<<grid, threads, stage + redB, stream()>>>(W, X, nullptr, Y, N, K,
                                                                            npairs, ntiles, TW, KW);
    FHIP_CHECK_LAUNCH("q8_gemv_kernel<lds>");
    return FHIP_OK;
  }
  void *xop = workspace(stage);
  if (!xop) return FHIP_ENOMEM;
  if (int rc = check_disjoint("q8_0_gemv", X, (size_t)M * K * 4, xop, stage)) return rc;
  q8_xprep_kernel<M><<<ceil_div(ns * M, 128), 128, 0, stream()>>>(X, K, ns, K / 32,
                                                                   (uint4 *)xop);
  FHIP_CHECK_LAUNCH("q8_xprep_kernel");
  q8_gemv_kernel<M, false, 2><<<grid, threads, redB, stream()>>>(W, X, (const uint4 *)xop, Y, N,
                                                                 K, npairs, ntiles, TW, KW);
  FHIP_CHECK_LAUNCH("q8_gemv_kernel<global>");
  return FHIP_OK;
}

int check_q8_shape(const char *who, int out, int in) {
  if (out <= 0 || in <= 0 || in % 32 != 0)
    return fail(FHIP_EINVAL, "%s: need out > 0 and in a positive multiple of 32 (out=%d in=%d)",
                who, out, in);
  return FHIP_OK;
}

}  // namespace

int q8_0_gemv(const void *Wv, const float *X, float *Y, int N, int K, int M) {
  const uint8_t *W = (const uint8_t *)Wv;
#define FHIP_Q8_CASE(m) \
  case m: return launch_q8<m>(W, X, Y, N, K);
  switch (M) {
    FHIP_Q8_CASE(1) FHIP_Q8_CASE(2) FHIP_Q8_CASE(3) FHIP_Q8_CASE(4)
    FHIP_Q8_CASE(5) FHIP_Q8_CASE(6) FHIP_Q8_CASE(7) FHIP_Q8_CASE(8)
    FHIP_Q8_CASE(9) FHIP_Q8_CASE(10) FHIP_Q8_CASE(11) FHIP_Q8_CASE(12)
    FHIP_Q8_CASE(13) FHIP_Q8_CASE(14) FHIP_Q8_CASE(15) FHIP_Q8_CASE(16)
  }
#undef FHIP_Q8_CASE
  return fail(FHIP_EINVAL, "q8_0_gemv: M=%d outside 1..16", M);
}

}  // namespace fhip

using namespace fhip;

extern "C" {

size_t fhip_q8_0_packed_bytes(int out, int in) {
  if (out <= 0 || in <= 0 || in % 32) return 0;
  return q8_packed_bytes(out, in);
}

int fhip_q8_0_repack(void *dPacked, const uint8_t *dRaw, int out, int in) {
  clear_error();
  if (int rc = check_q8_shape("fhip_q8_0_repack", out, in)) return rc;
  if (!dPacked || !dRaw) return fail(FHIP_EINVAL, "fhip_q8_0_repack: null pointer");
  const int nb = in / 32, npairs = q8_groups(in);
  const long long units = (long long)q4k_tiles(out) * npairs * kUnits;
  untag_range(dPacked, q8_packed_bytes(out, in));
  q8_repack_kernel<<<(unsigned)((units + 255) / 256), 256, 0, stream()>>>(
      (uint8_t *)dPacked, dRaw, out, nb, npairs, units);
  FHIP_CHECK_LAUNCH("q8_repack_kernel");
  tag_weight(dPacked, q8_packed_bytes(out, in), kWeightQ8_0, out, in);
  return FHIP_OK;
}

int fhip_q8_0_unpack(uint8_t *dRaw, const void *dPacked, int out, int in) {
  clear_error();
  if (int rc = check_q8_shape("fhip_q8_0_unpack", out, in)) return rc;
  if (!dPacked || !dRaw) return fail(FHIP_EINVAL, "fhip_q8_0_unpack: null pointer");
  if (int rc = check_weight("fhip_q8_0_unpack", dPacked, kWeightQ8_0, out, in)) return rc;
  untag_range(dRaw, (size_t)out * (in / 32) * kQ8Block);
  const int nb = in / 32, npairs = q8_groups(in);
  const long long units = (long long)q4k_tiles(out) * npairs * kUnits;
  q8_unpack_kernel<<<(unsigned)((units + 255) / 256), 256, 0, stream()>>>(
      dRaw, (const uint8_t *)dPacked, out, nb, npairs, units);
  FHIP_CHECK_LAUNCH("q8_unpack_kernel");
  return FHIP_OK;
}

int fhip_q8_0_dequant_f32(float *dW, const void *dPacked, int out, int in) {
  clear_error();
  if (int rc = check_q8_shape("fhip_q8_0_dequant_f32", out, in)) return rc;
  if (!dPacked || !dW) return fail(FHIP_EINVAL, "fhip_q8_0_dequant_f32: null pointer");
  if (int rc = check_weight("fhip_q8_0_dequant_f32", dPacked, kWeightQ8_0, out, in)) return rc;
  untag_range(dW, (size_t)out * in * 4);
  const int nb = in / 32, npairs = q8_groups(in);
  const long long items = (long long)out * nb;
  q8_dequant_kernel<<<(unsigned)((items + 255) / 256), 256, 0, stream()>>>(
      dW, (const uint8_t *)dPacked, out, nb, npairs);
  FHIP_CHECK_LAUNCH("q8_dequant_kernel");
  return FHIP_OK;
}

void *fhip_q8_0_upload(const uint8_t *hRaw, int out, int in) {
  clear_error();
  if (check_q8_shape("fhip_q8_0_upload", out, in)) return nullptr;
  if (!hRaw) { fail(FHIP_EINVAL, "fhip_q8_0_upload: null host pointer"); return nullptr; }
  const size_t rawBytes = (size_t)out * (in / 32) * kQ8Block;
  void *packed = fhip_malloc(q8_packed_bytes(out, in));
  if (!packed) return nullptr;
  void *staging = fhip_malloc(rawBytes);
  if (!staging) { fhip_free(packed); return nullptr; }
  int rc = fhip_h2d(staging, hRaw, rawBytes);
  if (rc == FHIP_OK) rc = fhip_q8_0_repack(packed, (const uint8_t *)staging, out, in);
  if (rc == FHIP_OK) {
    hipError_t e = hipStreamSynchronize(stream());
    if (e != hipSuccess) rc = hip_fail(e, "fhip_q8_0_upload: hipStreamSynchronize");
  }
  fhip_free(staging);
  if (rc != FHIP_OK) { fhip_free(packed); return nullptr; }
  return packed;
}

int fhip_q8_0_matmul_f32(const void *dPacked, const float *dX, float *dY, int out, int in,
                         int P) {
  clear_error();
  if (int rc = check_q8_shape("fhip_q8_0_matmul_f32", out, in)) return rc;
  if (P < 0) return fail(FHIP_EINVAL, "fhip_q8_0_matmul_f32: P=%d < 0", P);
  if (P == 0) return FHIP_OK;
  if (!dPacked || !dX || !dY) return fail(FHIP_EINVAL, "fhip_q8_0_matmul_f32: null pointer");
  if (((uintptr_t)dX & 15) || ((uintptr_t)dPacked & 15))
    return fail(FHIP_EINVAL, "fhip_q8_0_matmul_f32: dX and dPacked must be 16-byte aligned");
  if (int rc = check_weight("fhip_q8_0_matmul_f32", dPacked, kWeightQ8_0, out, in)) return rc;
  untag_range(dY, (size_t)P * out * 4);
  // The raw-GGUF Q8_0 path is a decode GEMV in the reference; longer batches run in 16-token
  // slices of the same kernel.
  for (int t0 = 0; t0 < P; t0 += 16) {
    const int m = P - t0 < 16 ? P - t0 : 16;
    if (int rc = q8_0_gemv(dPacked, dX + (size_t)t0 * in, dY + (size_t)t0 * out, out, in, m))
      return rc;
  }
  return FHIP_OK;
}

}  // extern "C"
