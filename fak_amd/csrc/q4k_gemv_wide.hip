// q4k_gemv_wide.hip — small-M Q4_K matmul with f16 activation operands: used for 5..16 tokens
// (speculative verify); 1..4 tokens go to the int8 kernel of q4k_gemv.hip.
//
// Computes Y[t][o] = sum_k W[o][k] * X[t][k] with W the dequantized Q4_K weight
// (w = d*sc*n - dmin*m per 32-weight sub-block, internal/model/quant_q4k.go:90-111) without
// ever materialising w. Per sub-block s of row o and token t the sum factors as
//   sum_k w x = d*sc_s * sum_k n_k x_k  -  dmin*m_s * S_s,      S_s = sum_k x_k
// and the inner integer-weight dot runs on a 16x16x32 f16 MFMA:
//   * weight operand: the 4-bit codes themselves, exact in f16. A nibble pair becomes two f16
//     values with one and-or: (q & 0x000F000F) | 0x64006400 = (1024 + n0, 1024 + n2) (the high
//     nibbles, masked in place, give 1024 + 16 n). The 1024 * S_s this adds is subtracted after
//     the MFMA.
//   * activation operand: X split into f16 hi and lo rows (gemv_common.hpp), so each token uses
//     two of the MFMA's 16 rows and the products carry ~22 bits of the activation.
// After each MFMA the f32 result is scaled per (row, sub-block) on the VALU.
//
// Work split. A workgroup owns TW 16-row tiles over the whole K; each tile is worked by KW
// waves, each on a contiguous part of the super-blocks, and the KW partials are summed through
// LDS in part order (deterministic, no cross-workgroup traffic). Every wave streams its tiled
// weight records (tiled.hpp) exactly once with three coalesced 16-byte loads per lane per
// 2304-byte record and keeps the next record in flight while it computes the current one.
//
// Activation operands: with LX the workgroup stages them for all of K into LDS itself (decode:
// one launch per matmul); otherwise a separate gemv_xprep_kernel writes them to global memory
// (used when M*K is too large for LDS) and the waves prefetch them with the weights.
#include "gemv_common.hpp"

namespace fhip {
namespace {

template <int M, bool LX>
__global__ __launch_bounds__((LX && M == 1) ? 1024 : 512) void q4k_gemv_kernel(
    const uint8_t *__restrict__ W, const float *__restrict__ X, const uint4 *__restrict__ xg,
    float *__restrict__ Y, int N, int K, int nblk, int ntiles, int TW, int KW) {
  constexpr int R2 = 2 * M;             // operand rows (hi, lo per token)
  constexpr int NSET = (R2 + 15) / 16;  // MFMA row sets
  constexpr int J = M < 2 ? M : 2;      // tokens per lane group per set
  extern __shared__ __align__(16) unsigned char smem[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane >> 4, r = lane & 15;
  const int tile = wave / KW, part = wave - tile * KW;
  const int T = blockIdx.x * TW + tile;
  const bool tvalid = T < ntiles;
  const int b0 = (int)((long long)part * nblk / KW);
  const int b1 = (int)((long long)(part + 1) * nblk / KW);
  const int ns = 8 * nblk;
  const uint8_t *base = W + (size_t)(tvalid ? T : 0) * nblk * kQ4kRecord;

  // Activation operands. LDS path: every wave stages its own K part into a private region
  // (slices 8*b0 .. 8*b1 of size `cap` super-blocks), so no workgroup barrier precedes the
  // first MFMA. Global path: one shared buffer for all of K.
  const int cap = (nblk + KW - 1) / KW;  // super-blocks per part, rounded up
  const uint4 *A;
  const float *Sx;
  int sbase;  // super-block index of A/Sx slice 0
  if (LX) {
    unsigned char *mine = smem + (size_t)wave * xop_bytes(M, 8 * cap);
    A = reinterpret_cast<const uint4 *>(mine);
    Sx = reinterpret_cast<const float *>(mine + xop_a_bytes(M, 8 * cap));
    sbase = b0;
  } else {
    A = xg;
    Sx = reinterpret_cast<const float *>(reinterpret_cast<const unsigned char *>(xg) +
                                         xop_a_bytes(M, ns));
    sbase = 0;
  }
  float *red = reinterpret_cast<float *>(smem + (LX ? (size_t)TW * KW * xop_bytes(M, 8 * cap) : 0));

  // Operands of one super-block: the weight record and (global path) the activation operands.
  struct Ops {
    uint4 h, qa, qb;
    f16x8 a[LX ? 1 : 8][NSET];
    float s[LX ? 1 : NSET][J][8];
  };
  auto load = [&](int b, Ops &o) {
    const uint8_t *rec = base + (size_t)b * kQ4kRecord;
    o.h = *reinterpret_cast<const uint4 *>(rec + 16 * r);
    o.qa = *reinterpret_cast<const uint4 *>(rec + kQ4kHdr + 16 * lane);
    o.qb = *reinterpret_cast<const uint4 *>(rec + kQ4kHdr + 1024 + 16 * lane);
    if (!LX) {
#pragma unroll
      for (int s = 0; s < 8; ++s)
#pragma unroll
        for (int k = 0; k < NSET; ++k) {
          const int rho = r + 16 * k, rr = rho < R2 ? rho : rho % R2;
          o.a[s][k] = __builtin_bit_cast(f16x8, A[((8 * (b - sbase) + s) * 4 + g) * R2 + rr]);
        }
#pragma unroll
      for (int k = 0; k < NSET; ++k)
#pragma unroll
        for (int jj = 0; jj < J; ++jj) {
          const int t = 8 * k + 2 * g + jj, tt = t < M ? t : 0;
          const float4 s0 = *reinterpret_cast<const float4 *>(Sx + ((b - sbase) * M + tt) * 8);
          const float4 s1 = *reinterpret_cast<const float4 *>(Sx + ((b - sbase) * M + tt) * 8 + 4);
          o.s[k][jj][0] = s0.x; o.s[k][jj][1] = s0.y; o.s[k][jj][2] = s0.z; o.s[k][jj][3] = s0.w;
          o.s[k][jj][4] = s1.x; o.s[k][jj][5] = s1.y; o.s[k][jj][6] = s1.z; o.s[k][jj][7] = s1.w;
        }
    }
  };

  // PF records per wave in flight: a ring of register sets; a set is refilled with the record
  // PF ahead as soon as its own record has been consumed.
  constexpr int PF = LX ? 4 : (NSET == 1 ? 2 : 1);
  Ops ring[PF];
#pragma unroll
  for (int u = 0; u < PF; ++u)
    if (b0 + u < b1) load(b0 + u, ring[u]);
  if (LX) {
    stage_x<M>(X, K, 8 * b0, 8 * (b1 - b0), ns, const_cast<uint4 *>(A), const_cast<float *>(Sx),
               lane, 64);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
  const uint32_t kLoMask = in_reg(0x000F000Fu), kHiMask = in_reg(0x00F000F0u);
  const uint32_t kMagic = in_reg(0x64006400u), k3F = in_reg(0x3F3F3F3Fu);
  const uint32_t k0F = in_reg(0x0F0F0F0Fu), k30 = in_reg(0x30303030u);

  float acc[NSET][J];
#pragma unroll
  for (int k = 0; k < NSET; ++k)
#pragma unroll
    for (int jj = 0; jj < J; ++jj) acc[k][jj] = 0.f;

  for (int bb = b0; bb < b1; bb += PF) {
#pragma unroll
    for (int u = 0; u < PF; ++u) {
      const int b = bb + u;
      if (b >= b1) break;
      Ops &cur = ring[u];

      // Per-token sub-block sums of this super-block (rows of tokens >= M are never stored,
      // so their lanes may use any finite value).
      float S[NSET][J][8];
#pragma unroll
      for (int k = 0; k < NSET; ++k)
#pragma unroll
        for (int jj = 0; jj < J; ++jj) {
          if (LX) {
            const int t = 8 * k + 2 * g + jj, tt = t < M ? t : 0;
            const float4 s0 = *reinterpret_cast<const float4 *>(Sx + ((b - sbase) * M + tt) * 8);
            const float4 s1 = *reinterpret_cast<const float4 *>(Sx + ((b - sbase) * M + tt) * 8 + 4);
            S[k][jj][0] = s0.x; S[k][jj][1] = s0.y; S[k][jj][2] = s0.z; S[k][jj][3] = s0.w;
            S[k][jj][4] = s1.x; S[k][jj][5] = s1.y; S[k][jj][6] = s1.z; S[k][jj][7] = s1.w;
          } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) S[k][jj][i] = cur.s[k][jj][i];
          }
        }

      // d, dmin and the 8 six-bit (scale, min) pairs (GetScaleMinK4 geometry, byte-parallel):
      // four packed bytes per word, then one v_cvt_f32_ubyteN per value.
      const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)(cur.h.x & 0xffffu));
      const float dm = (float)__builtin_bit_cast(_Float16, (uint16_t)(cur.h.x >> 16));
      const uint32_t scl = in_reg(cur.h.y & k3F), mnl = in_reg(cur.h.z & k3F);
      const uint32_t sch = in_reg((cur.h.w & k0F) | ((cur.h.y >> 2) & k30));
      const uint32_t mnh = in_reg(((cur.h.w >> 4) & k0F) | ((cur.h.z >> 2) & k30));
      const uint32_t q[8] = {cur.qa.x, cur.qa.y, cur.qa.z, cur.qa.w,
                             cur.qb.x, cur.qb.y, cur.qb.z, cur.qb.w};
      const uint32_t scw[2] = {scl, sch}, mnw[2] = {mnl, mnh};
      // Operand rows >= 2M only feed output rows that are never stored, so every lane loads a
      // valid (finite) row instead of masking: no exec-mask juggling, no zero fills.
      f16x8 aop[8][NSET];
      if (LX) {
#pragma unroll
        for (int sidx = 0; sidx < 8; ++sidx)
#pragma unroll
          for (int k = 0; k < NSET; ++k) {
            const int rho = r + 16 * k, rr = rho < R2 ? rho : rho % R2;
            aop[sidx][k] = __builtin_bit_cast(f16x8, A[((8 * (b - sbase) + sidx) * 4 + g) * R2 + rr]);
          }
      }

      float aL[NSET][J], aH[NSET][J], V[NSET][J];
#pragma unroll
      for (int k = 0; k < NSET; ++k)
#pragma unroll
        for (int jj = 0; jj < J; ++jj) aL[k][jj] = aH[k][jj] = V[k][jj] = 0.f;

      // Phase 1: all 8 MFMAs of the record back to back (independent), so their latency
      // overlaps; phase 2 scales and accumulates the results on the VALU.
      f32x4 dres[4][2][NSET];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const uint32_t x0 = q[2 * c], x1 = q[2 * c + 1];
        const uint32_t y0 = x0 >> 8, y1 = x1 >> 8;
        const f16x8 bl8 = __builtin_bit_cast(
            f16x8, u32x4{(x0 & kLoMask) | kMagic, (y0 & kLoMask) | kMagic,
                         (x1 & kLoMask) | kMagic, (y1 & kLoMask) | kMagic});
        const f16x8 bh8 = __builtin_bit_cast(
            f16x8, u32x4{(x0 & kHiMask) | kMagic, (y0 & kHiMask) | kMagic,
                         (x1 & kHiMask) | kMagic, (y1 & kHiMask) | kMagic});
#pragma unroll
        for (int k = 0; k < NSET; ++k) {
          const f16x8 al = LX ? aop[2 * c][k] : cur.a[2 * c][k];
          const f16x8 ah = LX ? aop[2 * c + 1][k] : cur.a[2 * c + 1][k];
          const f32x4 z = {0.f, 0.f, 0.f, 0.f};
          dres[c][0][k] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bl8, z, 0, 0, 0);
          dres[c][1][k] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bh8, z, 0, 0, 0);
        }
      }
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int sl = 2 * c, sh = 2 * c + 1;  // sub-blocks of the low / high nibbles of chunk c
        const int bsel = (c & 1) * 2;  // byte of the packed word holding sc[sl]; sc[sh] is next
        const uint32_t sw = scw[c >> 1], mw = mnw[c >> 1];
        const float scL = (float)((sw >> (8 * bsel)) & 0xffu);
        const float scH = (float)((sw >> (8 * bsel + 8)) & 0xffu);
        const float mL = (float)((mw >> (8 * bsel)) & 0xffu);
        const float mH = (float)((mw >> (8 * bsel + 8)) & 0xffu);
#pragma unroll
        for (int k = 0; k < NSET; ++k) {
          const f32x4 dl = dres[c][0][k], dh = dres[c][1][k];
#pragma unroll
          for (int jj = 0; jj < J; ++jj) {
            const float Sl = S[k][jj][sl], Sh = S[k][jj][sh];
            const float tl = dl[2 * jj] + dl[2 * jj + 1];
            const float th = dh[2 * jj] + dh[2 * jj + 1];
            aL[k][jj] = fmaf(scL, fmaf(-1024.f, Sl, tl), aL[k][jj]);
            aH[k][jj] = fmaf(scH, fmaf(-1024.f, Sh, th), aH[k][jj]);
            V[k][jj] = fmaf(mL, Sl, fmaf(mH, Sh, V[k][jj]));
          }
        }
      }
#pragma unroll
      for (int k = 0; k < NSET; ++k)
#pragma unroll
        for (int jj = 0; jj < J; ++jj)
          acc[k][jj] =
              fmaf(d, fmaf(0.0625f, aH[k][jj], aL[k][jj]), fmaf(-dm, V[k][jj], acc[k][jj]));
      if (b + PF < b1) load(b + PF, cur);
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

// One thread per (slice, token) into the global operand buffer; slices >= nsv are zero.
template <int M>
__global__ void gemv_xprep_kernel(const float *__restrict__ X, int K, int ns, int nsv,
                                  uint4 *__restrict__ A) {
  const int id = blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= ns * M) return;
  const int t = id / ns, sl = id - t * ns;
  float *S = reinterpret_cast<float *>(reinterpret_cast<unsigned char *>(A) + xop_a_bytes(M, ns));
  split_slice<M>(X + (size_t)t * K + 32 * (sl < nsv ? sl : 0), sl < nsv, sl, t, A, S);
}

template <int M>
int launch_xprep_m(const float *X, int K, int ns, void *xop) {
  const int n = ns * M, bs = 128;
  gemv_xprep_kernel<M><<<ceil_div(n, bs), bs, 0, stream()>>>(X, K, ns, K / 32, (uint4 *)xop);
  FHIP_CHECK_LAUNCH("gemv_xprep_kernel");
  return FHIP_OK;
}

// Pick the workgroup shape: TW tiles x KW waves per tile (<= 16 waves per workgroup), aiming at
// >= ~12 waves per CU in total. FAK_HIP_GEMV_TW / FAK_HIP_GEMV_KW override (tuning).
void gemv_shape(int ntiles, int nblk, int max_waves, int &TW, int &KW) {
  const int cus = cu_count() > 0 ? cu_count() : 256;
  TW = env_int("FAK_HIP_GEMV_TW");
  KW = env_int("FAK_HIP_GEMV_KW");
  if (KW <= 0) {
    const int want_waves = 6 * cus;  // measured best on the 7B FFN shapes (KW=2 up, KW=8 down)
    KW = 1;
    while (2 * KW <= max_waves && ntiles * KW < want_waves && nblk / (2 * KW) >= 2) KW *= 2;
  }
  if (KW > nblk) KW = nblk;
  if (KW > max_waves) KW = max_waves;
  if (TW <= 0) TW = 1;  // each wave stages its own K part: more tiles per WG would repeat it
  if (TW < 1) TW = 1;
  while (TW * KW > max_waves) TW--;
}

template <int M>
int launch_gemv(const uint8_t *W, const float *X, float *Y, int N, int K) {
  const int nblk = K / 256, ntiles = q4k_tiles(N), ns = K / 32;
  constexpr int VALS = ((2 * M + 15) / 16) * (M < 2 ? M : 2);
  const int max_waves = M == 1 ? 16 : 8;
  int TW, KW;
  gemv_shape(ntiles, nblk, max_waves, TW, KW);
  const int cap = ceil_div(nblk, KW);
  const size_t redB = KW > 1 ? (size_t)TW * KW * 64 * VALS * 4 : 0;
  const size_t ldsx = (size_t)TW * KW * xop_bytes(M, 8 * cap);
  const bool lds_x = !env_int("FAK_HIP_GEMV_GLOBALX") && ldsx + redB <= (size_t)lds_limit();
  if (!lds_x) gemv_shape(ntiles, nblk, 8, TW, KW);
  const int grid = ceil_div(ntiles, TW), threads = 64 * TW * KW;
  if (lds_x) {
    q4k_gemv_kernel<M, true><<<grid, threads, ldsx + redB, stream()>>>(W, X, nullptr, Y, N, K,
                                                                       nblk, ntiles, TW, KW);
    FHIP_CHECK_LAUNCH("q4k_gemv_kernel<lds>");
    return FHIP_OK;
  }
  const size_t redG = KW > 1 ? (size_t)TW * KW * 64 * VALS * 4 : 0;
  void *xop = workspace(xop_bytes(M, ns));
  if (!xop) return FHIP_ENOMEM;
  if (int rc = launch_xprep_m<M>(X, K, ns, xop)) return rc;
  q4k_gemv_kernel<M, false><<<grid, threads, redG, stream()>>>(W, X, (const uint4 *)xop, Y, N, K,
                                                               nblk, ntiles, TW, KW);
  FHIP_CHECK_LAUNCH("q4k_gemv_kernel<global>");
  return FHIP_OK;
}

}  // namespace

int launch_gemv_xprep(const float *X, int M, int K, int ns, void *xop) {
#define FHIP_XPREP_CASE(m) \
  case m: return launch_xprep_m<m>(X, K, ns, xop);
  switch (M) {
    FHIP_XPREP_CASE(1) FHIP_XPREP_CASE(2) FHIP_XPREP_CASE(3) FHIP_XPREP_CASE(4)
    FHIP_XPREP_CASE(5) FHIP_XPREP_CASE(6) FHIP_XPREP_CASE(7) FHIP_XPREP_CASE(8)
    FHIP_XPREP_CASE(9) FHIP_XPREP_CASE(10) FHIP_XPREP_CASE(11) FHIP_XPREP_CASE(12)
    FHIP_XPREP_CASE(13) FHIP_XPREP_CASE(14) FHIP_XPREP_CASE(15) FHIP_XPREP_CASE(16)
  }
#undef FHIP_XPREP_CASE
  return fail(FHIP_EINVAL, "gemv_xprep: M=%d outside 1..16", M);
}

int q4k_gemv_wide(const void *Wv, const float *X, float *Y, int N, int K, int M) {
  const uint8_t *W = (const uint8_t *)Wv;
#define FHIP_GEMV_CASE(m) \
  case m: return launch_gemv<m>(W, X, Y, N, K);
  switch (M) {
    FHIP_GEMV_CASE(1) FHIP_GEMV_CASE(2) FHIP_GEMV_CASE(3) FHIP_GEMV_CASE(4)
    FHIP_GEMV_CASE(5) FHIP_GEMV_CASE(6) FHIP_GEMV_CASE(7) FHIP_GEMV_CASE(8)
    FHIP_GEMV_CASE(9) FHIP_GEMV_CASE(10) FHIP_GEMV_CASE(11) FHIP_GEMV_CASE(12)
    FHIP_GEMV_CASE(13) FHIP_GEMV_CASE(14) FHIP_GEMV_CASE(15) FHIP_GEMV_CASE(16)
  }
#undef FHIP_GEMV_CASE
  return fail(FHIP_EINVAL, "q4k_gemv: M=%d outside 1..16", M);
}

}  // namespace fhip
