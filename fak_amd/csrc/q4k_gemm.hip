// q4k_gemm.hip — large-M (prefill) Q4_K matmul on 16x16x32 f16 MFMA.
//
// Y[t][o] = sum_k W[o][k] X[t][k], W dequantized from the tiled Q4_K records (tiled.hpp) and X
// pre-converted once to f16 MFMA operand tiles (xprep.hip). Each workgroup computes a tile of
// 16*TM tokens x 256 rows; wave w owns 4 consecutive 16-row tiles:
//   * weights go global -> registers -> f16 in registers, never through LDS: the lane's 16-byte
//     record part is already its MFMA operand. Dequant is w = d1*n - m1 evaluated in f16
//     (d1 = f16(d*sc), m1 = f16(dmin*m); the nibble becomes an exact f16 via the 0x6400
//     exponent trick) with one packed fma per pair of weights;
//   * activations go global -> registers -> LDS (double-buffered, one 64-wide K chunk per
//     stage) and are shared by the 4 waves;
//   * weight record parts are reloaded for the next super-block as soon as they are consumed,
//     and the next stage's activation tiles are in flight while the current stage's MFMAs run.
// The f16 weight and activation rounding bound the error at max|dY|/RMS(Y) ~ 2e-3 (< 1e-2).
#include "kernels.hpp"

namespace fhip {
namespace {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));

// Mask and magic constants held in registers (in_reg) so each (q & mask) | magic is one
// v_and_or_b32.
struct Magic {
  uint32_t lo, hi, byte02, magic;
};
__device__ __forceinline__ Magic magic_consts() {
  return Magic{in_reg(0x000F000Fu), in_reg(0x00F000F0u), in_reg(0x00FF00FFu), in_reg(0x64006400u)};
}
__device__ __forceinline__ h2 as_h2(uint32_t u) { return __builtin_bit_cast(h2, u); }
__device__ __forceinline__ uint32_t as_u(h2 v) { return __builtin_bit_cast(uint32_t, v); }

// Per-super-block scale pairs for one row: d1[s] = f16(d*sc_s) (odd s pre-divided by 16 to
// absorb the 16n of the in-place high-nibble mask) and m1[s] = f16(dmin*m_s).
struct RowScales {
  h2 d1e[2], d1o[2];  // (d1_0, d1_2), (d1_4, d1_6) ; (d1_1, d1_3)/16, (d1_5, d1_7)/16
  h2 m1e[2], m1o[2];
};

__device__ __forceinline__ RowScales row_scales(uint4 h, const Magic &K) {
  const h2 k1024 = {(_Float16)1024.f, (_Float16)1024.f};
  const _Float16 d = __builtin_bit_cast(_Float16, (uint16_t)(h.x & 0xffffu));
  const _Float16 dm = __builtin_bit_cast(_Float16, (uint16_t)(h.x >> 16));
  const h2 dd = {d, d}, mm = {dm, dm};
  const uint32_t scl = h.y & 0x3F3F3F3Fu, mnl = h.z & 0x3F3F3F3Fu;
  const uint32_t sch = (h.w & 0x0F0F0F0Fu) | ((h.y >> 2) & 0x30303030u);
  const uint32_t mnh = ((h.w >> 4) & 0x0F0F0F0Fu) | ((h.z >> 2) & 0x30303030u);
  const h2 k16 = {(_Float16)0.0625f, (_Float16)0.0625f};
  RowScales s;
  // (v & 0x00FF00FF) | 0x64006400 = (1024 + byte0, 1024 + byte2) exactly.
  s.d1e[0] = (as_h2((scl & K.byte02) | K.magic) - k1024) * dd;
  s.d1o[0] = (as_h2(((scl >> 8) & K.byte02) | K.magic) - k1024) * dd * k16;
  s.d1e[1] = (as_h2((sch & K.byte02) | K.magic) - k1024) * dd;
  s.d1o[1] = (as_h2(((sch >> 8) & K.byte02) | K.magic) - k1024) * dd * k16;
  s.m1e[0] = (as_h2((mnl & K.byte02) | K.magic) - k1024) * mm;
  s.m1o[0] = (as_h2(((mnl >> 8) & K.byte02) | K.magic) - k1024) * mm;
  s.m1e[1] = (as_h2((mnh & K.byte02) | K.magic) - k1024) * mm;
  s.m1o[1] = (as_h2(((mnh >> 8) & K.byte02) | K.magic) - k1024) * mm;
  return s;
}

// Dequantize chunk c (bytes 32c.. of the row's nibbles) of one row tile into the two f16 MFMA
// weight operands: sub-block 2c (low nibbles) and 2c+1 (high nibbles).
__device__ __forceinline__ void dequant_chunk(uint32_t x0, uint32_t x1, const RowScales &s, int c,
                                              const Magic &K, f16x8 &bl, f16x8 &bh) {
  auto lo02 = [&](uint32_t q) { return (q & K.lo) | K.magic; };
  auto hi02 = [&](uint32_t q) { return (q & K.hi) | K.magic; };
  const h2 k1024 = {(_Float16)1024.f, (_Float16)1024.f};
  const int p = c >> 1, hsel = c & 1;
  const h2 de = s.d1e[p], dodd = s.d1o[p], me = s.m1e[p], mo = s.m1o[p];
  const _Float16 dl = hsel ? de.y : de.x, dh = hsel ? dodd.y : dodd.x;
  const _Float16 ml = hsel ? me.y : me.x, mh = hsel ? mo.y : mo.x;
  const h2 DL = {dl, dl}, DH = {dh, dh}, ML = {-ml, -ml}, MH = {-mh, -mh};
  const uint32_t y0 = x0 >> 8, y1 = x1 >> 8;
  u32x4 l, hh;
  l[0] = as_u((as_h2(lo02(x0)) - k1024) * DL + ML);
  l[1] = as_u((as_h2(lo02(y0)) - k1024) * DL + ML);
  l[2] = as_u((as_h2(lo02(x1)) - k1024) * DL + ML);
  l[3] = as_u((as_h2(lo02(y1)) - k1024) * DL + ML);
  hh[0] = as_u((as_h2(hi02(x0)) - k1024) * DH + MH);
  hh[1] = as_u((as_h2(hi02(y0)) - k1024) * DH + MH);
  hh[2] = as_u((as_h2(hi02(x1)) - k1024) * DH + MH);
  hh[3] = as_u((as_h2(hi02(y1)) - k1024) * DH + MH);
  bl = __builtin_bit_cast(f16x8, l);
  bh = __builtin_bit_cast(f16x8, hh);
}

// Workgroup = 4 waves over TM 16-token tiles x 16 row tiles; wave w owns row tiles 4w..4w+3
// (its weights stay in its registers) and all four share the token tiles through LDS.
template <int TM, int R, int WPE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(WPE, WPE))) void
q4k_gemm_kernel(const uint8_t *__restrict__ W, const uint4 *__restrict__ xa,
                float *__restrict__ Y, int N, int M, int nblk, int ntiles, int MTG, int remap) {
  // R: row tiles per wave; the workgroup's 4 waves cover 4 R row tiles
  constexpr int AU = TM * 2 * 64;   // uint4 operand units per stage (TM tiles x 2 slices x 64)
  constexpr int APT = AU / 256;     // per thread
  __shared__ uint4 As[2][AU];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // Workgroups are dispatched round-robin over the 8 XCDs (each with its own L2). The remap
  // gives consecutive logical ids -- the token groups of one row group, which read the same
  // weights -- to one XCD, so its L2 serves the repeated weight reads.
  int wg = blockIdx.x;
  if (remap) wg = (wg & 7) * (gridDim.x >> 3) + (wg >> 3);
  const int mg = wg % MTG, ng = wg / MTG;
  const int nslices = nblk * 8;
  const int rt0 = ng * 4 * R + wave * R;
  const uint4 *xg = xa + (size_t)mg * TM * nslices * 64;  // this group's token tiles (padded)

  const Magic K = magic_consts();
  f32x4 acc[TM][R];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < R; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const uint8_t *rbase[R];
#pragma unroll
  for (int j = 0; j < R; ++j)
    rbase[j] = W + (size_t)(rt0 + j < ntiles ? rt0 + j : 0) * nblk * kQ4kRecord;

  // Stage st = chunk (64 K) st: token tile i, slice sl -> As[.][(2 i + sl) * 64 + l].
  auto load_a = [&](int st, uint4 (&regs)[APT]) {
#pragma unroll
    for (int k = 0; k < APT; ++k) {
      const int u = tid + 256 * k;
      const int i = u >> 7, sl = (u >> 6) & 1, l = u & 63;
      regs[k] = xg[((size_t)i * nslices + 2 * st + sl) * 64 + l];
    }
  };
  // Weight records: the header of the next super-block is loaded as soon as this one's scales
  // are decoded; each half of the nibbles (qa: chunks 0-1, qb: chunks 2-3) is reloaded for the
  // next super-block as soon as its second chunk is consumed, two chunks ahead of its use.
  auto load_h = [&](int b, uint4 (&h)[R]) {
#pragma unroll
    for (int j = 0; j < R; ++j)
      h[j] = *reinterpret_cast<const uint4 *>(rbase[j] + (size_t)b * kQ4kRecord + 16 * (lane & 15));
  };
  auto load_q = [&](int b, int part, uint4 (&q)[R]) {
#pragma unroll
    for (int j = 0; j < R; ++j)
      q[j] = *reinterpret_cast<const uint4 *>(rbase[j] + (size_t)b * kQ4kRecord + kQ4kHdr +
                                              1024 * part + 16 * lane);
  };

  uint4 areg[APT];
  uint4 h[R], qa[R], qb[R];
  load_h(0, h);
  load_q(0, 0, qa);
  load_q(0, 1, qb);
  load_a(0, areg);
#pragma unroll
  for (int k = 0; k < APT; ++k) As[0][tid + 256 * k] = areg[k];
  __syncthreads();

  const int nst = nblk * 4;
  for (int b = 0; b < nblk; ++b) {
    RowScales rs[R];
#pragma unroll
    for (int j = 0; j < R; ++j) rs[j] = row_scales(h[j], K);
    const bool more = b + 1 < nblk;
    if (more) load_h(b + 1, h);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int st = 4 * b + c, cur = c & 1;  // 4 stages per super-block: parity == c & 1
      if (st + 1 < nst) load_a(st + 1, areg);
      f16x8 bl[R], bh[R];
#pragma unroll
      for (int j = 0; j < R; ++j) {
        const uint4 q = c < 2 ? qa[j] : qb[j];
        const uint32_t x0 = (c & 1) ? q.z : q.x, x1 = (c & 1) ? q.w : q.y;
        dequant_chunk(x0, x1, rs[j], c, K, bl[j], bh[j]);
      }
      if (more && c == 1) load_q(b + 1, 0, qa);
      if (more && c == 3) load_q(b + 1, 1, qb);
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const f16x8 al = __builtin_bit_cast(f16x8, As[cur][(2 * i) * 64 + lane]);
        const f16x8 ah = __builtin_bit_cast(f16x8, As[cur][(2 * i + 1) * 64 + lane]);
#pragma unroll
        for (int j = 0; j < R; ++j) {
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bl[j], acc[i][j], 0, 0, 0);
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bh[j], acc[i][j], 0, 0, 0);
        }
      }
      if (st + 1 < nst) {
#pragma unroll
        for (int k = 0; k < APT; ++k) As[cur ^ 1][tid + 256 * k] = areg[k];
      }
      __syncthreads();
    }
  }

  const int g = lane >> 4, r = lane & 15;
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int tbase = 16 * (mg * TM + i) + 4 * g;
#pragma unroll
    for (int j = 0; j < R; ++j) {
      const int o = 16 * (rt0 + j) + r;
      if (rt0 + j >= ntiles || o >= N) continue;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int t = tbase + e;
        if (t < M) Y[(size_t)t * N + o] = acc[i][j][e];
      }
    }
  }
}

template <int TM, int R, int WPE>
int launch_gemm(const uint8_t *W, const uint4 *xa, float *Y, int N, int M, int nblk) {
  const int ntiles = q4k_tiles(N), MTG = gemm_mt(M) / TM;
  const int NTG = ceil_div(ntiles, 4 * R);
  const int grid = MTG * NTG;
  // XCD-grouped order is opt-in (FAK_HIP_GEMM_REMAP=1): measured 2-20% slower on the C3 shapes.
  const int remap = (grid % 8 == 0 && env_int("FAK_HIP_GEMM_REMAP")) ? 1 : 0;
  q4k_gemm_kernel<TM, R, WPE><<<grid, 256, 0, stream()>>>(W, xa, Y, N, M, nblk, ntiles, MTG, remap);
  FHIP_CHECK_LAUNCH("q4k_gemm_kernel");
  return FHIP_OK;
}

}  // namespace

int q4k_gemm(const void *Wv, const float *X, float *Y, int N, int K, int M) {
  if (!env_int("FAK_HIP_GEMM16")) return q4k_gemm32(Wv, X, Y, N, K, M);
  const uint8_t *W = (const uint8_t *)Wv;
  const int nblk = K / 256;
  uint4 *xa = (uint4 *)workspace(gemm_xa_bytes(M, K));
  if (!xa) return FHIP_ENOMEM;
  if (int rc = launch_gemm_xprep(X, M, K, xa)) return rc;
  // Shape: TM*100 + R*10 + waves per SIMD. 4x2 tiles at 3 waves/SIMD fill the chip better for
  // a few hundred tokens; 4x4 at 2 waves/SIMD reuses each activation tile more for long prompts.
  int cfg = env_int("FAK_HIP_GEMM_CFG");
  if (cfg == 0) cfg = M <= 1024 ? 423 : 442;
  switch (cfg) {
    case 442: return launch_gemm<4, 4, 2>(W, xa, Y, N, M, nblk);
    case 841: return launch_gemm<8, 4, 1>(W, xa, Y, N, M, nblk);
    case 423: return launch_gemm<4, 2, 3>(W, xa, Y, N, M, nblk);
    case 822: return launch_gemm<8, 2, 2>(W, xa, Y, N, M, nblk);
  }
  return fail(FHIP_EINVAL, "q4k_gemm: FAK_HIP_GEMM_CFG=%d is not a built shape", cfg);
}

}  // namespace fhip
