// q4k_gemm32.hip — large-M (prefill) Q4_K matmul on the 32x32x16 f16 MFMA.
//
// Y[t][o] = sum_k W[o][k] X[t][k] with W dequantized from the tiled Q4_K records (tiled.hpp) in
// registers and X pre-converted once to f16 operand tiles. On gfx950 v_mfma_f32_32x32x16_f16
// delivers about twice the throughput of the 16x16x32 form (measured 2.2-2.3 vs 1.2 PFLOP/s in a
// register-only loop), so the prefill GEMM is built on it:
//   * workgroup = 4 waves over 128 tokens x 128 rows; wave (wm, wn) owns 64 tokens x 64 rows =
//     2 x 2 MFMA tiles of 32 x 32, accumulated in f32 (64 registers);
//   * per super-block the workgroup stages the 8 tiled records of its 128 rows (18 KB, still
//     4-bit) in LDS, double-buffered; each lane reads the 8 nibble bytes its MFMA operand needs
//     (row rho of a 32-row MFMA tile = row rho % 16 of 16-row tile rho / 16) and dequantizes
//     them to f16 in registers exactly like the 16x16 GEMM did (w = d1*n - m1 with the 0x6400
//     exponent trick, one packed fma per pair);
//   * activations go global -> registers -> LDS one 64-wide K chunk at a time (16 KB),
//     double-buffered, each 16-byte lane unit already in operand order (gemm32_xprep_kernel).
// The MFMA sums over K, so any mapping of (lane group, element) to K positions works as long
// as both operands use it: here the K16 slice q holds positions 16q + 8 (lane / 32) + perm8(j),
// which is where the nibble unpack leaves the weights.
#include "kernels.hpp"

namespace fhip {
namespace {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ h2 as_h2(uint32_t u) { return __builtin_bit_cast(h2, u); }
__device__ __forceinline__ uint32_t as_u(h2 v) { return __builtin_bit_cast(uint32_t, v); }

struct Magic {
  uint32_t lo, hi, byte02, magic;
};
__device__ __forceinline__ Magic magic_consts() {
  return Magic{in_reg(0x000F000Fu), in_reg(0x00F000F0u), in_reg(0x00FF00FFu), in_reg(0x64006400u)};
}

// d1[s] = f16(d*sc_s) (odd s pre-divided by 16 for the in-place high-nibble mask) and
// m1[s] = f16(dmin*m_s) for the 8 sub-blocks of one row's super-block.
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

// The 8 nibble bytes (x0, x1) of chunk c at positions 8g..8g+7 become two f16 operands:
// sub-block 2c (low nibbles) and 2c + 1 (high nibbles), elements in perm8 order.
__device__ __forceinline__ void dequant8(uint32_t x0, uint32_t x1, const RowScales &s, int c,
                                         const Magic &K, f16x8 &bl, f16x8 &bh) {
  const h2 k1024 = {(_Float16)1024.f, (_Float16)1024.f};
  const int p = c >> 1, hsel = c & 1;
  const h2 de = s.d1e[p], dodd = s.d1o[p], me = s.m1e[p], mo = s.m1o[p];
  const _Float16 dl = hsel ? de.y : de.x, dh = hsel ? dodd.y : dodd.x;
  const _Float16 ml = hsel ? me.y : me.x, mh = hsel ? mo.y : mo.x;
  const h2 DL = {dl, dl}, DH = {dh, dh}, ML = {-ml, -ml}, MH = {-mh, -mh};
  const uint32_t y0 = x0 >> 8, y1 = x1 >> 8;
  u32x4 l, hh;
  l[0] = as_u((as_h2((x0 & K.lo) | K.magic) - k1024) * DL + ML);
  l[1] = as_u((as_h2((y0 & K.lo) | K.magic) - k1024) * DL + ML);
  l[2] = as_u((as_h2((x1 & K.lo) | K.magic) - k1024) * DL + ML);
  l[3] = as_u((as_h2((y1 & K.lo) | K.magic) - k1024) * DL + ML);
  hh[0] = as_u((as_h2((x0 & K.hi) | K.magic) - k1024) * DH + MH);
  hh[1] = as_u((as_h2((y0 & K.hi) | K.magic) - k1024) * DH + MH);
  hh[2] = as_u((as_h2((x1 & K.hi) | K.magic) - k1024) * DH + MH);
  hh[3] = as_u((as_h2((y1 & K.hi) | K.magic) - k1024) * DH + MH);
  bl = __builtin_bit_cast(f16x8, l);
  bh = __builtin_bit_cast(f16x8, hh);
}

constexpr int kBM = 128;               // tokens per workgroup
constexpr int kBT = 8;                 // 16-row tiles per workgroup (128 rows)
constexpr int kAU = 4 * 4 * 64;        // uint4 units of one activation stage (4 tiles x 4 K16)
constexpr int kWU = kBT * kQ4kRecord / 16;  // uint4 units of one super-block's records (1152)
constexpr int kWPT = (kWU + 255) / 256;     // per thread (5); the last 128 threads' fifth unit
constexpr int kWUP = kWPT * 256;            // re-reads a valid unit into LDS padding

// Activation operands: xa[(tt * (K/16) + q) * 64 + l] = 8 f16 of token 32 tt + l % 32 at
// K = 16 q + 8 (l / 32) + perm8(j); token tiles padded to whole workgroups (zeros).
__global__ void gemm32_xprep_kernel(const float *__restrict__ X, int M, int K, long long total,
                                    uint4 *__restrict__ xa) {
  const long long id = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= total) return;
  const int nq = K / 16;
  const int l = (int)(id & 63);
  const long long tq = id >> 6;
  const int tt = (int)(tq / nq), q = (int)(tq - (long long)tt * nq);
  const int t = 32 * tt + (l & 31);
  f16x8 h;
  if (t < M) {
    const float *x = X + (size_t)t * K + 16 * q + 8 * (l >> 5);
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

// NWB: LDS buffers for the weight records (2: the next super-block loads while the current one
// is read; 1: a second barrier per super-block, 52 KB of LDS, three workgroups per CU).
template <int NWB, int WPE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(WPE, WPE))) void q4k_gemm32_kernel(const uint8_t *__restrict__ W,
                                                         const uint4 *__restrict__ xa,
                                                         float *__restrict__ Y, int N, int M,
                                                         int nblk, int ntiles, int MTG) {
  __shared__ u32x4 As[2][kAU];
  __shared__ u32x4 Ws[NWB][kWUP];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 1, wn = wave >> 1;
  const int kap = lane >> 5, rho = lane & 31;
  const int mg = blockIdx.x % MTG, ng = blockIdx.x / MTG;
  const int nq = nblk * 16;
  const Magic K = magic_consts();

  // Global sources: this workgroup's 4 token tiles and 8 row tiles (clamped to the last tile,
  // whose outputs are not written).
  const u32x4 *xg = reinterpret_cast<const u32x4 *>(xa) + (size_t)(4 * mg) * nq * 64;
  // Unit u of a workgroup stage: activation tile u >> 8, K16 slice (u >> 6) & 3, lane u & 63;
  // record (u / 144) of the 8 row tiles, 16-byte unit u % 144 (past 1152: unit 0 again).
  // 16-byte unit offsets from xg / W (32-bit). Unit tid + 256 k of an activation stage is token
  // tile k, K16 slice tid >> 6, lane tid & 63: a uniform stride of one token tile per k.
  const uint32_t aoff = (uint32_t)(tid >> 6) * 64 + lane, astride = (uint32_t)nq * 64;
  // Weight unit tid + 256 k is record rec_k = u / 144, unit off_k = u % 144 of it (u past the
  // 1152 real units re-reads unit 0); the five (rec, off) pairs are packed 12 bits each.
  uint64_t wpack = 0;
#pragma unroll
  for (int k = 0; k < kWPT; ++k) {
    const int u = tid + 256 * k < kWU ? tid + 256 * k : 0;
    const int rec = u / (kQ4kRecord / 16), off = u - rec * (kQ4kRecord / 16);
    wpack |= (uint64_t)((rec << 8) | off) << (12 * k);
  }
  const int tile0 = kBT * ng;
  auto woff = [&](int k) {
    uint64_t wp = wpack;
    asm volatile("" : "+v"(wp));  // recomputed per load, not hoisted into five live registers
    const uint32_t f = (uint32_t)(wp >> (12 * k)) & 0xFFFu;
    const int T = min(tile0 + (int)(f >> 8), ntiles - 1);
    return (uint32_t)T * nblk * (kQ4kRecord / 16) + (f & 0xFFu);
  };
  const u32x4 *Wv = reinterpret_cast<const u32x4 *>(W);
#define LOAD_A(st, regs)                                                             \
  _Pragma("unroll") for (int k = 0; k < 4; ++k) regs[k] = xg[aoff + k * astride + (uint32_t)(st) * 256];
#define LOAD_W(b, regs)                                                              \
  _Pragma("unroll") for (int k = 0; k < kWPT; ++k) regs[k] = Wv[woff(k) + (uint32_t)(b) * (kQ4kRecord / 16)];
#define STORE_W(buf, regs) \
  _Pragma("unroll") for (int k = 0; k < kWPT; ++k) Ws[buf][tid + 256 * k] = regs[k];

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  u32x4 areg[4], wreg[kWPT];
  LOAD_W(0, wreg)
  LOAD_A(0, areg)
  STORE_W(0, wreg)
#pragma unroll
  for (int k = 0; k < 4; ++k) As[0][tid + 256 * k] = areg[k];
  __syncthreads();

  // This lane's 16-row tiles (local to the workgroup) for its two 32-row MFMA tiles, and the
  // byte offset of its row inside a record.
  const int Tl0 = 4 * wn + (rho >> 4), Tl1 = Tl0 + 2;
  const int r16 = rho & 15;
  const int nst = nblk * 4;
  for (int b = 0; b < nblk; ++b) {
    const int wb = NWB == 2 ? (b & 1) : 0;
    const unsigned char *wbase = reinterpret_cast<const unsigned char *>(Ws[wb]);
    RowScales rs[2];
    rs[0] = row_scales(__builtin_bit_cast(uint4, *reinterpret_cast<const u32x4 *>(wbase + Tl0 * kQ4kRecord + 16 * r16)), K);
    rs[1] = row_scales(__builtin_bit_cast(uint4, *reinterpret_cast<const u32x4 *>(wbase + Tl1 * kQ4kRecord + 16 * r16)), K);
    const bool more = b + 1 < nblk;
    if (more) {
      LOAD_W(b + 1, wreg)
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int st = 4 * b + c, cur = c & 1;
      if (st + 1 < nst) {
        LOAD_A(st + 1, areg)
      }
      // nibble bytes: lane group g = 2h + kap of chunk c, for both MFMA row tiles
      uint2 xb[2][2];
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int T = t ? Tl1 : Tl0, g = 2 * h + kap;
          xb[t][h] = *reinterpret_cast<const uint2 *>(wbase + T * kQ4kRecord + kQ4kHdr +
                                                      1024 * (c >> 1) + 16 * (16 * g + r16) +
                                                      8 * (c & 1));
        }
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        f16x8 bl[2], bh[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) dequant8(xb[t][h].x, xb[t][h].y, rs[t], c, K, bl[t], bh[t]);
#pragma unroll
        for (int hi = 0; hi < 2; ++hi) {
          const int ql = 2 * hi + h;  // K16 slice within the chunk
#pragma unroll
          for (int i = 0; i < 2; ++i) {
            const f16x8 a = __builtin_bit_cast(f16x8, As[cur][((2 * wm + i) * 4 + ql) * 64 + lane]);
#pragma unroll
            for (int t = 0; t < 2; ++t)
              acc[i][t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, hi ? bh[t] : bl[t], acc[i][t],
                                                                  0, 0, 0);
          }
        }
      }
      if (st + 1 < nst) {
#pragma unroll
        for (int k = 0; k < 4; ++k) As[cur ^ 1][tid + 256 * k] = areg[k];
      }
      if (c == 3 && more) {
        if (NWB == 1) __syncthreads();  // every wave is done reading this super-block's records
        STORE_W(NWB == 2 ? wb ^ 1 : 0, wreg)
      }
      __syncthreads();
    }
  }

#undef LOAD_A
#undef LOAD_W
#undef STORE_W

  // D layout: lane (kap, rho) holds column rho (the row o) and tokens 8 (v / 4) + 4 kap + v % 4.
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int t0 = kBM * mg + 32 * (2 * wm + i) + 4 * kap;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int o = 16 * (kBT * ng + 4 * wn + 2 * t) + rho;
      if (o >= N) continue;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int tok = t0 + 8 * (v >> 2) + (v & 3);
        if (tok < M) Y[(size_t)tok * N + o] = acc[i][t][v];
      }
    }
  }
}

}  // namespace

size_t gemm32_xa_bytes(int M, int K) { return (size_t)ceil_div(M, kBM) * kBM * K * 2; }

int q4k_gemm32(const void *Wv, const float *X, float *Y, int N, int K, int M) {
  const int nblk = K / 256;
  uint4 *xa = (uint4 *)workspace(gemm32_xa_bytes(M, K));
  if (!xa) return FHIP_ENOMEM;
  const int MTG = ceil_div(M, kBM);
  const long long total = (long long)MTG * 4 * (K / 16) * 64;
  gemm32_xprep_kernel<<<(unsigned)((total + 255) / 256), 256, 0, stream()>>>(X, M, K, total, xa);
  FHIP_CHECK_LAUNCH("gemm32_xprep_kernel");
  const int ntiles = q4k_tiles(N);
  const int grid = MTG * ceil_div(ntiles, kBT);
  int nwb = env_int("FAK_HIP_GEMM32_NWB");
  if (nwb == 0) nwb = 1;
  if (nwb == 1)
    q4k_gemm32_kernel<1, 3><<<grid, 256, 0, stream()>>>((const uint8_t *)Wv, xa, Y, N, M, nblk,
                                                        ntiles, MTG);
  else
    q4k_gemm32_kernel<2, 2><<<grid, 256, 0, stream()>>>((const uint8_t *)Wv, xa, Y, N, M, nblk,
                                                        ntiles, MTG);
  FHIP_CHECK_LAUNCH("q4k_gemm32_kernel");
  return FHIP_OK;
}

}  // namespace fhip
