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
//
// Q4_K runs q4k_gemm32s_kernel<4>: the same tile and K order with four waves of 128 tokens x
// 32 rows each and activations staged by direct-to-LDS loads (described there).
//
// The same kernel runs Q6_K weights (FMT 1) from the Q6_K tiled records (tiled.hpp): the K16
// slice q of a row is its 16-weight group q, whose codes sit in one 16-byte ql unit (a nibble)
// and one 16-byte qh unit (a 2-bit field); a lane takes the 8 codes of its half (8 kap ..) and
// makes w = (c - 32) * f16(d * sc) in f16: (1024 + c) - 1056 is exact, one rounding for the
// product.
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

// Q6_K: the 8 codes of slices a (group g' = h) and b (g' = 2 + h) of chunk c = 2 h' + k from
// their ql bytes (nibble k) and the shared qh bytes (fields 4k and 4k + 2), as f16 weights.
__device__ __forceinline__ void dequant6(uint2 qa, uint2 qb, uint2 qh, int k, _Float16 Sa,
                                         _Float16 Sb, uint32_t m0F, uint32_t m03,
                                         const Magic &K, f16x8 &ba, f16x8 &bb) {
  const h2 k1056 = {(_Float16)1056.f, (_Float16)1056.f};
  const h2 SA = {Sa, Sa}, SB = {Sb, Sb};
  const uint32_t qav[2] = {qa.x, qa.y}, qbv[2] = {qb.x, qb.y}, qhv[2] = {qh.x, qh.y};
  u32x4 ra, rb;
#pragma unroll
  for (int m = 0; m < 2; ++m) {
    const uint32_t ca = ((qav[m] >> (4 * k)) & m0F) | (((qhv[m] >> (4 * k)) & m03) << 4);
    const uint32_t cb = ((qbv[m] >> (4 * k)) & m0F) | (((qhv[m] >> (4 * k + 2)) & m03) << 4);
    // bytes (0, 2) and (1, 3) of each code word: elements in perm8 order
    ra[2 * m] = as_u((as_h2((ca & K.byte02) | K.magic) - k1056) * SA);
    ra[2 * m + 1] = as_u((as_h2(((ca >> 8) & K.byte02) | K.magic) - k1056) * SA);
    rb[2 * m] = as_u((as_h2((cb & K.byte02) | K.magic) - k1056) * SB);
    rb[2 * m + 1] = as_u((as_h2(((cb >> 8) & K.byte02) | K.magic) - k1056) * SB);
  }
  ba = __builtin_bit_cast(f16x8, ra);
  bb = __builtin_bit_cast(f16x8, rb);
}

constexpr int kBM = 128;               // tokens per workgroup
constexpr int kBT = 8;                 // 16-row tiles per workgroup (128 rows)
constexpr int kTileElems = kBM * 128;  // outputs of one workgroup tile
constexpr int kAU = 4 * 4 * 64;        // uint4 units of one activation stage (4 tiles x 4 K16)

// Per weight format: record bytes, uint4 units of one super-block's records for the workgroup's
// 8 row tiles, units per thread (the last threads re-read a valid unit into LDS padding).
template <int FMT>
struct GemmFmt {
  static constexpr int kRec = FMT == 0 ? kQ4kRecord : kQ6kRecord;
  static constexpr int kUnits = kRec / 16;         // 144 or 210
  static constexpr int kWU = kBT * kUnits;         // 1152 or 1680
  static constexpr int kWPT = (kWU + 255) / 256;   // 5 or 7
  static constexpr int kWUP = kWPT * 256;
};

// Activation operands: xa[(tt * (K/16) + q) * 64 + l] = 8 f16 of token 32 tt + l % 32 at
// K = 16 q + 8 (l / 32) + perm8(j); token tiles padded to whole workgroups (zeros). Each token
// row is scaled by a power of two 2^-k that puts its largest magnitude in [2^14, 2^15), so any
// finite f32 row converts to f16 without overflow and keeps 11-bit relative precision down to
// 2^-28 of its maximum; the GEMM multiplies the token's outputs by tscale[t] = 2^k (exact), NaN
// for a row holding a NaN or an infinity (its operands are zeros), 1 for an all-zero row.
// One workgroup per (padded) token: a max-reduce over the row, then the conversion. UPT > 0: each
// thread loads its UPT 8-value units of the row at once (unconditionally, indices clamped to the
// row; a repeated unit changes neither the maximum nor the NaN flag) and converts them from its
// registers, so the row is read once with every load in flight together (rows of K <= 8 NT UPT).
// UPT = 0: a loop over the row, read twice (the second pass hits L2), for longer rows.
// NT: threads per workgroup, 256, or 1024 for rows longer than 8192 values, so that each thread
// holds fewer of them (K=18944 at M=512: 15.1 us against 16.2 with 256 threads of 12 units).
template <int UPT, int NT>
__global__ __launch_bounds__(NT) void gemm32_xprep_kernel(
    const float *__restrict__ X, int M, int K, uint4 *__restrict__ xa, float *__restrict__ tscale) {
  constexpr int kXprepThreads = NT;
  __shared__ float wmax[kXprepThreads / 64];
  // Token of this workgroup: the 32 tokens of an operand tile run on one XCD (workgroups go to
  // the 8 XCDs round-robin), so one L2 assembles each 512-byte operand block from its 32 16-byte
  // pieces instead of eight L2s writing back partial lines (M=512 6.2 -> 5.2 us, M=2048 19.8 ->
  // 13.2 us). Whole groups of 256 workgroups are remapped; a remainder keeps its order.
  int t = blockIdx.x;
  if (t < (int)(gridDim.x & ~255u)) {
    const int x = t & 7, slot = t >> 3;
    t = 32 * (8 * (slot >> 5) + x) + (slot & 31);
  }
  const int tid = threadIdx.x;
  const int nq = K / 16, nu = K / 8;  // 16-K slices and 8-value units of the row
  const bool valid = t < M;
  const float4 *row = reinterpret_cast<const float4 *>(X + (size_t)(valid ? t : 0) * K);
  // fmaxf drops NaN: a NaN anywhere must still mark the row, so it is tracked separately.
  float amax = 0.f;
  bool bad = false;
  auto see = [&](const float4 v) {
    amax = fmaxf(fmaxf(amax, fabsf(v.x)), fmaxf(fmaxf(fabsf(v.y), fabsf(v.z)), fabsf(v.w)));
    bad |= (v.x != v.x) | (v.y != v.y) | (v.z != v.z) | (v.w != v.w);
  };
  float4 reg[UPT > 0 ? UPT : 1][2];
  if (UPT > 0) {
#pragma unroll
    for (int j = 0; j < UPT; ++j) {
      const int u = min(tid + j * kXprepThreads, nu - 1);
      reg[j][0] = row[2 * u];
      reg[j][1] = row[2 * u + 1];
    }
#pragma unroll
    for (int j = 0; j < UPT; ++j) {
      see(reg[j][0]);
      see(reg[j][1]);
    }
  } else {
    for (int i = tid; i < K / 4; i += kXprepThreads) see(row[i]);
  }
  if (!valid) amax = 0.f, bad = false;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
  const bool wbad = __any(bad);
  if ((tid & 63) == 0) wmax[tid >> 6] = wbad ? __builtin_nanf("") : amax;
  __syncthreads();
  float m = 0.f;
  bool nan = false;
#pragma unroll
  for (int w = 0; w < kXprepThreads / 64; ++w) {
    nan |= wmax[w] != wmax[w];
    m = fmaxf(m, wmax[w]);
  }
  const bool finite = !nan && m <= 3.4028235e38f;
  int E = 0;
  (void)frexpf(m, &E);
  const int k = E - 15;  // m / 2^k in [2^14, 2^15)
  if (tid == 0) tscale[t] = !finite ? __builtin_nanf("") : m > 0.f ? ldexpf(1.f, k) : 1.f;
  const int tt = t >> 5, lt = t & 31;
  auto put = [&](int u, const float4 v0, const float4 v1) {
    const int q = u >> 1, half = u & 1;
    f16x8 h;
    if (valid && finite) {
      const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
#pragma unroll
      for (int j = 0; j < 8; ++j) h[j] = (_Float16)ldexpf(v[perm8(j)], -k);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) h[j] = (_Float16)0.f;
    }
    xa[((size_t)tt * nq + q) * 64 + 32 * half + lt] = __builtin_bit_cast(uint4, h);
  };
  if (UPT > 0) {
#pragma unroll
    for (int j = 0; j < UPT; ++j) {
      const int u = tid + j * kXprepThreads;
      if (u < nu) put(u, reg[j][0], reg[j][1]);
    }
  } else {
    for (int u = tid; u < nu; u += kXprepThreads) put(u, row[2 * u], row[2 * u + 1]);
  }
}

// Launches the activation prep with the smallest register-resident unit count that covers K:
// 256 threads per token up to 8192 values, 1024 above.
void launch_xprep(const float *X, int M, int K, int MTG, uint4 *xa, float *ts) {
  const unsigned grid = MTG * kBM;
  if (K <= 8192) {
    const int upt = ceil_div(K / 8, 256);
    if (upt <= 2)
      gemm32_xprep_kernel<2, 256><<<grid, 256, 0, stream()>>>(X, M, K, xa, ts);
    else
      gemm32_xprep_kernel<4, 256><<<grid, 256, 0, stream()>>>(X, M, K, xa, ts);
    return;
  }
  const int upt = ceil_div(K / 8, 1024);
  if (upt <= 1)
    gemm32_xprep_kernel<1, 1024><<<grid, 1024, 0, stream()>>>(X, M, K, xa, ts);
  else if (upt <= 2)
    gemm32_xprep_kernel<2, 1024><<<grid, 1024, 0, stream()>>>(X, M, K, xa, ts);
  else if (upt <= 3)
    gemm32_xprep_kernel<3, 1024><<<grid, 1024, 0, stream()>>>(X, M, K, xa, ts);
  else if (upt <= 4)
    gemm32_xprep_kernel<4, 1024><<<grid, 1024, 0, stream()>>>(X, M, K, xa, ts);
  else
    gemm32_xprep_kernel<0, 1024><<<grid, 1024, 0, stream()>>>(X, M, K, xa, ts);
}

// FMT: 0 Q4_K, 1 Q6_K. NWB: LDS buffers for the weight records (2: the next super-block loads
// while the current one is read; 1: a second barrier per super-block; Q4_K with one buffer uses
// 52 KB of LDS, three workgroups per CU).
template <int FMT, int NWB, int WPE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(WPE, WPE))) void quant_gemm32_kernel(const uint8_t *__restrict__ W,
                                                         const uint4 *__restrict__ xa,
                                                         const float *__restrict__ tscale,
                                                         float *__restrict__ Y, int N, int M,
                                                         int nblk, int ntiles, int MTG, int F0,
                                                         int S, int R, float *__restrict__ part) {
  using F = GemmFmt<FMT>;
  constexpr int kRec = F::kRec, kWU = F::kWU, kWPT = F::kWPT, kWUP = F::kWUP;
  __shared__ u32x4 As[2][kAU];
  __shared__ u32x4 Ws[NWB][kWUP];
  __shared__ __align__(16) float ts_lds[kBM];  // the token scales of this token tile
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 1, wn = wave >> 1;
  const int kap = lane >> 5, rho = lane & 31;
  // Workgroup -> (tile task, K range sp of ns), as in q4k_gemm32s_kernel: the first F0
  // workgroups run whole tiles, the next R * S the last R tiles in S K ranges each; range 0
  // writes Y, the others their partial sums for gemm32_reduce_kernel.
  const int w = blockIdx.x;
  const bool split = w >= F0;
  const int pw = split ? w - F0 : 0;
  const int task = split ? F0 + pw / S : w, sp = split ? pw % S : 0, ns = split ? S : 1;
  const int mg = task % MTG, ng = task / MTG;
  const int kb0 = sp * nblk / ns, kb1 = (sp + 1) * nblk / ns;  // >= 1 super-block: S <= nblk
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
  // Weight unit tid + 256 k is record rec_k = u / units, unit off_k = u % units of it (u past
  // the real units re-reads unit 0). Q4_K packs the five (rec, off) pairs 12 bits each.
  uint64_t wpack = 0;
  if (FMT == 0) {
#pragma unroll
    for (int k = 0; k < kWPT; ++k) {
      const int u = tid + 256 * k < kWU ? tid + 256 * k : 0;
      const int rec = u / F::kUnits, off = u - rec * F::kUnits;
      wpack |= (uint64_t)((rec << 8) | off) << (12 * k);
    }
  }
  const int tile0 = kBT * ng;
  auto woff = [&](int k) {
    uint32_t rec, off;
    if (FMT == 0) {
      uint64_t wp = wpack;
      asm volatile("" : "+v"(wp));  // recomputed per load, not hoisted into five live registers
      const uint32_t f = (uint32_t)(wp >> (12 * k)) & 0xFFFu;
      rec = f >> 8;
      off = f & 0xFFu;
    } else {
      const int u = tid + 256 * k < kWU ? tid + 256 * k : 0;
      rec = (uint32_t)(u / F::kUnits);
      off = (uint32_t)u - rec * F::kUnits;
    }
    const int T = min(tile0 + (int)rec, ntiles - 1);
    return (uint32_t)T * nblk * F::kUnits + off;
  };
  const u32x4 *Wv = reinterpret_cast<const u32x4 *>(W);
#define LOAD_A(st, regs)                                                             \
  _Pragma("unroll") for (int k = 0; k < 4; ++k) regs[k] = xg[aoff + k * astride + (uint32_t)(st) * 256];
#define LOAD_W(b, regs)                                                              \
  _Pragma("unroll") for (int k = 0; k < kWPT; ++k) regs[k] = Wv[woff(k) + (uint32_t)(b) * F::kUnits];
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
  LOAD_W(kb0, wreg)
  LOAD_A(4 * kb0, areg)
  if (tid < kBM) ts_lds[tid] = tscale[kBM * mg + tid];  // tscale holds MTG * kBM entries
  STORE_W(0, wreg)
#pragma unroll
  for (int k = 0; k < 4; ++k) As[0][tid + 256 * k] = areg[k];
  __syncthreads();

  // This lane's 16-row tiles (local to the workgroup) for its two 32-row MFMA tiles, and the
  // byte offset of its row inside a record.
  const int Tl0 = 4 * wn + (rho >> 4), Tl1 = Tl0 + 2;
  const int r16 = rho & 15;
  const int nst = kb1 * 4;
  for (int b = kb0; b < kb1; ++b) {
    const int wb = NWB == 2 ? (b & 1) : 0;
    const unsigned char *wbase = reinterpret_cast<const unsigned char *>(Ws[wb]);
    RowScales rs[2];
    uint4 sc6[2];  // Q6_K: the row's 16 int8 scales
    float d6[2];   // Q6_K: the row's d
    if (FMT == 0) {
      rs[0] = row_scales(__builtin_bit_cast(uint4, *reinterpret_cast<const u32x4 *>(wbase + Tl0 * kRec + 16 * r16)), K);
      rs[1] = row_scales(__builtin_bit_cast(uint4, *reinterpret_cast<const u32x4 *>(wbase + Tl1 * kRec + 16 * r16)), K);
    } else {
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const unsigned char *rec = wbase + (t ? Tl1 : Tl0) * kRec;
        sc6[t] = __builtin_bit_cast(uint4, *reinterpret_cast<const u32x4 *>(rec + 16 * r16));
        d6[t] = (float)__builtin_bit_cast(_Float16, *reinterpret_cast<const uint16_t *>(rec + kQ6kD + 2 * r16));
      }
    }
    const bool more = b + 1 < kb1;
    if (more) {
      LOAD_W(b + 1, wreg)
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int st = 4 * b + c, cur = c & 1;
      if (st + 1 < nst) {
        LOAD_A(st + 1, areg)
      }
      // Q4_K: nibble bytes of lane group g = 2h + kap of chunk c, for both MFMA row tiles.
      // Q6_K: ql bytes of groups 4c + h and 4c + 2 + h and their qh bytes (half kap).
      uint2 xb[2][2], x6[2][2][3];
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int T = t ? Tl1 : Tl0;
          if (FMT == 0) {
            const int g = 2 * h + kap;
            xb[t][h] = *reinterpret_cast<const uint2 *>(wbase + T * kRec + kQ4kHdr +
                                                        1024 * (c >> 1) + 16 * (16 * g + r16) +
                                                        8 * (c & 1));
          } else {
            const unsigned char *rec = wbase + T * kRec;
            const int hh = c >> 1;
            x6[t][h][0] = *reinterpret_cast<const uint2 *>(rec + kQ6kQl + 1024 * hh +
                                                           16 * (16 * h + r16) + 8 * kap);
            x6[t][h][1] = *reinterpret_cast<const uint2 *>(rec + kQ6kQl + 1024 * hh +
                                                           16 * (16 * (2 + h) + r16) + 8 * kap);
            x6[t][h][2] = *reinterpret_cast<const uint2 *>(rec + kQ6kQh + 512 * hh + 256 * h +
                                                           16 * r16 + 8 * kap);
          }
        }
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        f16x8 bl[2], bh[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          if (FMT == 0) {
            dequant8(xb[t][h].x, xb[t][h].y, rs[t], c, K, bl[t], bh[t]);
          } else {
            const uint32_t scw = c == 0 ? sc6[t].x : c == 1 ? sc6[t].y : c == 2 ? sc6[t].z : sc6[t].w;
            const _Float16 Sa = (_Float16)(d6[t] * (float)(int8_t)(scw >> (8 * h)));
            const _Float16 Sb = (_Float16)(d6[t] * (float)(int8_t)(scw >> (8 * (2 + h))));
            dequant6(x6[t][h][0], x6[t][h][1], x6[t][h][2], c & 1, Sa, Sb,
                     in_reg(0x0F0F0F0Fu), in_reg(0x03030303u), K, bl[t], bh[t]);
          }
        }
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
  // The token scales come from LDS, four per read: a global load per output would make every
  // store wait for the previous one.
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int tl0 = 32 * (2 * wm + i) + 4 * kap, t0 = kBM * mg + tl0;
    float sc[16];
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      const float4 s4 = *reinterpret_cast<const float4 *>(ts_lds + tl0 + 8 * a);
      sc[4 * a] = s4.x; sc[4 * a + 1] = s4.y; sc[4 * a + 2] = s4.z; sc[4 * a + 3] = s4.w;
    }
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int o = 16 * (kBT * ng + 4 * wn + 2 * t) + rho;
      if (o >= N) continue;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int tok = t0 + 8 * (v >> 2) + (v & 3);
        if (tok >= M) continue;
        const float val = acc[i][t][v] * sc[v];
        if (sp == 0)
          Y[(size_t)tok * N + o] = val;
        else
          part[((size_t)(sp - 1) * R + (task - F0)) * kTileElems + (tok - kBM * mg) * 128 +
               (o - 128 * ng)] = val;
      }
    }
  }
}


// s_waitcnt immediate (vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] at [15:14]) followed
// by a bare workgroup barrier. __syncthreads() would add a workgroup fence, and with LDS DMA in
// flight the fence waits for every outstanding load (vmcnt(0)), including the ones issued early
// on purpose. The asm statements keep the compiler from moving LDS accesses across the barrier.
#define FHIP_LDS_BARRIER(imm)        \
  do {                               \
    __builtin_amdgcn_s_waitcnt(imm); \
    asm volatile("" ::: "memory");   \
    __builtin_amdgcn_s_barrier();    \
    asm volatile("" ::: "memory");   \
  } while (0)
constexpr int wait_vm(int n) { return 0x0070 | (n & 15) | ((n >> 4) << 14); }  // vmcnt(n), lgkmcnt(0)

// Q4_K: the staged form. Same 128-token x 128-row workgroup tile, grid and K order as
// quant_gemm32_kernel (bit-identical results), but
//   * each of the four waves owns all 128 tokens x 32 rows (4 MFMA tiles), so every dequantized
//     weight operand feeds four MFMAs instead of two and each weight is dequantized once per
//     workgroup (the four-wave 2x2 form dequantizes every row twice);
//   * activations go global -> LDS directly (global_load_lds_dwordx4, no staging registers) in
//     8 KB stages of two K16 slices {h, 2 + h} of a 64-K chunk, four stage buffers, each stage
//     loaded three stages ahead; every load is issued unconditionally (indices clamped at the
//     end of K) so each wait is a compile-time count that leaves the later stages in flight;
//   * the weights go straight from the tiled records to the registers of the lanes that use
//     them (a header and four nibble units per lane and super-block), with no LDS round trip and
//     no second barrier per super-block (measured 4-5% faster than records staged through LDS
//     at M = 128 / 512 / 2048: 41.5 / 97 / 367 us against 43.6 / 100-103 / 382-394).
// 166 VGPRs and 33 KB of LDS: three workgroups (12 waves) per CU, so the 592 workgroups of
// M=512 spread to at most three 32-row waves per SIMD. Two waves of 64 rows per workgroup
// (256 VGPRs, two per SIMD) measured slower at every size (M=512 112.7 against 106.5 us, M=2048
// 413 against 376, with the records still in LDS) and no longer fit their registers.
constexpr int kGemmWaves = 4;
// Loads a wave may leave pending at the end of stage ls (0..7) of a super-block, with nt 32-row
// tiles per wave: the DMA of the two later stages (kdma each), and for Q6_K the record group
// issued at stage 0 (6 nt loads) through stage 2 and the one issued at stage 4 (8 nt loads)
// through stage 6. Q4_K's records (2 nt and 3 nt loads) complete within the stage after their
// issue: with plain loads pending beside the LDS DMA the compiler no longer trusts the counter's
// order and drains it (vmcnt(0)) before the next read of a DMA buffer, twice per super-block,
// which measured the same.
constexpr int gemm32s_wait(int fmt, int nt, int ls, int kdma) {
  return fmt == 0 ? 2 * kdma + (ls <= 1 ? 2 * (nt - 1) : 0) + (ls == 4 || ls == 5 ? 3 * (nt - 1) : 0)
                  : 2 * kdma + (ls <= 2 ? 6 * nt : 0) + (ls >= 4 && ls <= 6 ? 8 * nt : 0);
}
template <int FMT, int WPE, int NTW>
__global__ __launch_bounds__(64 * kGemmWaves) __attribute__((amdgpu_waves_per_eu(WPE, WPE))) void quant_gemm32s_kernel(
    const uint8_t *__restrict__ W, const uint4 *__restrict__ xa,
    const float *__restrict__ tscale, float *__restrict__ Y, int N,
    int M, int nblk, int ntiles, int MTG, int F, int S, int R, float *__restrict__ part) {
  constexpr int NW = kGemmWaves;
  constexpr int kUnits = kQ4kRecord / 16;                       // 144 units per Q4_K record
  constexpr int kSU = 4 * 2 * 64;                               // 512 units (8 KB) per stage
  constexpr int NT = NTW;                                       // 32-row MFMA tiles per wave
  constexpr int kBTn = 2 * NT * NW;                             // 16-row tiles per workgroup
  constexpr int kRT = 16 * kBTn;                                // rows per workgroup tile
  constexpr int kDMA = 8 / NW;                                  // stage loads per wave
  // Four named arrays, not one indexed array: the compiler tracks LDS DMA per object, so a read
  // of one stage does not wait for the DMA into another.
  __shared__ u32x4 As0[kSU];
  __shared__ u32x4 As1[kSU];
  __shared__ u32x4 As2[kSU];
  __shared__ u32x4 As3[kSU];
  __shared__ __align__(16) float ts_lds[kBM];  // the token scales of this token tile
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kap = lane >> 5, rho = lane & 31;
  // Workgroup -> (tile task, K range sp of ns): the first F workgroups run whole tiles, the
  // next R * S the last R tiles in S K ranges each. Range 0 writes Y, the others their partial
  // sums, which gemm32_reduce_kernel adds to Y in range order.
  const int w = blockIdx.x;
  const bool split = w >= F;
  const int pw = split ? w - F : 0;
  const int task = split ? F + pw / S : w, sp = split ? pw % S : 0, ns = split ? S : 1;
  const int mg = task % MTG, ng = task / MTG;
  const int kb0 = sp * nblk / ns, kb1 = (sp + 1) * nblk / ns;  // >= 1 super-block: S <= nblk
  const int nq = nblk * 16;
  const Magic K = magic_consts();
  const u32x4 *xg = reinterpret_cast<const u32x4 *>(xa) + (size_t)(4 * mg) * nq * 64;
  const int tile0 = kBTn * ng;
  // Stage s = 8 b + 2 c + h: slices 16 (4 b + c) + h + 2 hi of token tile i at [(2 i + hi) * 64],
  // one 1 KB wave load each; wave w loads units kDMA w .. kDMA w + kDMA - 1 (unit 2 i + hi).
  auto load_stage = [&](int s, u32x4 *dst) {
    const int ch = 4 * kb0 + (s >> 1), h = s & 1;  // s counts from the range start
#pragma unroll
    for (int j = 0; j < kDMA; ++j) {
      const int p = kDMA * wave + j, i = p >> 1, hi = p & 1;
      __builtin_amdgcn_global_load_lds(
          (const void *)(xg + ((size_t)i * nq + 4 * ch + h + 2 * hi) * 64 + lane),
          (__attribute__((address_space(3))) void *)(dst + (2 * i + hi) * 64), 16, 0, 0);
    }
  };
  auto buf = [&](int k) -> u32x4 * { return k == 0 ? As0 : k == 1 ? As1 : k == 2 ? As2 : As3; };

  // The weights go straight to registers. Q4_K: lane (kap, rho) needs, per super-block and
  // 32-row tile t, the 16 header bytes of row rho % 16 of 16-row tile tl(t) and four 16-byte
  // units of nibble bytes (lane group 2 h + kap of chunks 2 c2, 2 c2 + 1). Q6_K: the row's 16
  // int8 scales and f16 d, and per half hh of the super-block (chunks 2 hh, 2 hh + 1) the lane's
  // 8 ql bytes of each of the four groups and 8 qh bytes of each K16 half. Rows past N read the
  // last tile.
  auto tl = [&](int t) { return 2 * NT * wave + 2 * t + (rho >> 4); };
  const int r16 = rho & 15;
  const u32x4 *Wv = reinterpret_cast<const u32x4 *>(W);
  auto rec = [&](int t, int b) {
    return Wv + ((size_t)min(tile0 + tl(t), ntiles - 1) * nblk + b) * kUnits;
  };
  auto rec6 = [&](int t, int b) {
    return W + ((size_t)min(tile0 + tl(t), ntiles - 1) * nblk + b) * kQ6kRecord;
  };
  auto nib = [&](int c2, int h) { return kQ4kHdr / 16 + 64 * c2 + 16 * (2 * h + kap) + r16; };
  u32x4 hdr[NT], u0[NT][2], u1[NT][2];    // Q4_K
  uint2 ql6[NT][2][4], qh6[NT][2][2];     // Q6_K: [half][group], [half][K16 half]
  uint32_t dw6[NT];                       // Q6_K: the row's d (f16 bits)
  auto load_hu0 = [&](int b) {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      if (FMT == 0) {
        const u32x4 *r = rec(t, b);
        hdr[t] = r[r16];
        u0[t][0] = r[nib(0, 0)];
        u0[t][1] = r[nib(0, 1)];
      } else {
        const uint8_t *r = rec6(t, b);
        hdr[t] = *reinterpret_cast<const u32x4 *>(r + 16 * r16);
        dw6[t] = *reinterpret_cast<const uint16_t *>(r + kQ6kD + 2 * r16);
#pragma unroll
        for (int g = 0; g < 4; ++g)
          ql6[t][0][g] = *reinterpret_cast<const uint2 *>(r + kQ6kQl + 16 * (16 * g + r16) + 8 * kap);
#pragma unroll
        for (int h = 0; h < 2; ++h)
          qh6[t][0][h] = *reinterpret_cast<const uint2 *>(r + kQ6kQh + 256 * h + 16 * r16 + 8 * kap);
      }
    }
  };
  auto load_u1 = [&](int b) {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      if (FMT == 0) {
        const u32x4 *r = rec(t, b);
        u1[t][0] = r[nib(1, 0)];
        u1[t][1] = r[nib(1, 1)];
      } else {
        const uint8_t *r = rec6(t, b);
#pragma unroll
        for (int g = 0; g < 4; ++g)
          ql6[t][1][g] = *reinterpret_cast<const uint2 *>(r + kQ6kQl + 1024 + 16 * (16 * g + r16) +
                                                          8 * kap);
#pragma unroll
        for (int h = 0; h < 2; ++h)
          qh6[t][1][h] = *reinterpret_cast<const uint2 *>(r + kQ6kQh + 512 + 256 * h + 16 * r16 +
                                                          8 * kap);
      }
    }
  };

  f32x16 acc[4][NT];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  const int nstage = (kb1 - kb0) * 8;
  // Issue order as in the loop below at the start of a super-block: header and chunk 0-1
  // units, then stages 0-2.
  load_hu0(kb0);
  load_stage(0, As0);
  load_stage(1, As1);
  load_stage(2, As2);
  for (int k = tid; k < kBM; k += 64 * NW) ts_lds[k] = tscale[kBM * mg + k];  // MTG * kBM entries
  FHIP_LDS_BARRIER(wait_vm(2 * kDMA));

  // A record register enters the arithmetic through an empty asm at the stage that first uses
  // it: the compiler would otherwise hoist the dequantization next to the load and wait for it
  // there (vmcnt(0)), with the registers of both held at once.
  auto pin = [](u32x4 &v) { asm volatile("" : "+v"(v)); };
  auto pin2 = [](uint2 &v) { asm volatile("" : "+v"(v.x), "+v"(v.y)); };
  for (int b = kb0; b < kb1; ++b) {
    RowScales rs[NT];
    uint32_t sc6[NT][4];  // Q6_K: the row's 16 int8 scales, one word per chunk
    float d6[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      pin(hdr[t]);
      if (FMT == 0) {
        rs[t] = row_scales(__builtin_bit_cast(uint4, hdr[t]), K);
      } else {
        asm volatile("" : "+v"(dw6[t]));
#pragma unroll
        for (int j = 0; j < 4; ++j) sc6[t][j] = hdr[t][j];
        d6[t] = (float)__builtin_bit_cast(_Float16, (uint16_t)dw6[t]);
      }
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      if (c == 0 || c == 2)
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          if (FMT == 0) {
#pragma unroll
            for (int h = 0; h < 2; ++h) pin(c == 0 ? u0[t][h] : u1[t][h]);
          } else {
#pragma unroll
            for (int g = 0; g < 4; ++g) pin2(ql6[t][c >> 1][g]);
#pragma unroll
            for (int h = 0; h < 2; ++h) pin2(qh6[t][c >> 1][h]);
          }
        }
      uint2 xb[NT][2];  // Q4_K: nibble bytes of lane group g = 2 h + kap of chunk c
      if (FMT == 0) {
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const u32x4 v = c < 2 ? u0[t][h] : u1[t][h];
            xb[t][h] = (c & 1) ? make_uint2(v[2], v[3]) : make_uint2(v[0], v[1]);
          }
      }
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int ls = 2 * c + h;  // stage within the super-block (its buffer is ls & 3)
        const int s = 8 * (b - kb0) + ls;
        load_stage(min(s + 3, nstage - 1), buf((ls + 3) & 3));
        // Each record register is reloaded once its last use has been read out: chunk 2-3
        // units of this super-block at stage 0 (used from stage 4), header and chunk 0-1 units
        // of the next one at stage 4 (used from its stage 0).
        if (ls == 0) load_u1(b);
        if (ls == 4) load_hu0(min(b + 1, kb1 - 1));
        const u32x4 *Acur = buf(ls & 3);
        f16x8 bl[NT], bh[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          if (FMT == 0) {
            dequant8(xb[t][h].x, xb[t][h].y, rs[t], c, K, bl[t], bh[t]);
          } else {
            // K16 slices h (ql group h) and 2 + h (group 2 + h) of chunk c: nibble c & 1 of the
            // half's ql bytes, 2-bit fields of its qh bytes; scales of sub-blocks 4c + h, 4c + 2 + h
            uint32_t scw = sc6[t][c];
            float dd6 = d6[t];
            uint2 qa = ql6[t][c >> 1][h], qb = ql6[t][c >> 1][2 + h], qhh = qh6[t][c >> 1][h];
            pin2(qa); pin2(qb); pin2(qhh);
            asm volatile("" : "+v"(scw), "+v"(dd6));
            const _Float16 Sa = (_Float16)(dd6 * (float)(int8_t)(scw >> (8 * h)));
            const _Float16 Sb = (_Float16)(dd6 * (float)(int8_t)(scw >> (8 * (2 + h))));
            dequant6(qa, qb, qhh, c & 1, Sa, Sb,
                     in_reg(0x0F0F0F0Fu), in_reg(0x03030303u), K, bl[t], bh[t]);
          }
        }
#pragma unroll
        for (int hi = 0; hi < 2; ++hi) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const f16x8 a = __builtin_bit_cast(f16x8, Acur[(2 * i + hi) * 64 + lane]);
#pragma unroll
            for (int t = 0; t < NT; ++t)
              acc[i][t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, hi ? bh[t] : bl[t], acc[i][t], 0, 0, 0);
          }
          // Q6_K, and 64 rows per wave: the second K16 half's operand reads wait for the first
          // half's MFMAs (and Q6_K's code words enter each stage through fresh pinned copies):
          // so scheduled Q6_K needs 145 VGPRs and runs three workgroups per CU (219, and two,
          // before), and 64 rows per wave fit 256 VGPRs without a spill.
          if ((FMT == 1 || NT == 2) && hi == 0) __builtin_amdgcn_sched_barrier(0);
        }
        // Stage s + 1 has landed (for every wave, after the barrier) once at most stages s + 2
        // and s + 3 (kDMA loads each) and the record loads that gemm32s_wait allows are
        // pending.
        switch (ls) {
          case 0: FHIP_LDS_BARRIER(wait_vm(gemm32s_wait(FMT, NT, 0, kDMA))); break;
          case 1: FHIP_LDS_BARRIER(wait_vm(gemm32s_wait(FMT, NT, 1, kDMA))); break;
          case 2: FHIP_LDS_BARRIER(wait_vm(gemm32s_wait(FMT, NT, 2, kDMA))); break;
          case 3: FHIP_LDS_BARRIER(wait_vm(gemm32s_wait(FMT, NT, 3, kDMA))); break;
          case 4: FHIP_LDS_BARRIER(wait_vm(gemm32s_wait(FMT, NT, 4, kDMA))); break;
          case 5: FHIP_LDS_BARRIER(wait_vm(gemm32s_wait(FMT, NT, 5, kDMA))); break;
          case 6: FHIP_LDS_BARRIER(wait_vm(gemm32s_wait(FMT, NT, 6, kDMA))); break;
          default: FHIP_LDS_BARRIER(wait_vm(gemm32s_wait(FMT, NT, 7, kDMA))); break;
        }
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(wait_vm(0));  // no LDS DMA may be pending when the workgroup ends

  // D layout: lane (kap, rho) holds column rho (the row o) and tokens 8 (v / 4) + 4 kap + v % 4.
  // The token scales come from LDS, four per read: a global load per output would make every
  // store wait for the previous one.
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int tl0 = 32 * i + 4 * kap, t0 = kBM * mg + tl0;
    float sc[16];
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      const float4 s4 = *reinterpret_cast<const float4 *>(ts_lds + tl0 + 8 * a);
      sc[4 * a] = s4.x; sc[4 * a + 1] = s4.y; sc[4 * a + 2] = s4.z; sc[4 * a + 3] = s4.w;
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int o = 16 * (kBTn * ng + 2 * NT * wave + 2 * t) + rho;
      if (o >= N) continue;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int tok = t0 + 8 * (v >> 2) + (v & 3);
        if (tok >= M) continue;
        const float val = acc[i][t][v] * sc[v];
        if (sp == 0)
          Y[(size_t)tok * N + o] = val;
        else
          part[((size_t)(sp - 1) * R + (task - F)) * (kBM * kRT) + (tok - kBM * mg) * kRT +
               (o - kRT * ng)] = val;
      }
    }
  }
}
#undef FHIP_LDS_BARRIER


// Y += the partial sums of K ranges 1 .. S-1 of the R split tiles (tasks F .. F+R-1), added in
// range order after range 0, which the GEMM wrote to Y (deterministic). part holds 128 x RT
// f32 per (range, tile), token-major (RT: the workgroup tile's rows, 128 or 256). Each thread
// adds four outputs of one token row.
template <int RT>
__global__ __launch_bounds__(256) void gemm32_reduce_kernel(const float *__restrict__ part,
                                                            float *__restrict__ Y, int N, int M,
                                                            int MTG, int F, int S, int R) {
  constexpr int kQuads = kBM * RT / 4;
  const long long id = (long long)blockIdx.x * 256 + threadIdx.x;
  if (id >= (long long)R * kQuads) return;
  const int r = (int)(id / kQuads), e4 = (int)(id - (long long)r * kQuads);
  const int task = F + r, mg = task % MTG, ng = task / MTG;
  const int tok = kBM * mg + e4 / (RT / 4), o0 = RT * ng + 4 * (e4 % (RT / 4));
  if (tok >= M || o0 >= N) return;
  // Range s (1 .. S-1) of this tile's quad: part + ((s - 1) R + r) kQuads + e4.
  const float4 *pp = reinterpret_cast<const float4 *>(part) + (size_t)r * kQuads + e4;
  float *y = Y + (size_t)tok * N + o0;
  const size_t stride = (size_t)R * kQuads;
  if ((N & 3) == 0 && ((uintptr_t)Y & 15) == 0) {
    // the quad is 16-byte aligned and whole: one load and one store of Y
    float4 *y4 = reinterpret_cast<float4 *>(y);
    *y4 = add_ranges(*y4, pp, stride, S - 1);
    return;
  }
  const int nv = min(4, N - o0);
  float4 v0;
  v0.x = y[0];
  v0.y = nv > 1 ? y[1] : 0.f;
  v0.z = nv > 2 ? y[2] : 0.f;
  v0.w = nv > 3 ? y[3] : 0.f;
  const float4 v = add_ranges(v0, pp, stride, S - 1);
  y[0] = v.x;
  if (nv > 1) y[1] = v.y;
  if (nv > 2) y[2] = v.z;
  if (nv > 3) y[3] = v.w;
}

}  // namespace

namespace {

// Launch plan of one GEMM call: form, K split and the scratch it needs (activation operands,
// token scales, then the K-range partial results).
struct GemmPlan {
  int MTG, tasks, form, F, S, R;  // tile tasks; F whole, then R split into S K ranges each
  int nt;                         // 32-row MFMA tiles per wave: 1 (128-row tiles) or 2 (256)
  size_t xab, tsb, pb;
};

GemmPlan plan_gemm32(int fmt, int N, int K, int M) {
  GemmPlan p{};
  const int nblk = K / 256;
  p.MTG = ceil_div(M, kBM);
  // FAK_HIP_GEMM32_FORM=1: the four-wave 2x2 kernel (a comparison; it agrees bit for bit with
  // the default without a K split). Default: the staged kernel, measured faster from 64 to 2048
  // tokens.
  p.form = tuning().gemm32_form;
  const int cus = cu_count() > 0 ? cu_count() : 256;
  // The staged kernel from eight token tiles (M > 896) takes 256-row workgroups (four waves of
  // 64 rows, two workgroups per CU): each staged activation byte then feeds twice the MFMAs.
  // One MI355X, Q4_K gate/up shape, M = 1024 / 2048 / 4096: 175-178 / 320 / 582 us against
  // 181-183 / 333-337 / 618-621 with 128-row tiles; the down shape at M=2048 361 against 371;
  // Q6_K gate/up at M = 1024 / 2048 207-210 / 374 against 215 / 381, down 231 / 413 against
  // 242 / 440. With fewer token tiles the uneven spread of fewer, larger tiles costs more
  // (M=512: Q4_K gate/up 100-103 against 96, down 117 against 112). FAK_HIP_GEMM32_NT=1 / 2
  // forces the choice.
  p.nt = 1;
  if (p.form != 1) {
    if (tuning().gemm32_nt == 1 || tuning().gemm32_nt == 2)
      p.nt = tuning().gemm32_nt;
    else if (tuning().gemm32_sk <= 0 && p.MTG >= 8)
      p.nt = 2;
  }
  p.tasks = p.MTG * ceil_div(q4k_tiles(N), kBT * p.nt);
  p.F = p.tasks;
  p.S = 1;
  p.R = 0;
  {  // every form and format (the 2x2 form takes the same ranges, so the forms stay bit-identical)
    // K splits (partial sums added in range order), for both forms: without them the 2x2 form
    // ran a 3584 x 18944 Q6_K down projection on 28 workgroups at 64..128 tokens (315 us, 55-60
    // with the split):
    //  * a grid smaller than the GPU (the 3584-row down projection, or 128 tokens) splits every
    //    tile into as many ranges as keep the grid within two workgroups per CU (at least 4
    //    super-blocks each): a third workgroup on some CUs sets the time (down projection at
    //    M=512: 4 ranges 116 us, 5 ranges 128 us; 27B gate/up at M=128: 2 ranges 62 us, 3: 66);
    //  * a larger grid runs whole tiles in rounds of one per CU and splits only the tiles of
    //    the last, partial round, so that every CU gets the same whole tiles plus at most one
    //    range (M=512 on the gate/up shape: 512 whole tiles and 80 tiles in 3 ranges, where 80
    //    CUs ran a third whole tile; ranges of at least 2 super-blocks);
    //  * FAK_HIP_GEMM32_SK=n splits every tile in n (1: no split).
    const int sk = tuning().gemm32_sk;
    int S = 1, R = 0;
    if (sk > 0) {
      S = min(sk, nblk);
      R = p.tasks;
    } else if (p.tasks < cus) {
      S = min(2 * cus / p.tasks, nblk / 4);
      R = p.tasks;
    } else if (p.tasks % cus) {
      R = p.tasks % cus;
      S = min(cus / R, nblk / 2);
    }
    if (S > 1) {
      p.S = S;
      p.R = R;
      p.F = p.tasks - R;
    }
  }
  p.xab = ((size_t)p.MTG * kBM * K * 2 + 255) & ~(size_t)255;
  p.tsb = ((size_t)p.MTG * kBM * 4 + 255) & ~(size_t)255;
  p.pb = p.R ? (size_t)(p.S - 1) * p.R * kTileElems * p.nt * 4 : 0;
  return p;
}

int launch_gemm32(int fmt, const void *Wv, const float *X, float *Y, int N, int K, int M) {
  const int nblk = K / 256;
  const int ntiles = q4k_tiles(N);
  const GemmPlan p = plan_gemm32(fmt, N, K, M);
  const int MTG = p.MTG;
  unsigned char *ws = (unsigned char *)workspace(p.xab + p.tsb + p.pb);
  if (!ws) return FHIP_ENOMEM;
  if (int rc = check_disjoint("gemm32", X, (size_t)M * K * 4, ws, p.xab + p.tsb + p.pb)) return rc;
  uint4 *xa = (uint4 *)ws;
  float *ts = (float *)(ws + p.xab);
  float *part = p.R ? (float *)(ws + p.xab + p.tsb) : nullptr;
  launch_xprep(X, M, K, MTG, xa, ts);
  FHIP_CHECK_LAUNCH("gemm32_xprep_kernel");
  const uint8_t *W = (const uint8_t *)Wv;
  auto reduce = [&]() -> int {
    if (p.R) {
      const long long quads = (long long)p.R * (kTileElems * p.nt / 4);
      if (p.nt == 2)
        gemm32_reduce_kernel<256><<<(unsigned)((quads + 255) / 256), 256, 0, stream()>>>(
            part, Y, N, M, MTG, p.F, p.S, p.R);
      else
        gemm32_reduce_kernel<128><<<(unsigned)((quads + 255) / 256), 256, 0, stream()>>>(
            part, Y, N, M, MTG, p.F, p.S, p.R);
      FHIP_CHECK_LAUNCH("gemm32_reduce_kernel");
    }
    return FHIP_OK;
  };
  const int grid2 = p.F + p.R * p.S;
  if (fmt == 1 && p.form != 1) {
    if (p.nt == 2)
      quant_gemm32s_kernel<1, 2, 2><<<grid2, 64 * kGemmWaves, 0, stream()>>>(
          W, xa, ts, Y, N, M, nblk, ntiles, MTG, p.F, p.S, p.R, part);
    else
      quant_gemm32s_kernel<1, 3, 1><<<grid2, 64 * kGemmWaves, 0, stream()>>>(
          W, xa, ts, Y, N, M, nblk, ntiles, MTG, p.F, p.S, p.R, part);
    FHIP_CHECK_LAUNCH("quant_gemm32s_kernel<1>");
    return reduce();
  }
  if (fmt == 1) {  // 60 KB of LDS with one weight buffer: two workgroups per CU
    quant_gemm32_kernel<1, 1, 2><<<grid2, 256, 0, stream()>>>(W, xa, ts, Y, N, M, nblk, ntiles,
                                                               MTG, p.F, p.S, p.R, part);
    FHIP_CHECK_LAUNCH("quant_gemm32_kernel");
    return reduce();
  }
  if (p.form != 1) {
    if (p.nt == 2)
      quant_gemm32s_kernel<0, 2, 2><<<grid2, 64 * kGemmWaves, 0, stream()>>>(
          W, xa, ts, Y, N, M, nblk, ntiles, MTG, p.F, p.S, p.R, part);
    else
      quant_gemm32s_kernel<0, 3, 1><<<grid2, 64 * kGemmWaves, 0, stream()>>>(
          W, xa, ts, Y, N, M, nblk, ntiles, MTG, p.F, p.S, p.R, part);
    FHIP_CHECK_LAUNCH("quant_gemm32s_kernel<0>");
    return reduce();
  }
  if (tuning().gemm32_nwb == 2)
    quant_gemm32_kernel<0, 2, 2><<<grid2, 256, 0, stream()>>>(W, xa, ts, Y, N, M, nblk, ntiles,
                                                               MTG, p.F, p.S, p.R, part);
  else
    quant_gemm32_kernel<0, 1, 3><<<grid2, 256, 0, stream()>>>(W, xa, ts, Y, N, M, nblk, ntiles,
                                                               MTG, p.F, p.S, p.R, part);
  FHIP_CHECK_LAUNCH("quant_gemm32_kernel");
  return reduce();
}
}  // namespace

size_t gemm32_ws_bytes(int fmt, int N, int K, int M) {
  const GemmPlan p = plan_gemm32(fmt, N, K, M);
  return p.xab + p.tsb + p.pb;
}

int q4k_gemm32(const void *Wv, const float *X, float *Y, int N, int K, int M) {
  return launch_gemm32(0, Wv, X, Y, N, K, M);
}

int q6k_gemm32(const void *Wv, const float *X, float *Y, int N, int K, int M) {
  return launch_gemm32(1, Wv, X, Y, N, K, M);
}

}  // namespace fhip
