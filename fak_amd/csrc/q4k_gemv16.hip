// q4k_gemv16.hip — Q4_K (and Q6_K) matmul for 5..16 tokens (speculative verify) on the
// 32x32x16 f16 MFMA.
//
// Y[t][o] = sum_k W[o][k] X[t][k] with W the Q4_K weight (w = d*sc_s*n - dmin*m_s per 32-weight
// sub-block s, internal/model/quant_q4k.go:90-111). Per super-block b of row o and token t
//   sum_k w x = d * sum_s sc_s * (sum_{k in s} n_k x_k)  -  dmin * sum_s m_s * S_s,
// S_s = sum_{k in s} x_k. Both sums run on the MFMA with exact operands:
//   * weight operand: the integer sc_s * n_k (<= 63 * 15 = 945), exact in f16, made from a
//     nibble pair with one and-or and one packed fma: (1024 + n) * sc - 1024 * sc, or for the
//     high nibbles masked in place (1024 + 16 n) * (sc / 16) - 64 * sc. The fma rounds once and
//     the result is an integer below 2048, so it is exact;
//   * activation operand: 32 operand rows, the f16 of v = x / s_t (rows 0..15 = tokens 0..15) and
//     the f16 of the remainder v - f16(v) (rows 16..31), so the products carry ~22 bits of x.
//     s_t is a power of two per (token, K range of the workgroup) that puts the range's largest
//     magnitude in [2^13, 2^14): any finite f32 activation becomes f16 operands without overflow
//     and with full precision down to 2^-28 of the range's maximum;
//   * the min term is one more MFMA per super-block: activation rows S_s / 32 (hi and lo parts;
//     S_s / 32 <= 2^14), weight columns 32 * m_s.
// The f32 result of a super-block is scaled by d and dmin of the lane's row and accumulated; the
// hi and lo rows of a token are added at the end and multiplied by s_t (exact). A range holding a
// NaN or an infinity gets s_t = NaN, which reaches every output of that token.
//
// Work split: a workgroup = 4 waves x 64 rows (16 tiled records of 16 rows) over one K range of
// the weight; K is split into SK ranges of about 4 super-blocks across workgroups, and a second
// kernel adds the SK partial results in range order (deterministic). Each wave streams its 4
// records per super-block straight into registers (two super-blocks in flight). The workgroup
// builds the activation operands of each super-block itself, one super-block ahead, from X
// (16 KB of f32, L2-resident) into an LDS stage shared by its 4 waves: no separate prep launch.
//
// Q6_K weights (w = d * sc_g * (q - 32) per 16-weight group g, internal/model/quant_kquant.go
// :139-163) run the same kernel with one 32-row tile per wave (their records need more
// registers): the K16 slice g of a super-block is group g, the integer sc_g * (q - 32) (up to
// 4096 in magnitude, more than f16 holds exactly) is the sum of two exact f16 operands, f16 of
// it and the remainder, fed to two MFMAs; there is no min term, and the f32 result of a
// super-block is scaled by d.
#include "kernels.hpp"

namespace fhip {
namespace {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ h2 as_h2(uint32_t u) { return __builtin_bit_cast(h2, u); }
__device__ __forceinline__ uint32_t as_u(h2 v) { return __builtin_bit_cast(uint32_t, v); }


// LDS stage of one super-block b: 17 units of 64 lanes x 16 B.
//   unit s < 16, lane l: 8 f16 of operand row v = l & 31 at K = 256 b + 16 s + 8 (l >> 5) +
//     perm8(j): the f16 of x[v] / s_v for v < 16, of the remainder of x[v - 16] / s_{v - 16}
//     for v >= 16;
//   unit 16, lane l < 32: element j = the hi (v < 16) or lo part of S[t][perm8(j)] / 32, the f32
//     sum of the scaled sub-block perm8(j) of b; lanes >= 32 zero.
// Tokens >= M are zero (scale 1).
constexpr int kUnitsSB = 17;

// s_waitcnt immediate for vmcnt(n) with lgkmcnt(0); see q4k_gemm32.hip for the bare barrier.
constexpr int wait_vm16(int n) { return 0x0070 | (n & 15) | ((n >> 4) << 14); }
#define FHIP_LDS_BARRIER16(imm)      \
  do {                               \
    __builtin_amdgcn_s_waitcnt(imm); \
    asm volatile("" ::: "memory");   \
    __builtin_amdgcn_s_barrier();    \
    asm volatile("" ::: "memory");   \
  } while (0)

// 32-row MFMA tiles per wave: two for Q4_K, one for Q6_K (its records need more registers).
template <int FMT>
constexpr int tiles16() { return FMT == 0 ? 2 : 1; }

// One super-block's weight data of a lane.
// Q4_K (two 32-row MFMA tiles per wave): per tile the 16-byte header of the lane's row and the
// four 16-byte nibble units it takes operands from.
// Q6_K (one tile per wave): the row's 16 int8 scales, its d, and for each K half hh and lane
// group h the 8 ql bytes of groups 4c + h and 4c + 2 + h (c = 2 hh, 2 hh + 1: low and high
// nibble) and their 8 qh bytes.
template <int FMT>
struct W16;
template <>
struct W16<0> {
  uint4 hd[2];
  uint4 nb[2][2][2];  // [tile][K half hh][lane group h]
};
template <>
struct W16<1> {
  uint4 sc;
  uint32_t d;
  uint2 q[2][2][3];  // [K half hh][lane group h][ql a, ql b, qh]
};

// T32 (17..32 tokens): the 32 operand rows are 32 tokens, each the f16 of x / s_t with no
// remainder row (the prefill GEMM's activation precision), the Q4_K min term's rows S_s / 32 in
// f16; one 32-row tile per wave (for Q4_K the second token's staging registers leave no room for
// two; Q6_K always runs one).
template <int FMT, bool T32>  // FMT 0: Q4_K, 1: Q6_K
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void quant_gemv16_kernel(
    const uint8_t *__restrict__ W, const float *__restrict__ X, float *__restrict__ Y,
    float *__restrict__ part, int N, int K, int M, int nblk, int ntiles, int SK) {
  // Two stage buffers: the one being read and the one being built.
  __shared__ u32x4 As0[kUnitsSB * 64];
  __shared__ u32x4 As1[kUnitsSB * 64];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kap = lane >> 5, rho = lane & 31, r16 = rho & 15;
  const int rb = blockIdx.x / SK, sp = blockIdx.x - rb * SK;
  const int kb0 = sp * nblk / SK, kb1 = (sp + 1) * nblk / SK;  // >= 1 super-block: SK <= nblk
  const int nb = kb1 - kb0;
  constexpr int NT = T32 ? 1 : tiles16<FMT>();    // 32-row MFMA tiles per wave
  constexpr int TWG = 8 * NT;                      // 16-row tiles per workgroup
  constexpr int kRec = FMT == 0 ? kQ4kRecord : kQ6kRecord;
  constexpr int kWL = FMT == 0 ? 10 : 14;          // record loads per super-block per lane
  // This lane's row tiles (row rho of a 32-row MFMA tile = row rho % 16 of 16-row tile
  // rho / 16); loads use the last tile in place of ones past the end.
  auto tile_of = [&](int t) { return TWG * rb + 2 * NT * wave + 2 * t + (rho >> 4); };
  const uint8_t *rec[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t)
    rec[t] = W + (size_t)min(tile_of(t), ntiles - 1) * nblk * kRec;
  auto load_w = [&](int b, W16<FMT> &o) {
    if constexpr (FMT == 0) {
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const uint8_t *r = rec[t] + (size_t)b * kRec;
        o.hd[t] = *reinterpret_cast<const uint4 *>(r + 16 * r16);
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
          for (int h = 0; h < 2; ++h)
            o.nb[t][hh][h] = *reinterpret_cast<const uint4 *>(r + kQ4kHdr + 1024 * hh +
                                                              16 * (16 * (2 * h + kap) + r16));
      }
    } else {
      const uint8_t *r = rec[0] + (size_t)b * kRec;
      o.sc = *reinterpret_cast<const uint4 *>(r + 16 * r16);
      o.d = *reinterpret_cast<const uint16_t *>(r + kQ6kD + 2 * r16);
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          o.q[hh][h][0] = *reinterpret_cast<const uint2 *>(r + kQ6kQl + 1024 * hh +
                                                           16 * (16 * h + r16) + 8 * kap);
          o.q[hh][h][1] = *reinterpret_cast<const uint2 *>(r + kQ6kQl + 1024 * hh +
                                                           16 * (16 * (2 + h) + r16) + 8 * kap);
          o.q[hh][h][2] = *reinterpret_cast<const uint2 *>(r + kQ6kQh + 512 * hh + 256 * h +
                                                           16 * r16 + 8 * kap);
        }
    }
  };
  // Stage building: thread (t, sb, half) = tid (16 x 8 x 2) owns the 16 activations of token t
  // at K = 256 b + 32 sb + 16 half (two 8-runs). The loads go out at the start of a pass and are
  // turned into operands at its end, after the MFMA work.
  const int xt = tid >> 4, xsb = (tid >> 1) & 7, xhalf = tid & 1;
  const bool xvalid = xt < M;
  const float4 *xrow = reinterpret_cast<const float4 *>(X + (size_t)(xvalid ? xt : 0) * K +
                                                        32 * xsb + 16 * xhalf);
  // T32: the thread also stages token xt + 16 (operand row 16 + xt).
  const bool xvalid1 = T32 && xt + 16 < M;
  const float4 *xrow1 = reinterpret_cast<const float4 *>(X + (size_t)(xvalid1 ? xt + 16 : 0) * K +
                                                         32 * xsb + 16 * xhalf);
  constexpr int XV = T32 ? 8 : 4;  // float4 of activations per thread per super-block
  // Unconditional loads (tokens past M read token 0's row; store_x zeroes them): a load under
  // the token test sits in an exec-masked branch, and the merge after it made the compiler wait
  // for every load in flight, the records of the next super-block included.
  auto load_x = [&](int b, float4 (&xv)[XV]) {
#pragma unroll
    for (int q = 0; q < 4; ++q) xv[q] = xrow[64 * (size_t)b + q];
    if constexpr (T32) {
#pragma unroll
      for (int q = 0; q < 4; ++q) xv[4 + q] = xrow1[64 * (size_t)b + q];
    }
  };
  // sk: the token's range scale exponent (0 for a range holding a NaN or an infinity: those
  // values reach the token's own operand rows only, and so only its outputs)
  // T32: both tokens' values as f16 rows xt and 16 + xt, sub-block sums S / 32 as f16 (the
  // half-0 thread writes token xt's, the half-1 thread token xt + 16's).
  auto store_x32 = [&](float4 (&xv)[XV], u32x4 *dst, int sk0, int sk1) {
    float ps[2];
#pragma unroll
    for (int tk = 0; tk < 2; ++tk) {
      const bool ok = tk ? xvalid1 : xvalid;
      const int sk = tk ? sk1 : sk0;
      float f[16];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float4 w = xv[4 * tk + q];
        f[4 * q] = ok ? ldexpf(w.x, -sk) : 0.f;
        f[4 * q + 1] = ok ? ldexpf(w.y, -sk) : 0.f;
        f[4 * q + 2] = ok ? ldexpf(w.z, -sk) : 0.f;
        f[4 * q + 3] = ok ? ldexpf(w.w, -sk) : 0.f;
      }
      ps[tk] = 0.f;
#pragma unroll
      for (int k = 0; k < 16; ++k) ps[tk] += f[k];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        f16x8 hv;
#pragma unroll
        for (int j = 0; j < 8; ++j) hv[j] = (_Float16)f[8 * i + perm8(j)];
        u32x4 *unit = dst + (2 * xsb + xhalf) * 64 + 32 * i;
        unit[16 * tk + xt] = __builtin_bit_cast(u32x4, hv);
      }
    }
    const float o0 = __shfl_xor(ps[0], 1), o1 = __shfl_xor(ps[1], 1);
    const float S0 = (xhalf ? o0 + ps[0] : ps[0] + o0) * 0.03125f;
    const float S1 = (xhalf ? o1 + ps[1] : ps[1] + o1) * 0.03125f;
    _Float16 *su = reinterpret_cast<_Float16 *>(dst + 16 * 64);
    const int j = perm8(xsb);
    if (xhalf == 0)
      su[xt * 8 + j] = (_Float16)S0;
    else
      su[(16 + xt) * 8 + j] = (_Float16)S1;
  };
  auto store_x = [&](float4 (&xv)[XV], u32x4 *dst, int sk) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      xv[q].x = xvalid ? ldexpf(xv[q].x, -sk) : 0.f;
      xv[q].y = xvalid ? ldexpf(xv[q].y, -sk) : 0.f;
      xv[q].z = xvalid ? ldexpf(xv[q].z, -sk) : 0.f;
      xv[q].w = xvalid ? ldexpf(xv[q].w, -sk) : 0.f;
    }
    const float f[16] = {xv[0].x, xv[0].y, xv[0].z, xv[0].w, xv[1].x, xv[1].y, xv[1].z, xv[1].w,
                         xv[2].x, xv[2].y, xv[2].z, xv[2].w, xv[3].x, xv[3].y, xv[3].z, xv[3].w};
    float ps = 0.f;
#pragma unroll
    for (int k = 0; k < 16; ++k) ps += f[k];
#pragma unroll
    for (int i = 0; i < 2; ++i) {  // 8-run i: K16 slice 2 xsb + xhalf, lane group i
      f16x8 hv, lv;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float xv1 = f[8 * i + perm8(j)];
        const _Float16 hi = (_Float16)xv1;
        hv[j] = hi;
        lv[j] = (_Float16)(xv1 - (float)hi);
      }
      u32x4 *unit = dst + (2 * xsb + xhalf) * 64 + 32 * i;
      unit[xt] = __builtin_bit_cast(u32x4, hv);
      unit[16 + xt] = __builtin_bit_cast(u32x4, lv);
    }
    // Sub-block sum = the two halves' partial sums (neighbour lanes), in half order.
    const float other = __shfl_xor(ps, 1);
    const float S = (xhalf ? other + ps : ps + other) * 0.03125f;  // exact: a power of two
    const _Float16 Sh = (_Float16)S;
    _Float16 *su = reinterpret_cast<_Float16 *>(dst + 16 * 64);
    const int j = perm8(xsb);  // perm8 is its own inverse
    if (xhalf == 0)
      su[xt * 8 + j] = Sh;
    else
      su[(16 + xt) * 8 + j] = (_Float16)(S - (float)Sh);
  };
  auto buf = [&](int k) -> u32x4 * { return k == 0 ? As0 : As1; };

  const uint32_t kLo = in_reg(0x000F000Fu), kHi = in_reg(0x00F000F0u);
  const uint32_t kMagic = in_reg(0x64006400u), kB02 = in_reg(0x00FF00FFu);
  const h2 k1024 = {(_Float16)1024.f, (_Float16)1024.f};
  const h2 kN1024 = {(_Float16)-1024.f, (_Float16)-1024.f};
  const h2 k16th = {(_Float16)0.0625f, (_Float16)0.0625f};
  const h2 k32 = {(_Float16)32.f, (_Float16)32.f};
  const h2 k1056 = {(_Float16)1056.f, (_Float16)1056.f};
  const uint32_t k0F = in_reg(0x0F0F0F0Fu), k03 = in_reg(0x03030303u);

  f32x16 acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[t][e] = 0.f;

  W16<FMT> wr[2];
  float4 xv[XV];
  // Largest magnitude bit pattern of token tk's four float4 (tk = 1: the second token of T32).
  auto absmax = [](uint32_t m, const float4 (&v)[XV], int tk = 0) {
#pragma unroll
    for (int q = 0; q < 4; ++q)
      m = max(max(max(m, __float_as_uint(v[4 * tk + q].x) & 0x7FFFFFFFu),
                  __float_as_uint(v[4 * tk + q].y) & 0x7FFFFFFFu),
              max(__float_as_uint(v[4 * tk + q].z) & 0x7FFFFFFFu,
                  __float_as_uint(v[4 * tk + q].w) & 0x7FFFFFFFu));
    return m;
  };
  // Vector loads complete in issue order per CU: activation loads issued behind the first
  // records land only when the records of every wave on the CU have. So a range of at most kPre
  // super-blocks loads all its activations first (kept in registers for the range scale and the
  // first stage), and a bare barrier holds every wave's records behind every wave's activation
  // loads; longer ranges read them after the records.
  constexpr int kPre = 5;
  const bool xfirst = !T32 && nb <= kPre;  // uniform over the workgroup
  float4 xp[kPre][XV];
  if (xfirst) {
    // Straight-line (a range shorter than kPre repeats its last super-block, which leaves the
    // maximum unchanged), so the waits below count exactly.
#pragma unroll
    for (int j = 0; j < kPre; ++j) load_x(kb0 + min(j, nb - 1), xp[j]);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  }
  __builtin_amdgcn_sched_barrier(0);
  // The first two super-blocks' records stream in while the range scale below is worked out.
  load_w(kb0, wr[0]);
  load_w(min(kb0 + 1, kb1 - 1), wr[1]);
  if (xfirst) {
    // Empty asm on the held activations: the range scale computed from them cannot be hoisted
    // above the record loads (it would wait for the activations before any record went out).
#pragma unroll
    for (int j = 0; j < kPre; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) asm volatile("" : "+v"(xp[j][q].x), "+v"(xp[j][q].y), "+v"(xp[j][q].z), "+v"(xp[j][q].w));
  }
  // The token's largest magnitude over the K range, as the largest magnitude bit pattern (it
  // orders like the magnitudes; a NaN or an infinity makes it >= 0x7F800000): each stage lane
  // reads its 16 values of every super-block of the range, then the 16 lanes of the token
  // (adjacent: tid = 16 xt + ...) reduce with xor-swizzles (bit-mask mode, no address registers).
  uint32_t mb = 0, mb1 = 0;
  if (xfirst) {
#pragma unroll
    for (int j = 0; j < kPre; ++j) mb = absmax(mb, xp[j]);
  } else {
    for (int b = kb0; b < kb1; ++b) {
      load_x(b, xv);
      mb = absmax(mb, xv);
      if (T32) mb1 = absmax(mb1, xv, 1);
    }
  }
  auto token_max = [](uint32_t m) {
    m = max(m, (uint32_t)__builtin_amdgcn_ds_swizzle((int)m, (1 << 10) | 0x1F));
    m = max(m, (uint32_t)__builtin_amdgcn_ds_swizzle((int)m, (2 << 10) | 0x1F));
    m = max(m, (uint32_t)__builtin_amdgcn_ds_swizzle((int)m, (4 << 10) | 0x1F));
    m = max(m, (uint32_t)__builtin_amdgcn_ds_swizzle((int)m, (8 << 10) | 0x1F));
    return m;
  };
  // The range maximum / 2^sk is in [2^13, 2^14); a range holding a NaN or an infinity gets
  // sk = 0 and the scale NaN.
  auto range_exp = [](uint32_t m) {
    int e = 0;
    (void)frexpf(__uint_as_float(m), &e);
    return m < 0x7F800000u ? e - 14 : 0;
  };
  auto range_scale = [](uint32_t m, int sk) {
    return m >= 0x7F800000u ? __builtin_nanf("") : m ? ldexpf(1.f, sk) : 1.f;
  };
  mb = token_max(mb);
  const int xsk = range_exp(mb);
  __shared__ float tscale[T32 ? 32 : 16];
  if (xsb == 0 && xhalf == 0) tscale[xt] = range_scale(mb, xsk);
  int xsk1 = 0;
  if constexpr (T32) {
    mb1 = token_max(mb1);
    xsk1 = range_exp(mb1);
    if (xsb == 0 && xhalf == 0) tscale[16 + xt] = range_scale(mb1, xsk1);
  }
  if (xfirst) {
#pragma unroll
    for (int q = 0; q < 4; ++q) xv[q] = xp[0][q];
  } else {
    load_x(kb0, xv);
  }
  if (tid < 64) {  // lanes 32..63 of both S units: zero for the whole kernel
    const int k = tid & 31;
    (tid < 32 ? As0 : As1)[16 * 64 + 32 + k] = u32x4{0u, 0u, 0u, 0u};
  }
  if constexpr (T32)
    store_x32(xv, As0, xsk, xsk1);
  else
    store_x(xv, As0, xsk);
  // The first stage is in LDS; the first two super-blocks' records (2 kWL loads per lane) may
  // still be in flight: the first pass waits for its own.
  if (xfirst)
    FHIP_LDS_BARRIER16(wait_vm16(2 * kWL));
  else
    FHIP_LDS_BARRIER16(wait_vm16(0));

  // Passes of two super-blocks (stage buffer and weight slot u are compile-time). Every pass
  // issues the same loads (indices clamped) and reaches the same barrier; a pass past the end of
  // the range computes on its clamped copy with d = dmin = 0, so the loop has no branch and
  // each wait below is an exact count.
  const int nbp = (nb + 1) & ~1;
  for (int i0 = 0; i0 < nbp; i0 += 2) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int i = i0 + u;
      const int b = kb0 + i;
      // This slot's records (issued two passes ago) are older than the kWL loads of the other
      // slot: the wait makes that explicit for the compiler, which otherwise drains everything.
      __builtin_amdgcn_s_waitcnt(wait_vm16(kWL));
      load_x(min(b + 1, kb1 - 1), xv);
      const u32x4 *Ab = buf(u);
      W16<FMT> &cw = wr[u];
      const float live = i < nb ? 1.f : 0.f;
      if constexpr (FMT == 0) {
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const uint4 hd = cw.hd[t];
        const float d = live * (float)__builtin_bit_cast(_Float16, (uint16_t)(hd.x & 0xffffu));
        const float dm = live * (float)__builtin_bit_cast(_Float16, (uint16_t)(hd.x >> 16));
        const uint32_t scl = hd.y & 0x3F3F3F3Fu, mnl = hd.z & 0x3F3F3F3Fu;
        const uint32_t sch = (hd.w & 0x0F0F0F0Fu) | ((hd.y >> 2) & 0x30303030u);
        const uint32_t mnh = ((hd.w >> 4) & 0x0F0F0F0Fu) | ((hd.z >> 2) & 0x30303030u);
        // (sc_0, sc_2), (sc_1, sc_3), (sc_4, sc_6), (sc_5, sc_7) as exact f16 pairs.
        const h2 e0 = as_h2((scl & kB02) | kMagic) - k1024;
        const h2 o0 = as_h2(((scl >> 8) & kB02) | kMagic) - k1024;
        const h2 e1 = as_h2((sch & kB02) | kMagic) - k1024;
        const h2 o1 = as_h2(((sch >> 8) & kB02) | kMagic) - k1024;
        // Min operand: element j = 32 m_perm8(j) (every lane: the activation S unit is zero in
        // the lanes of K half 1, so those products vanish).
        u32x4 mw;
        mw[0] = as_u((as_h2((mnl & kB02) | kMagic) - k1024) * k32);
        mw[1] = as_u((as_h2(((mnl >> 8) & kB02) | kMagic) - k1024) * k32);
        mw[2] = as_u((as_h2((mnh & kB02) | kMagic) - k1024) * k32);
        mw[3] = as_u((as_h2(((mnh >> 8) & kB02) | kMagic) - k1024) * k32);

        f32x16 tmp;
#pragma unroll
        for (int e = 0; e < 16; ++e) tmp[e] = 0.f;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const h2 ep = c < 2 ? e0 : e1, op = c < 2 ? o0 : o1;
          const _Float16 sa = (c & 1) ? ep.y : ep.x;  // sc of sub-block 2c (low nibbles)
          const _Float16 sb = (c & 1) ? op.y : op.x;  // sc of sub-block 2c + 1 (high nibbles)
          const h2 SL = {sa, sa}, SH = h2{sb, sb} * k16th;
          const h2 NL = SL * kN1024, NH = SH * kN1024;
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const uint4 q = cw.nb[t][c >> 1][h];
            const uint32_t x0 = (c & 1) ? q.z : q.x, x1 = (c & 1) ? q.w : q.y;
            const uint32_t y0 = x0 >> 8, y1 = x1 >> 8;
            u32x4 lw, hw;
            lw[0] = as_u(__builtin_elementwise_fma(as_h2((x0 & kLo) | kMagic), SL, NL));
            lw[1] = as_u(__builtin_elementwise_fma(as_h2((y0 & kLo) | kMagic), SL, NL));
            lw[2] = as_u(__builtin_elementwise_fma(as_h2((x1 & kLo) | kMagic), SL, NL));
            lw[3] = as_u(__builtin_elementwise_fma(as_h2((y1 & kLo) | kMagic), SL, NL));
            hw[0] = as_u(__builtin_elementwise_fma(as_h2((x0 & kHi) | kMagic), SH, NH));
            hw[1] = as_u(__builtin_elementwise_fma(as_h2((y0 & kHi) | kMagic), SH, NH));
            hw[2] = as_u(__builtin_elementwise_fma(as_h2((x1 & kHi) | kMagic), SH, NH));
            hw[3] = as_u(__builtin_elementwise_fma(as_h2((y1 & kHi) | kMagic), SH, NH));
            const f16x8 bl = __builtin_bit_cast(f16x8, lw), bh = __builtin_bit_cast(f16x8, hw);
#pragma unroll
            for (int hi = 0; hi < 2; ++hi) {
              const f16x8 a = __builtin_bit_cast(f16x8, Ab[(4 * c + 2 * hi + h) * 64 + lane]);
              tmp = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, hi ? bh : bl, tmp, 0, 0, 0);
            }
          }
        }
        f32x16 mt;
#pragma unroll
        for (int e = 0; e < 16; ++e) mt[e] = 0.f;
        mt = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, Ab[16 * 64 + lane]),
                                                    __builtin_bit_cast(f16x8, mw), mt, 0, 0, 0);
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[t][e] = fmaf(d, tmp[e], fmaf(-dm, mt[e], acc[t][e]));
      }
      } else {
        // Q6_K: w = d * sc_g * (q - 32) per 16-weight group g = K16 slice g. The integer
        // sc_g * (q - 32) (up to 4096 in magnitude) goes in as two exact f16 operands; the f32
        // result of the super-block is scaled by d.
        const float d = live * (float)__builtin_bit_cast(_Float16, (uint16_t)(cw.d & 0xffffu));
        const uint32_t scv[4] = {cw.sc.x, cw.sc.y, cw.sc.z, cw.sc.w};
        f32x16 tmp;
#pragma unroll
        for (int e = 0; e < 16; ++e) tmp[e] = 0.f;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const int k = c & 1;  // nibble of ql, qh fields 4k (slice a) and 4k + 2 (slice b)
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const _Float16 sa = (_Float16)(float)(int8_t)(scv[c] >> (8 * h));
            const _Float16 sb = (_Float16)(float)(int8_t)(scv[c] >> (8 * (2 + h)));
            const h2 SA = {sa, sa}, SB = {sb, sb};
            const uint2 qa = cw.q[c >> 1][h][0], qb = cw.q[c >> 1][h][1], qh = cw.q[c >> 1][h][2];
            const uint32_t qav[2] = {qa.x, qa.y}, qbv[2] = {qb.x, qb.y}, qhv[2] = {qh.x, qh.y};
            // Operand = v_hi + v_lo with v = sc * (q - 32): v_hi = f16(v) and v_lo = v - v_hi
            // (0 or +-1, from one fma with the exact product), so the pair is exact.
            u32x4 ra, rbw, la, lbw;
#pragma unroll
            for (int m = 0; m < 2; ++m) {
              const uint32_t ca = ((qav[m] >> (4 * k)) & k0F) | (((qhv[m] >> (4 * k)) & k03) << 4);
              const uint32_t cb =
                  ((qbv[m] >> (4 * k)) & k0F) | (((qhv[m] >> (4 * k + 2)) & k03) << 4);
              // bytes (0, 2) and (1, 3) of each code word: elements in perm8 order
              const h2 qa0 = as_h2((ca & kB02) | kMagic) - k1056;
              const h2 qa1 = as_h2(((ca >> 8) & kB02) | kMagic) - k1056;
              const h2 qb0 = as_h2((cb & kB02) | kMagic) - k1056;
              const h2 qb1 = as_h2(((cb >> 8) & kB02) | kMagic) - k1056;
              const h2 va0 = qa0 * SA, va1 = qa1 * SA, vb0 = qb0 * SB, vb1 = qb1 * SB;
              ra[2 * m] = as_u(va0);
              ra[2 * m + 1] = as_u(va1);
              rbw[2 * m] = as_u(vb0);
              rbw[2 * m + 1] = as_u(vb1);
              la[2 * m] = as_u(__builtin_elementwise_fma(qa0, SA, -va0));
              la[2 * m + 1] = as_u(__builtin_elementwise_fma(qa1, SA, -va1));
              lbw[2 * m] = as_u(__builtin_elementwise_fma(qb0, SB, -vb0));
              lbw[2 * m + 1] = as_u(__builtin_elementwise_fma(qb1, SB, -vb1));
            }
#pragma unroll
            for (int hi = 0; hi < 2; ++hi) {
              const f16x8 a = __builtin_bit_cast(f16x8, Ab[(4 * c + 2 * hi + h) * 64 + lane]);
              tmp = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                  a, __builtin_bit_cast(f16x8, hi ? rbw : ra), tmp, 0, 0, 0);
              tmp = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                  a, __builtin_bit_cast(f16x8, hi ? lbw : la), tmp, 0, 0, 0);
            }
          }
        }
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[0][e] = fmaf(d, tmp[e], acc[0][e]);
      }
      load_w(min(b + 2, kb1 - 1), cw);
      // The activations of b + 1 have landed once at most kWL of this wave's later loads (the
      // records of b + 2) are pending; the stage they make is visible after the barrier. (The
      // sched_barrier keeps their conversion below the record loads: hoisted into the MFMA
      // work it would wait for the records of b + 1 too.)
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_waitcnt(wait_vm16(kWL));
      if constexpr (T32)
        store_x32(xv, buf(u ^ 1), xsk, xsk1);
      else
        store_x(xv, buf(u ^ 1), xsk);
      FHIP_LDS_BARRIER16(wait_vm16(kWL));
    }
  }
  // D layout: lane (kap, rho) holds column rho and operand rows 8 (e / 4) + 4 kap + e % 4:
  // e < 8 the hi rows of tokens 8 (e / 4) + 4 kap + e % 4, e + 8 the lo rows of the same tokens.
  // hi + lo rows, times the token's scale (the loop's barriers made tscale visible)
  // T32: every operand row is its own token (e = 0..15: rows 8 (e / 4) + 4 kap + e % 4).
  constexpr int NV = T32 ? 16 : 8;
  float v[NT][NV];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int e = 0; e < NV; ++e)
      v[t][e] = (T32 ? acc[t][e] : acc[t][e] + acc[t][e + 8]) *
                tscale[8 * (e >> 2) + 4 * kap + (e & 3)];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int row = 16 * tile_of(t) + (lane & 15);  // recomputed: not kept live in the loop
    if (row >= N) continue;
#pragma unroll
    for (int e = 0; e < NV; ++e) {
      const int tok = 8 * (e >> 2) + 4 * kap + (e & 3);
      if (tok >= M) continue;
      if (SK == 1)
        Y[(size_t)tok * N + row] = v[t][e];
      else
        part[((size_t)sp * M + tok) * N + row] = v[t][e];
    }
  }
}
#undef FHIP_LDS_BARRIER16

// Y = sum of the SK partial results in range order: four outputs per thread when M * N is a
// multiple of 4 and Y 16-byte aligned, else one.
__global__ void gemv16_reduce1_kernel(const float *__restrict__ part, float *__restrict__ Y,
                                      int SK, int total) {
  const int id = blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= total) return;
  Y[id] = add_ranges(part[id], part + total + id, (size_t)total, SK - 1);
}

__global__ void gemv16_reduce_kernel(const float4 *__restrict__ part, float4 *__restrict__ Y,
                                     int SK, int total4) {
  const int id = blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= total4) return;
  Y[id] = add_ranges(part[id], part + total4 + id, (size_t)total4, SK - 1);
}

// The same sum for up to kRangesAtOnce ranges, one output per thread in 64-thread workgroups,
// every range's load issued before the first addition: with many ranges and few outputs (a long
// down projection at a few tokens) the float4 form runs too few threads, each waiting on its
// loads eight at a time. Same order, same bits.
constexpr int kRangesAtOnce = 32;
__global__ __launch_bounds__(64) void gemv16_reduce_wide_kernel(const float *__restrict__ part,
                                                                float *__restrict__ Y, int SK,
                                                                int total) {
  const int id = blockIdx.x * 64 + threadIdx.x;
  if (id >= total) return;
  float q[kRangesAtOnce];
#pragma unroll
  for (int k = 0; k < kRangesAtOnce; ++k)
    if (k < SK) q[k] = part[(size_t)k * total + id];
  float v = q[0];
#pragma unroll
  for (int k = 1; k < kRangesAtOnce; ++k)
    if (k < SK) v = v + q[k];
  Y[id] = v;
}

}  // namespace

// K ranges per call: ranges of 4 super-blocks when K allows it, else of 4 to 5 (the kernel
// works in passes of two super-blocks, so an odd range pads one; measured at the 7B / 27B FFN
// shapes at 16 tokens, longer ranges lose parallelism and shorter ones pay more per-range start
// and partial-sum traffic).
int gemv16_splits(int nblk) {
  int sk = nblk % 4 == 0 ? nblk / 4 : (int)(nblk / 4.6);
  if (sk < 1) sk = 1;
  if (sk > nblk) sk = nblk;
  return sk;
}

namespace {
template <int FMT, bool T32 = false>
int launch_gemv16(const void *Wv, const float *X, float *Y, int N, int K, int M) {
  if (M < 1 || M > (T32 ? 32 : 16))
    return fail(FHIP_EINVAL, "gemv16: M=%d outside 1..%d", M, T32 ? 32 : 16);
  const int nblk = K / 256, ntiles = q4k_tiles(N);
  const int nrb = ceil_div(ntiles, 8 * (T32 ? 1 : tiles16<FMT>()));
  const int SK = gemv16_splits(nblk);
  float *part = nullptr;
  if (SK > 1) {
    part = (float *)workspace((size_t)SK * M * N * 4);
    if (!part) return FHIP_ENOMEM;
    if (int rc = check_disjoint("gemv16", X, (size_t)M * K * 4, part, (size_t)SK * M * N * 4))
      return rc;
  }
  quant_gemv16_kernel<FMT, T32><<<nrb * SK, 256, 0, stream()>>>((const uint8_t *)Wv, X, Y, part, N, K,
                                                            M, nblk, ntiles, SK);
  FHIP_CHECK_LAUNCH("quant_gemv16_kernel");
  if (SK > 1) {
    const int tot = M * N;
    if (SK >= 8 && SK <= kRangesAtOnce)
      gemv16_reduce_wide_kernel<<<ceil_div(tot, 64), 64, 0, stream()>>>(part, Y, SK, tot);
    else if (tot % 4 == 0 && ((uintptr_t)Y & 15) == 0)
      gemv16_reduce_kernel<<<ceil_div(tot / 4, 256), 256, 0, stream()>>>(
          (const float4 *)part, (float4 *)Y, SK, tot / 4);
    else
      gemv16_reduce1_kernel<<<ceil_div(tot, 256), 256, 0, stream()>>>(part, Y, SK, tot);
    FHIP_CHECK_LAUNCH("gemv16_reduce_kernel");
  }
  return FHIP_OK;
}
}  // namespace

size_t gemv16_ws_bytes(int fmt, int N, int K, int M) {
  (void)fmt;
  const int SK = gemv16_splits(K / 256);
  return SK > 1 ? (size_t)SK * M * N * 4 : 0;
}

int q4k_gemv16(const void *Wv, const float *X, float *Y, int N, int K, int M) {
  return launch_gemv16<0>(Wv, X, Y, N, K, M);
}

int q6k_gemv16(const void *Wv, const float *X, float *Y, int N, int K, int M) {
  return launch_gemv16<1>(Wv, X, Y, N, K, M);
}

// 17..32 tokens of a Q4_K matmul, at the prefill GEMM's activation precision (f16 of x / s per
// token and K range): a chunk of a few tens of tokens costs about what 16 do here, where the
// 128-token tile of the prefill GEMM costs nearly what 128 do.
int q4k_gemv32(const void *Wv, const float *X, float *Y, int N, int K, int M) {
  return launch_gemv16<0, true>(Wv, X, Y, N, K, M);
}

int q6k_gemv32(const void *Wv, const float *X, float *Y, int N, int K, int M) {
  return launch_gemv16<1, true>(Wv, X, Y, N, K, M);
}

}  // namespace fhip
