// q4k_gemv.hip — small-M (1..4 tokens) Q4_K matmul: the decode GEMV run for every generated
// token, and narrow speculative-verify batches. Wider batches (5..16, or 3..16 on rows of
// K >= 24576) use q4k_gemv16.hip.
//
// Computes Y[t][o] = sum_k W[o][k] * X[t][k] with W the dequantized Q4_K weight
// (w = d*sc_s*n - dmin*m_s for sub-block s, internal/model/quant_q4k.go:90-111) without ever
// materialising w. Per sub-block s of row o and token t the sum factors as
//   sum_k w x = d * sc_s * sum_k n_k x_k  -  dmin * m_s * S_s,        S_s = sum_k x_k,
// and the integer-weight dot sum_k n_k x_k runs on the int8 MFMA v_mfma_i32_16x16x64_i8:
//   * weight operand: the 4-bit codes n (0..15) are int8 values as they stand; a dword of 8
//     nibbles becomes two int8x4 words, `q & 0x0F0F0F0F` and `(q >> 4) & 0x0F0F0F0F`.
//   * activation operand: every 32-value sub-block of a token is quantized to three int8
//     digits, x ~= e * (q1 + q2 / 256 + q3 / 65536) = e * T / 65536 with e the smallest power of
//     two >= max|x| / 63 and T = rint(65536 x / e). The error is at most e / 2^17 per value
//     (< 2.4e-7 of the block's largest magnitude, so a lone huge value leaves its block-mates
//     ~22 bits), integer activations below 2^22 are exact, and the int32 products of every
//     digit are exact. S_s is the f32 sum of the unquantized values.
//
// Accumulator layout. One MFMA covers one 32-byte chunk c of a row's nibbles (sub-block 2c in
// the low nibbles, 2c + 1 in the high nibbles) for the 16 rows of a tile. A result's 16 operand
// rows are four groups of four: group g stands for one (sub-block, token) and its rows for the
// three digits and a zero row. Result lane group g then holds exactly that group's three digit
// sums for the 16 output rows (D[0..2]; D[3] is zero).
//   * one token: two results, sub-blocks 0-3 and 4-7 (chunks 0-1 and 2-3 each accumulate into
//     one result); a lane loads activation digits for the two chunks its group belongs to;
//   * two tokens: one result per chunk, groups (parity of the sub-block, token);
//   * three or four tokens: one result per sub-block (two per chunk), groups = tokens.
// Operand rows whose sub-block parity varies across the lanes of one result read their 16 bytes
// from a "split" unit (P0 | 8 zero bytes | P1) at offset 0 or 8, so every lane's operand is
// {its digits, zeros} in the right half without a per-lane select.
//
// Work split: a workgroup owns TW 16-row tiles, each worked by KW waves on contiguous parts of
// the super-blocks. The workgroup quantizes the activations of all of K once into LDS for its
// TW tiles (when that does not fit, gemv_i8_prep_kernel writes them to global memory once).
// Each wave streams its tiled weight records (tiled.hpp) exactly once with three 16-byte loads
// per lane, keeping PF in flight; the KW partials of a tile are summed through LDS in part
// order (deterministic).
//
// Launch order. Vector loads complete in issue order per CU, and at the start of a launch every
// CU puts a burst of weight records in flight (most of a 38 MB matrix when the grid is one
// 16-wave workgroup per CU). Activation loads issued behind that burst land only when it has
// drained, and the quantization, the barrier and the first MFMA with them. So when each wave
// has at most kXPre (token, super-block) chunks to quantize, the kernel's first instructions
// load them (coalesced: one 1 KB load per chunk), a bare barrier keeps every wave's records
// behind every wave's activation loads, and the chunks are quantized lane-parallel
// (quant_lanes) while the records stream in.
//
// SwiGLU mode (the first stage of the fused decode MLP): the group is {gate, up} with tiles
// interleaved (gate tile T, up tile T, gate tile T + 1, ...) and TW even, so both tiles of a row
// block sit in one workgroup; the gate tile's final wave writes silu(gate) * up for its rows
// instead of two separate outputs.
#include <hip/hip_ext.h>

#include "gemv_common.hpp"

namespace fhip {
namespace {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

// ---- Activation operand layout for MP (1, 2, 4) token rows --------------------------------
// Per super-block slot: the A units, then the {e, S} pairs.
// A unit (chunk c, token t, digit k, lane group g) holds the digit-k bytes of values 8g..8g+7 of
// sub-blocks 2c (payload P0) and 2c + 1 (P1) of token t: for one and two tokens 24 bytes
// P0 | 0 x 8 | P1 (a 16-byte read at offset 0 gives {P0, 0}, at offset 8 {0, P1}); for four
// tokens 16 bytes P0 | P1 (both halves feed the two MFMAs of the chunk).
template <int MP>
__host__ __device__ constexpr int unit_bytes() { return MP == 4 ? 16 : 24; }
template <int MP>
__host__ __device__ constexpr int unit_of(int c, int t, int k, int g) {
  return ((c * MP + t) * 3 + k) * 4 + g;
}
template <int MP>
__host__ __device__ constexpr size_t a_bytes() { return (size_t)48 * MP * unit_bytes<MP>(); }
// Byte offset of the payload of sub-block sig (token t, digit k, lane group g) in a slot.
template <int MP>
__host__ __device__ constexpr size_t pay_off(int sig, int t, int k, int g) {
  return (size_t)unit_of<MP>(sig >> 1, t, k, g) * unit_bytes<MP>() +
         (size_t)(sig & 1) * (MP == 4 ? 8 : 16);
}
// Results per record, and the result lane group g's (sub-block, token) in result rho.
template <int MP>
__host__ __device__ constexpr int n_res() { return 2 * MP; }
template <int MP>
__host__ __device__ constexpr int res_sig(int rho, int g) {
  return MP == 1 ? 4 * rho + g : MP == 2 ? 2 * rho + (g >> 1) : rho;
}
template <int MP>
__host__ __device__ constexpr bool res_hi(int rho) {  // res_sig >= 4
  return MP == 1 ? rho == 1 : MP == 2 ? rho >= 2 : rho >= 4;
}
template <int MP>
__host__ __device__ constexpr int lane_tok(int g) {
  return MP == 1 ? 0 : MP == 2 ? (g & 1) : g;
}
// Index of the {e, S} pair of (sub-block, token): result rho of lane group g reads pair
// 2 * es4_of(rho >> 1, g) + (rho & 1), so a lane's pairs come two to a float4.
template <int MP>
__host__ __device__ constexpr int es4_of(int j, int g) {
  return MP == 1 ? g : MP == 2 ? (j * 2 + (g >> 1)) * 2 + (g & 1) : g * 4 + j;
}
template <int MP>
__host__ __device__ constexpr int es_of(int sig, int t) {
  return MP == 1 ? 2 * (sig & 3) + (sig >> 2)
       : MP == 2 ? 2 * ((((sig >> 2) * 2 + (sig & 1)) * 2) + t) + ((sig >> 1) & 1)
                 : 8 * t + sig;
}
// Bytes of the operands of one super-block.
template <int MP>
__host__ __device__ constexpr size_t op_bytes() { return a_bytes<MP>() + (size_t)MP * 64; }

// The block scale of a sub-block whose largest magnitude has bit pattern mb: e = 2^k, the
// smallest power of two with 63 e >= amax (amax = f 2^E, f in [0.5, 1)), so |x| / e <= 63 and
// x / e is exact. Non-finite blocks get e = NaN, which carries into every output that uses them.
__device__ __forceinline__ float block_scale(float amax, int &k) {
  int E;
  const float f = frexpf(amax, &E);
  k = E - 6 + (f > 63.f / 64.f ? 1 : 0);
  float e = amax > 0.f ? ldexpf(1.f, k) : 0.f;
  if (!(amax <= 3.4e38f)) e = __builtin_nanf("");
  return e;
}

// The 32 values of one sub-block of one token (zeros when !valid).
__device__ __forceinline__ void load_block(const float *__restrict__ x, bool valid, float (&v)[32]) {
  if (valid) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float4 f = *reinterpret_cast<const float4 *>(x + 4 * i);
      v[4 * i] = f.x; v[4 * i + 1] = f.y; v[4 * i + 2] = f.z; v[4 * i + 3] = f.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 32; ++i) v[i] = 0.f;
  }
}

// S of a sub-block in a fixed pairwise order: quads p_k = (v0 + v1) + (v2 + v3) of values
// 4k..4k+3, then ((p0 + p1) + (p2 + p3)) + ((p4 + p5) + (p6 + p7)). quant_lanes computes the
// same tree across eight lanes, so every path gives the same bits.
__device__ __forceinline__ float quad_sum(float a, float b, float c, float d) {
  return (a + b) + (c + d);
}
__device__ __forceinline__ float block_sum(const float (&v)[32]) {
  float p[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) p[k] = quad_sum(v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]);
  return quad_sum(p[0], p[1], p[2], p[3]) + quad_sum(p[4], p[5], p[6], p[7]);
}

// Quantize the 32 values v of sub-block sig of token t into a slot: A the slot's operand bytes,
// ES its {e, S} pairs.
template <int MP>
__device__ __forceinline__ void quant_vals(const float (&v)[32], int sig, int t,
                                           unsigned char *__restrict__ A, float2 *__restrict__ ES) {
  uint32_t mb = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i)
    mb = max(mb, absmax4_bits(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]));
  int k;
  const float e = block_scale(__uint_as_float(mb), k);  // a NaN when the block holds one
  ES[es_of<MP>(sig, t)] = make_float2(e, block_sum(v));
  // T = rint(65536 x / e), |T| <= 63 * 65536: digits3.
  const int sh = 16 - k;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    uint32_t a0, b0, c0, a1, b1, c1;
    digits3(v[8 * g], v[8 * g + 1], v[8 * g + 2], v[8 * g + 3], sh, a0, b0, c0);
    digits3(v[8 * g + 4], v[8 * g + 5], v[8 * g + 6], v[8 * g + 7], sh, a1, b1, c1);
    *reinterpret_cast<uint2 *>(A + pay_off<MP>(sig, t, 0, g)) = make_uint2(a0, a1);
    *reinterpret_cast<uint2 *>(A + pay_off<MP>(sig, t, 1, g)) = make_uint2(b0, b1);
    *reinterpret_cast<uint2 *>(A + pay_off<MP>(sig, t, 2, g)) = make_uint2(c0, c1);
    if (MP != 4 && !(sig & 1))
#pragma unroll
      for (int d = 0; d < 3; ++d)
        *reinterpret_cast<uint2 *>(A + (size_t)unit_of<MP>(sig >> 1, t, d, g) * 24 + 8) =
            make_uint2(0u, 0u);
  }
}

// Quantize one 32-value sub-block of one token (zeros when !valid) into a slot.
template <int MP>
__device__ __forceinline__ void quant_block(const float *__restrict__ x, bool valid, int sig,
                                            int t, unsigned char *__restrict__ A,
                                            float2 *__restrict__ ES) {
  float v[32];
  load_block(x, valid, v);
  quant_vals<MP>(v, sig, t, A, ES);
}

// Lane-parallel quantization of one super-block of one token, loaded coalesced: lane l holds
// values 4 (l & 7) .. 4 (l & 7) + 3 of sub-block l >> 3 in v. Bit-identical to quant_vals: the
// scale comes from the block maximum (order-free), each digit from its own value, and the
// block sum is block_sum's tree, its levels taken across lanes (lane ^ 1, lane ^ 2, then the
// other quad of the eight, each pair added in either order: the sum commutes exactly).
#define FHIP_DPP(v, ctrl) \
  __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, (v)), (ctrl), 0xF, 0xF, false))
#define FHIP_DPP_U(v, ctrl) \
  (uint32_t) __builtin_amdgcn_update_dpp(0, (int)(v), (ctrl), 0xF, 0xF, false)

// The block maximum is taken on magnitude bit patterns (absmax4_bits): one DPP max per step, where
// fmaxf needed a NaN-quieting max and a separate DPP move. The digits use one fma per value
// (digits3s) unless a lane's scale 2^(16 - k) is not a normal float (blocks below ~2^-105, where
// the wave takes ldexpf).
template <int MP>
__device__ __forceinline__ void quant_lanes(const float4 v, int lane, int t,
                                            unsigned char *__restrict__ A,
                                            float2 *__restrict__ ES) {
  const int sig = lane >> 3, p = lane & 7;
  uint32_t mb = absmax4_bits(v.x, v.y, v.z, v.w);
  mb = max(mb, FHIP_DPP_U(mb, 0xB1));   // quad_perm [1,0,3,2]: lane ^ 1
  mb = max(mb, FHIP_DPP_U(mb, 0x4E));   // quad_perm [2,3,0,1]: lane ^ 2
  mb = max(mb, FHIP_DPP_U(mb, 0x141));  // row_half_mirror: the other quad of the eight
  float sum = quad_sum(v.x, v.y, v.z, v.w);
  sum = sum + FHIP_DPP(sum, 0xB1);
  sum = sum + FHIP_DPP(sum, 0x4E);
  sum = sum + FHIP_DPP(sum, 0x141);
  int k;
  const float e = block_scale(__uint_as_float(mb), k);  // a NaN when the block holds one
  if (p == 0) ES[es_of<MP>(sig, t)] = make_float2(e, sum);
  uint32_t a, b, c;
  const int sh = 16 - k;
  if (__builtin_expect(__builtin_amdgcn_ballot_w64(sh > 127) == 0, 1))
    digits3s(v.x, v.y, v.z, v.w, ldexpf(1.f, sh), a, b, c);
  else
    digits3(v.x, v.y, v.z, v.w, sh, a, b, c);
  const int g = p >> 1, h = 4 * (p & 1);
  const uint32_t dig[3] = {a, b, c};
#pragma unroll
  for (int d = 0; d < 3; ++d) {
    uint32_t *u = reinterpret_cast<uint32_t *>(A + (size_t)unit_of<MP>(sig >> 1, t, d, g) *
                                                       unit_bytes<MP>() + h);
    u[(sig & 1) * (MP == 4 ? 2 : 4)] = dig[d];
    // Split units: both sub-blocks' lanes write the zero dword between the payloads (the same
    // value twice), so no lane branches.
    if (MP != 4) u[2] = 0u;
  }
}

// Quantize super-blocks [s0, s0 + nb) of M tokens (tokens M..MP-1 zero) into slots 0..nb-1 of
// the operand buffers, `lane` of `nlanes` threads sharing the work.
template <int MP>
__device__ __forceinline__ void quant_range(const float *__restrict__ X, int K, int M, int s0,
                                            int nb, unsigned char *__restrict__ A,
                                            float2 *__restrict__ ES, int lane, int nlanes) {
  const int per_t = nb * 8;
  for (int task = lane; task < per_t * MP; task += nlanes) {
    const int t = task / per_t, rest = task - t * per_t;
    const int bl = rest >> 3, sig = rest & 7;
    const bool valid = t < M;
    quant_block<MP>(X + (valid ? (size_t)t * K + 256 * (size_t)(s0 + bl) + 32 * sig : 0), valid,
                    sig, t, A + (size_t)bl * a_bytes<MP>(), ES + (size_t)bl * 8 * MP);
  }
}

// Scale and min of sub-block 4 * hi + q (GetScaleMinK4, internal/model/quantbits.go:42-47) from
// the header words y = scales[0..3], z = scales[4..7], w = scales[8..11]; q may vary by lane.
__device__ __forceinline__ void scale_min(uint32_t y, uint32_t z, uint32_t w, bool hi, int q,
                                          float &sc, float &mn) {
  const uint32_t o = 8u * (uint32_t)q;
  uint32_t s, m;
  if (!hi) {
    s = __builtin_amdgcn_ubfe(y, o, 6);
    m = __builtin_amdgcn_ubfe(z, o, 6);
  } else {
    s = __builtin_amdgcn_ubfe(w, o, 4) | (__builtin_amdgcn_ubfe(y, o + 6, 2) << 4);
    m = __builtin_amdgcn_ubfe(w, o + 4, 4) | (__builtin_amdgcn_ubfe(z, o + 6, 2) << 4);
  }
  sc = (float)s;
  mn = (float)m;
}

// The eight 6-bit scales and mins of a row header (GetScaleMinK4 for j = 0..7), byte-parallel:
// byte i of sc[0] / mn[0] is the scale / min of sub-block i, of sc[1] / mn[1] sub-block 4 + i.
__device__ __forceinline__ void scale_min8(uint32_t y, uint32_t z, uint32_t w, uint32_t (&sc)[2],
                                           uint32_t (&mn)[2]) {
  const uint32_t m6 = 0x3F3F3F3Fu, m4 = 0x0F0F0F0Fu, m2 = 0x30303030u;
  sc[0] = y & m6;
  mn[0] = z & m6;
  sc[1] = (w & m4) | ((y >> 2) & m2);
  mn[1] = ((w >> 4) & m4) | ((z >> 2) & m2);
}
// Byte i of v as a float (one v_cvt_f32_ubyte<i>).
__device__ __forceinline__ float ubyte_f32(uint32_t v, int i) {
  return (float)((v >> (8 * i)) & 0xFFu);
}

// 65536 d0 + 256 d1 + d2 as two shift-adds. The empty asm (no instruction) only stops the
// compiler from re-associating the sum into three instructions; the arithmetic itself stays
// compiler code, which knows to wait for the MFMA results it reads.
__device__ __forceinline__ int digit_sum(int d0, int d1, int d2) {
  int t = (d0 << 8) + d1;
  asm volatile("" : "+v"(t));
  return (t << 8) + d2;
}

// silu(z) = z / (1 + e^-z) with e^-z evaluated in double and rounded to f32, the operation
// order of internal/model/forward.go:452.
__device__ __forceinline__ float silu_f32(float z) {
  return z / (1.f + (float)exp(-(double)z));
}

// Weight records each wave keeps in flight (LDS path) and the widest workgroup (waves) for one
// token. Measured at the 7B FFN shapes: an 8-record ring with 8-wave workgroups, the
// activation loads issued ahead of the ring, and lane-parallel coalesced quantization were all
// slower (11.9-12 us gate/up, 14.7-15.1 us down, against 10.6 and 13.8 us here); so were rings
// of 5 and 6 records with the present workgroups (gate/up 10.1 / 10.3 against 9.6 us, down
// 11.4 / 11.8-12.2 against 11.3), though every down wave then holds all its records at once.
constexpr int kPF1 = 4, kMaxWaves1 = 16;
// Most super-blocks (of all tokens) a wave quantizes from activations loaded before its records.
constexpr int kXPre = 8;

// XM: how the activations reach LDS (LX only). kXLate: quant_range after the first records;
// kXSpread: loaded first, chunk c by wave c % waves, one workgroup barrier before the records
// are used; kXOwn (one tile per workgroup): each wave loads and quantizes the super-blocks of
// its own K part, and no wave waits for another. PF0: records per wave put in flight before
// the activations are quantized (kXSpread, kXOwn); the rest of the ring follows. A smaller first
// burst lets the activations land sooner; a full one pays when every wave has several chunks.
// EX: each ring slot is refilled unconditionally (the repeat of the last record at the end of a
// part is never used), so every ring wait counts exactly; else only while records remain.
enum { kXLate = 0, kXSpread = 1, kXOwn = 2 };
template <int MP, bool LX, bool SWIGLU, int XM, int PF0, bool EX>
__global__ __launch_bounds__(MP == 1 ? 64 * kMaxWaves1 : 512) void q4k_gemv_i8_kernel(
    const GemvGroup grp, const float *__restrict__ X, const unsigned char *__restrict__ xg, int K,
    int M, int nblk, int TW, int KW) {
  constexpr int NR = n_res<MP>();
  extern __shared__ __align__(16) unsigned char smem[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: SGPRs
  const int nwaves = (int)(blockDim.x >> 6);

  // First instructions: this wave's activation chunks (chunk c = token c / nblk, super-block
  // c % nblk; see the launch order above), then the barrier that holds every record load
  // behind every wave's activation loads.
  const int nchunk = nblk * MP;
  constexpr bool xpre = LX && XM != kXLate;
  constexpr bool xown = LX && XM == kXOwn;
  auto chunk_tok = [&](int c) {  // c / nblk without a division (MP <= 4)
    return MP == 1 ? 0 : (c >= nblk) + (MP > 2 ? (c >= 2 * nblk) + (c >= 3 * nblk) : 0);
  };
  constexpr int kPT = kXPre / MP;  // super-blocks per token a kXOwn wave may hold
  int ob0 = 0, onb = 0;  // kXOwn: this wave's K part (TW == 1, KW = waves)
  if (xown) {
    ob0 = wave * nblk / KW;
    onb = (wave + 1) * nblk / KW - ob0;
  }
  float4 xv[kXPre];
  if (xown) {
#pragma unroll
    for (int t = 0; t < MP; ++t)
#pragma unroll
      for (int i = 0; i < kPT; ++i)
        if (i < onb)
          xv[t * kPT + i] = *reinterpret_cast<const float4 *>(
              X + (size_t)min(t, M - 1) * K + 256 * (size_t)(ob0 + i) + 4 * lane);
  } else if (xpre) {
#pragma unroll
    for (int j = 0; j < kXPre; ++j) {
      const int c = wave + j * nwaves;
      if (c < nchunk) {
        const int t = chunk_tok(c);
        xv[j] = *reinterpret_cast<const float4 *>(X + (size_t)min(t, M - 1) * K +
                                                  256 * (size_t)(c - t * nblk) + 4 * lane);
      }
    }
  }
  if (xpre) {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  }
  __builtin_amdgcn_sched_barrier(kNoVmemAcross);

  const int gq = lane >> 4, r = lane & 15;
  const int tile = wave / KW, part = wave - tile * KW;
  const int Tg = blockIdx.x * TW + tile;  // tile of the concatenated group
  const int ntiles = grp.tile0[grp.count];
  const bool tvalid = Tg < ntiles;
  int mem = 0;  // the member this tile belongs to (wave-uniform scalar search)
  int T;        // tile within the member
  if (SWIGLU) {
    mem = Tg & 1;
    T = tvalid ? Tg >> 1 : 0;
  } else {
    while (mem + 1 < grp.count && Tg >= grp.tile0[mem + 1]) ++mem;
    T = tvalid ? Tg - grp.tile0[mem] : 0;
  }
  const int N = grp.N[mem];
  float *__restrict__ Y = grp.Y[mem];
  // This wave's part [b0, b1) of the super-blocks.
  const int b0 = part * nblk / KW;
  const int b1 = (part + 1) * nblk / KW;
  const int nb = b1 - b0;  // >= 1: KW <= nblk
  const uint8_t *base = grp.W[mem] + (size_t)T * nblk * kQ4kRecord;

  // Operands: in LDS, quantized once by the whole workgroup for its TW tiles, or the prepared
  // global buffer; slot = super-block either way.
  const unsigned char *opA = LX ? smem : xg;
  const float4 *ES4 = reinterpret_cast<const float4 *>(opA + (size_t)nblk * a_bytes<MP>());
  float *red = reinterpret_cast<float *>(smem + (LX ? (size_t)nblk * op_bytes<MP>() : 0));

  // This lane's operand row: group ag = r >> 2 of its results, digit ad = r & 3 (3: the zero
  // row). With one token the group is sub-block 4 rho + ag, in chunks (ag >> 1) and
  // 2 + (ag >> 1); with two tokens (parity ag >> 1, token ag & 1) of every chunk; with four
  // tokens token ag of every chunk (both halves of the unit: the chunk's two results).
  const int ag = r >> 2, ad = r & 3;
  const bool arow = ad < 3;
  const int adc = arow ? ad : 2;  // a valid unit for the zero rows' (unused) global loads
  auto a_off = [&](int c) -> size_t {
    if (MP == 1) return (size_t)unit_of<1>(c, 0, adc, gq) * 24 + 8 * (ag & 1);
    if (MP == 2) return (size_t)unit_of<2>(c, ag & 1, adc, gq) * 24 + 8 * (ag >> 1);
    return (size_t)unit_of<4>(c, ag, adc, gq) * 16;
  };
  auto a_own = [&](int c) { return arow && (MP != 1 || (c & 1) == (ag >> 1)); };
  const unsigned char *alane = opA + a_off(0);  // LDS path: this lane's operand in slot 0
  auto ld16 = [](const unsigned char *p) {  // 8-byte aligned
    const uint2 lo = *reinterpret_cast<const uint2 *>(p);
    const uint2 hi = *reinterpret_cast<const uint2 *>(p + 8);
    return i32x4{(int)lo.x, (int)lo.y, (int)hi.x, (int)hi.y};
  };

  struct Ops {
    uint4 h, qa, qb;
    i32x4 a[LX ? 1 : 4];
    float4 es[LX ? 1 : MP];
  };
  auto load = [&](int b, Ops &o) {
    const uint8_t *rec = base + (size_t)b * kQ4kRecord;
    o.h = ld_stream(rec + 16 * r);
    o.qa = ld_stream(rec + kQ4kHdr + 16 * lane);
    o.qb = ld_stream(rec + kQ4kHdr + 1024 + 16 * lane);
    if (!LX) {
      // Every lane loads all four (an exec-masked load made the compiler wait for the whole
      // ring after it); the lanes that do not own a chunk zero it at use.
      const unsigned char *slot = opA + (size_t)b * a_bytes<MP>();
#pragma unroll
      for (int c = 0; c < 4; ++c) o.a[c] = ld16(slot + a_off(c));
#pragma unroll
      for (int j = 0; j < MP; ++j) o.es[j] = ES4[(size_t)b * 4 * MP + es4_of<MP>(j, gq)];
    }
  };
  constexpr int PF = LX ? (MP == 1 ? kPF1 : 4) : 2;
  Ops ring[PF];
#pragma unroll
  for (int u = 0; u < PF; ++u) {
    if (!LX)
#pragma unroll
      for (int c = 0; c < 4; ++c) ring[u].a[c] = i32x4{0, 0, 0, 0};
    if (!xpre || u < PF0) load(min(b0 + u, b1 - 1), ring[u]);  // a repeat is never used
  }
  // With the first records in flight, the workgroup quantizes the activations of its K range.
  unsigned char *wA = const_cast<unsigned char *>(opA);
  float2 *wES = reinterpret_cast<float2 *>(const_cast<float4 *>(ES4));
  if (LX) {
    if (xown) {
      // Only this wave reads these slots: LDS accesses of one wave complete in order, so no
      // barrier is needed before its own reads.
      const float4 z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int t = 0; t < MP; ++t)
#pragma unroll
        for (int i = 0; i < kPT; ++i)
          if (i < onb)
            quant_lanes<MP>(MP == 1 || t < M ? xv[t * kPT + i] : z, lane, t,
                            wA + (size_t)(ob0 + i) * a_bytes<MP>(),
                            wES + (size_t)(ob0 + i) * 8 * MP);
    } else if (xpre) {
#pragma unroll
      for (int j = 0; j < kXPre; ++j) {
        const int c = wave + j * nwaves;
        if (c < nchunk) {
          const int t = chunk_tok(c), bl = c - t * nblk;
          const float4 z = {0.f, 0.f, 0.f, 0.f};
          quant_lanes<MP>(MP == 1 || t < M ? xv[j] : z, lane, t, wA + (size_t)bl * a_bytes<MP>(),
                          wES + (size_t)bl * 8 * MP);
        }
      }
    } else {
      quant_range<MP>(X, K, M, 0, nblk, wA, wES, threadIdx.x, blockDim.x);
    }
    if (!xown) __syncthreads();
    if (xpre)
#pragma unroll
      for (int u = PF0; u < PF; ++u) load(min(b0 + u, b1 - 1), ring[u]);
  }
  const uint32_t k0F = 0x0F0F0F0Fu;

  // The activation operands of the current super-block, one per chunk; with four tokens the
  // chunk's unit is split into its two MFMA operands, each with a zero half that is never
  // written. Operands a lane does not load stay zero in that lane for the whole kernel.
  i32x4 areg[4], alo[4], ahi[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) areg[c] = alo[c] = ahi[c] = i32x4{0, 0, 0, 0};

  float acc = 0.f;

  for (int bb = b0; bb < b1; bb += PF) {
#pragma unroll
    for (int u = 0; u < PF; ++u) {
      const int b = bb + u;
      if (b >= b1) break;
      // This slot's three loads are older than the other slots' refills: saying so lets the
      // compiler wait for just this record instead of draining the ring at the top of a pass.
      if (LX) __builtin_amdgcn_s_waitcnt(0x0F70 | (3 * (PF - 1)));
      else __builtin_amdgcn_s_waitcnt(0x0F70 | ((11 + MP) * (PF - 1)));  // 3 + 8 + MP loads: < 16
      Ops &cur = ring[u];

      float4 es[MP];
      if (LX) {
        // The slot's base is a scalar: one address add per record, and each chunk's offset
        // (a_off(c) - a_off(0), a constant) fits the LDS instructions' immediate fields.
        const unsigned char *slot =
            alane + __builtin_amdgcn_readfirstlane((int)((size_t)b * a_bytes<MP>()));
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          if (!a_own(c)) continue;
          constexpr int kCS = a_bytes<MP>() / 4;  // a_off(c) = a_off(0) + c * kCS
          const uint2 lo = *reinterpret_cast<const uint2 *>(slot + c * kCS);
          const uint2 hi = *reinterpret_cast<const uint2 *>(slot + c * kCS + 8);
          if (MP == 4) {
            alo[c][0] = (int)lo.x; alo[c][1] = (int)lo.y;
            ahi[c][2] = (int)hi.x; ahi[c][3] = (int)hi.y;
          } else {
            areg[c] = i32x4{(int)lo.x, (int)lo.y, (int)hi.x, (int)hi.y};
          }
        }
        const float4 *es4 =
            ES4 + __builtin_amdgcn_readfirstlane((int)((size_t)b * 4 * MP));
#pragma unroll
        for (int j = 0; j < MP; ++j) es[j] = es4[es4_of<MP>(j, gq)];
      } else {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const i32x4 v = a_own(c) ? cur.a[c] : i32x4{0, 0, 0, 0};
          if (MP == 4) {
            alo[c][0] = v[0]; alo[c][1] = v[1];
            ahi[c][2] = v[2]; ahi[c][3] = v[3];
          } else {
            areg[c] = v;
          }
        }
#pragma unroll
        for (int j = 0; j < MP; ++j) es[j] = cur.es[j];
      }

      // Weight operands: chunk c = words 2c, 2c+1 of the lane's 32 bytes (8 nibble positions
      // of the chunk), low nibbles -> slots 0-7 (sub-block 2c), high -> slots 8-15 (2c + 1).
      const uint32_t q[8] = {cur.qa.x, cur.qa.y, cur.qa.z, cur.qa.w,
                             cur.qb.x, cur.qb.y, cur.qb.z, cur.qb.w};
      i32x4 D[NR];
#pragma unroll
      for (int rho = 0; rho < NR; ++rho) D[rho] = i32x4{0, 0, 0, 0};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const i32x4 B = {(int)(q[2 * c] & k0F), (int)(q[2 * c + 1] & k0F),
                         (int)((q[2 * c] >> 4) & k0F), (int)((q[2 * c + 1] >> 4) & k0F)};
        if (MP == 4) {
          D[2 * c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(alo[c], B, D[2 * c], 0, 0, 0);
          D[2 * c + 1] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ahi[c], B, D[2 * c + 1], 0, 0, 0);
        } else {
          const int rho = MP == 1 ? c >> 1 : c;
          D[rho] = __builtin_amdgcn_mfma_i32_16x16x64_i8(areg[c], B, D[rho], 0, 0, 0);
        }
      }
      // The header is decoded into what the epilogue needs (d, dmin and the scales and mins;
      // two and four tokens: every sub-block's, byte-parallel, with two tokens lane group g's
      // sub-blocks 2 rho + (g >> 1) brought to bytes 0 and 2 of each word), so that the slot
      // can be refilled right after: nothing then reads the old header behind the new load.
      const uint4 h = cur.h;
      float dd = (float)__builtin_bit_cast(_Float16, (uint16_t)(h.x & 0xffffu));
      float dmn = (float)__builtin_bit_cast(_Float16, (uint16_t)(h.x >> 16));
      uint32_t sc8[2], mn8[2];
      float sc1[NR], mn1[NR];
      if (MP >= 2) {
        scale_min8(h.y, h.z, h.w, sc8, mn8);
        if (MP == 2) {
          const uint32_t sh = 8u * (uint32_t)(gq >> 1);
#pragma unroll
          for (int i = 0; i < 2; ++i) {
            sc8[i] >>= sh;
            mn8[i] >>= sh;
          }
        }
      } else {
#pragma unroll
        for (int rho = 0; rho < NR; ++rho)
          scale_min(h.y, h.z, h.w, res_hi<MP>(rho), res_sig<MP>(rho, gq) & 3, sc1[rho], mn1[rho]);
      }
      // The slot is refilled with the record PF ahead once its operands and header are
      // consumed. The empty asm pins the decoded values before the refill's branch (otherwise
      // the decode sinks below it), and nothing moves across the barrier: either way the
      // header would need a second register and a copy back that waits for the new load.
      asm volatile("" : "+v"(dd), "+v"(dmn));
#pragma unroll
      for (int i = 0; i < (MP >= 2 ? 2 : 0); ++i) asm volatile("" : "+v"(sc8[i]), "+v"(mn8[i]));
#pragma unroll
      for (int rho = 0; rho < (MP == 1 ? NR : 0); ++rho)
        asm volatile("" : "+v"(sc1[rho]), "+v"(mn1[rho]));
      __builtin_amdgcn_sched_barrier(0);
      if (EX)
        load(min(b + PF, b1 - 1), cur);
      else if (b + PF < b1)
        load(b + PF, cur);

      // Per result: T-sum = 65536 D0 + 256 D1 + D2 (exact in int32: |D0| <= 32 * 15 * 63), then
      // sc * e * T-sum; the 2^-16 of the digits is folded into d.
      float xs = 0.f, vs = 0.f;
#pragma unroll
      for (int rho = 0; rho < NR; ++rho) {
        float sc, mn;
        if (MP >= 2) {
          const int byte = MP == 4 ? rho & 3 : 2 * (rho & 1);  // sub-block rho, or 2 rho + (g >> 1)
          sc = ubyte_f32(sc8[rho >> (MP == 4 ? 2 : 1)], byte);
          mn = ubyte_f32(mn8[rho >> (MP == 4 ? 2 : 1)], byte);
        } else {
          sc = sc1[rho];
          mn = mn1[rho];
        }
        const int ts = digit_sum(D[rho][0], D[rho][1], D[rho][2]);
        const float4 ep = es[rho >> 1];
        const float e = (rho & 1) ? ep.z : ep.x;
        const float S = (rho & 1) ? ep.w : ep.y;
        xs = fmaf(sc, e * (float)ts, xs);
        vs = fmaf(mn, S, vs);
      }
      acc = fmaf(dd * (1.f / 65536.f), xs, fmaf(-dmn, vs, acc));
    }
  }

  // Partials of the KW parts go through LDS; part 0 sums them in part order (deterministic),
  // then adds the lane groups that hold the same (token, row): all four (one token), g and
  // g ^ 2 (two tokens); with four tokens lane group g holds token g alone.
  red[(tile * KW + part) * 64 + lane] = acc;
  __syncthreads();
  const int row = T * 16 + r;
  const bool fin = part == 0 && tvalid;
  if (!SWIGLU && !fin) return;
  float v = acc;
  for (int q = 1; q < KW; ++q) v += red[(tile * KW + q) * 64 + lane];
  if (MP <= 2) v += __shfl_xor(v, 32);
  if (MP == 1) v += __shfl_xor(v, 16);
  const int t = lane_tok<MP>(gq);
  const bool writer = gq < MP && t < M;  // lane groups 0..MP-1 hold the tokens
  if (SWIGLU) {
    // Every wave reaches this barrier; the up tile's final values go through LDS to its gate
    // partner (tile + 1 holds up tile T when tile holds gate tile T).
    float *xch = red + (size_t)blockDim.x;
    if (fin) xch[tile * 64 + lane] = v;
    __syncthreads();
    if (!fin || mem != 0) return;
    if (row < N && writer) Y[(size_t)t * N + row] = silu_f32(v) * xch[(tile + 1) * 64 + lane];
    return;
  }
  if (row < N && writer) Y[(size_t)t * N + row] = v;
}

// Global-path operand writer: one thread per (token, 32-value sub-block) of all of K.
template <int MP>
__global__ void gemv_i8_prep_kernel(const float *__restrict__ X, int K, int M, int nblk,
                                    unsigned char *__restrict__ A) {
  const int id = blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= MP * nblk * 8) return;
  const int per_t = nblk * 8;
  const int t = id / per_t, rest = id - t * per_t;
  const int b = rest >> 3, sig = rest & 7;
  float2 *ES = reinterpret_cast<float2 *>(A + (size_t)nblk * a_bytes<MP>());
  const bool valid = t < M;
  quant_block<MP>(X + (valid ? (size_t)t * K + 256 * (size_t)b + 32 * sig : 0), valid, sig, t,
                  A + (size_t)b * a_bytes<MP>(), ES + (size_t)b * 8 * MP);
}

// Workgroup shape: TW tiles x KW waves per tile (TW * KW <= max_waves). Measured on the 7B
// and 27B FFN and lm_head shapes: each wave should stream >= ~6 records (KW), a workgroup
// should be as wide as possible so its quantized activations serve many tiles (TW) while the
// grid still covers about half the CUs, the grid should fit in one resident round when LDS
// limits residency (large K), and very tall matrices prefer narrow workgroups.
// FAK_HIP_GEMV_TW and FAK_HIP_GEMV_KW override (tuning).
void i8_shape(int ntiles, int nblk, int max_waves, size_t lds_fixed, size_t lds_per_wave,
              int &TW, int &KW) {
  const int cus = cu_count() > 0 ? cu_count() : 256;
  const size_t lds_max = (size_t)lds_limit();
  TW = tuning().gemv_tw;
  KW = tuning().gemv_kw;
  if (KW <= 0) {
    KW = 1;
    while (2 * KW <= max_waves && nblk >= 6 * 2 * KW) KW *= 2;
    // Small matrices: split K further until the grid has about two waves per CU.
    while (2 * KW <= max_waves && ntiles * KW < 2 * cus && nblk >= 2 * 2 * KW) KW *= 2;
  }
  if (KW > nblk) KW = nblk;
  if (KW > max_waves) KW = max_waves;
  if (TW <= 0) {
    TW = max_waves / KW;
    if (ntiles > 8 * cus) {
      TW = 4 / KW > 1 ? 4 / KW : 1;
    } else {
      while (TW > 1 && ceil_div(ntiles, TW) < cus / 2) TW /= 2;
      // A grid of about 80% of the CUs beats wider workgroups on fewer CUs (one token, 7B
      // gate/up, 1184 tiles: 6 tiles per workgroup 9.55 us, 5 9.6, 8 10.2; 27B gate/up, 1600
      // tiles: 8 either way, 14.7 us; a grid beyond the CU count runs a second round, 20.9 us).
      TW = min(TW, max(1, ceil_div(5 * ntiles, 4 * cus)));
      auto rounds = [&](int tw, int kw) {
        const size_t lds = lds_fixed + (size_t)tw * kw * lds_per_wave;
        const int by_lds = lds > 0 ? (int)(lds_max / lds) : 32;
        const int per_cu = by_lds < 32 / (tw * kw) ? by_lds : 32 / (tw * kw);
        return per_cu > 0 ? ceil_div(ceil_div(ntiles, tw), per_cu * cus) : 1 << 30;
      };
      while (KW > 1 && 2 * TW * (KW / 2) <= max_waves && rounds(TW, KW) > 1 &&
             rounds(2 * TW, KW / 2) < rounds(TW, KW)) {
        KW /= 2;
        TW *= 2;
      }
    }
  }
  if (TW < 1) TW = 1;
  while (TW > 1 && TW * KW > max_waves) TW--;
}

// Launch shape of one small-M call: TW tiles x KW waves per workgroup, activations in LDS or
// in a prepared global buffer, and the workspace it needs (the global operands). K is not split
// across workgroups: measured on the 7B and 27B down projections (partials combined through
// device-scope stores and a per-tile arrival counter) it gained at most 5% and lost elsewhere.
struct I8Plan {
  int TW, KW;
  bool lds_x;
  size_t lds_bytes, xop_bytes;
};

template <int MP>
I8Plan plan_i8(int ntiles, int K, bool swiglu) {
  const int nblk = K / 256;
  const int max_waves = MP == 1 ? kMaxWaves1 : 8;
  I8Plan p{};
  const size_t ldsx = (size_t)nblk * op_bytes<MP>();
  i8_shape(ntiles, nblk, max_waves, ldsx, (size_t)64 * 4, p.TW, p.KW);
  // At most two tiles per CU: one workgroup of up to max_waves waves per CU (one tile, or two
  // above one tile per CU), each wave streaming >= 1.5 records (>= 3 for one token on a grid of
  // half the CUs or more, see below). Two to four tokens over 2..8 tiles per CU: eight
  // one-wave tiles per workgroup, which share the (larger) quantization. Measured (us, this rule
  // / the rule above), one token: 3584 x 18944 13.2 / 13.8, 3584 x 3584 5.9 / 6.2, 4096 x 5120
  // 7.2 / 8.6, 5120 x 5120 7.4 / 8.7, 4608 x 3584 6.6 / 7.2, 8192 x 5120 8.2 / 10.0, 5120 x
  // 25600 21.7 / 22.1; four tokens: 3584 x 3584 8.0 / 8.6, 5120 x 5120 10.5 / 11.9, 18944 x
  // 3584 14.5 / 16.2, 25600 x 5120 19.9 / 20.1.
  const int cus = cu_count() > 0 ? cu_count() : 256;
  if (!tuning().gemv_tw && !tuning().gemv_kw) {
    if (ntiles <= 2 * cus) {
      p.TW = ntiles <= cus ? 1 : 2;
      p.KW = max_waves / p.TW;
      // Records per wave: at least 1.5, and for one token on a grid of half the CUs or more at
      // least 3 (4 against 8 K parts: 3584 x 3584 4.9-5.2 against 5.3 us, 4608 x 3584 5.7 / 6.6,
      // 5120 x 5120 6.4 / 7.2, 6144 x 5120 6.6 / 7.4, 4096 x 5120 5.5 / 6.0; 512 x 3584, 32
      // tiles, keeps 8 parts: 4.6 us either way; four tokens keep 8).
      const int rec2 = MP == 1 && 2 * ntiles >= cus ? 6 : 3;  // twice the minimum
      while (p.KW > 1 && 2 * nblk < rec2 * p.KW) p.KW /= 2;
    } else if (MP > 1 && ntiles <= 8 * cus) {
      p.TW = max_waves;
      p.KW = 1;
    }
  }
  if (p.KW > nblk) p.KW = nblk;
  if (swiglu && (p.TW & 1)) {  // both tiles of a row block in one workgroup
    if (p.TW > 1) {
      p.TW -= 1;
    } else {
      p.TW = 2;
      if (2 * p.KW > max_waves) p.KW = max_waves / 2;
    }
  }
  const size_t redB =
      (size_t)p.TW * p.KW * 64 * 4 + (swiglu ? (size_t)p.TW * 64 * 4 : 0);
  p.lds_x = !tuning().gemv_globalx && ldsx + redB <= (size_t)lds_limit();
  p.lds_bytes = (p.lds_x ? ldsx : 0) + redB;
  p.xop_bytes = p.lds_x ? 0 : (((size_t)nblk * op_bytes<MP>() + 255) & ~(size_t)255);
  return p;
}

// swiglu: the group is {gate, up} with tile0[2] = 2 * tiles (interleaved; see the kernel).
// ws: a caller-provided workspace of plan_i8(...).xop_bytes (nullptr: the library workspace).
template <int MP>
int launch_i8(const GemvGroup &g, const float *X, int K, int M, bool swiglu, void *ws) {
  const int nblk = K / 256, ntiles = g.tile0[g.count];
  const I8Plan p = plan_i8<MP>(ntiles, K, swiglu);
  const size_t wsB = p.xop_bytes;
  if (!ws && wsB) ws = workspace(wsB);
  if (wsB && !ws) return FHIP_ENOMEM;
  if (int rc = check_disjoint("q4k_gemv", X, (size_t)M * K * 4, ws, wsB)) return rc;
  unsigned char *xop = (unsigned char *)ws;
  const int grid = ceil_div(ntiles, p.TW), threads = 64 * p.TW * p.KW;
  const unsigned char *xg = nullptr;
  if (!p.lds_x) {
    const int nprep = MP * nblk * 8;
    gemv_i8_prep_kernel<MP><<<ceil_div(nprep, 128), 128, 0, stream()>>>(X, K, M, nblk,
                                                                        xop);
    FHIP_CHECK_LAUNCH("gemv_i8_prep_kernel");
    xg = xop;
  }
  // The kernel goes out through hipExtLaunchKernelGGL so that fhip_time_next_launch's events
  // (null otherwise, an ordinary launch) take the dispatch's own start and end timestamps.
  hipEvent_t ev0, ev1;
  take_launch_events(&ev0, &ev1);
#define FHIP_I8_LAUNCH_EX(LXV, SWV, XMV, PF0V, EXV)                                          \
  hipExtLaunchKernelGGL(q4k_gemv_i8_kernel<MP, LXV, SWV, XMV, PF0V, EXV>, dim3(grid),        \
                        dim3(threads), (uint32_t)p.lds_bytes, stream(), ev0, ev1, 0u, g, X, xg, \
                        K, M, nblk, p.TW, p.KW)
#define FHIP_I8_LAUNCH(LXV, SWV, XMV, PF0V)                                                  \
  do {                                                                                       \
    if (exact) FHIP_I8_LAUNCH_EX(LXV, SWV, XMV, PF0V, (MP > 1));                             \
    else FHIP_I8_LAUNCH_EX(LXV, SWV, XMV, PF0V, false);                                      \
  } while (0)
  // Activations loaded ahead of the records when each wave has at most kXPre chunks (kXOwn
  // when each wave's own K part fits, one tile per workgroup). The full first burst for one
  // token when every wave quantizes >= 3 chunks (the long-row down projections: 3584 x 18944
  // 11.5 vs 11.8 us, 5120 x 25600 19.1 vs 19.6), else two records (18944 x 3584 10.5 vs 10.9,
  // 3584 x 3584 5.1 vs 5.3, 5120 x 5120 7.3 vs 7.5).
  const int nwaves = p.TW * p.KW;
  const bool own = p.TW == 1 && ceil_div(nblk, p.KW) * MP <= kXPre;
  const bool spread = nblk * MP <= kXPre * nwaves;
  const bool full = MP == 1 && nblk >= 3 * nwaves;
  // Exact ring waits for two to four tokens when each wave streams >= 12 records (two to four
  // tokens, 18944 x 3584, 14 records: 11.3 / 13.8 / 13.8 us against 12.0 / 14.4 / 14.4; 25600 x
  // 5120, 20 records: 15.9 / 18.1 / 18.7 against 16.9 / 19.0 / 19.5). With shorter parts the
  // repeated loads cost more than the exact waits save (3584 x 18944, 10 records: 14.6 / 19.0 /
  // 19.1 against 14.2 / 18.2 / 18.4), and one token is faster with the conditional refill at
  // every shape (gate/up 10.2 against 11.5 us, 152064 x 3584 47 against 54 us).
  const bool exact = MP > 1 && ceil_div(nblk, p.KW) >= 12;
  if (p.lds_x) {
    if (swiglu) {
      if (spread) {
        if (full) FHIP_I8_LAUNCH(true, true, kXSpread, MP == 1 ? 4 : 2);
        else FHIP_I8_LAUNCH(true, true, kXSpread, 2);
      } else {
        FHIP_I8_LAUNCH(true, true, kXLate, 2);
      }
    } else if (own) {
      if (full) FHIP_I8_LAUNCH(true, false, kXOwn, MP == 1 ? 4 : 2);
      else FHIP_I8_LAUNCH(true, false, kXOwn, 2);
    } else if (spread) {
      if (full) FHIP_I8_LAUNCH(true, false, kXSpread, MP == 1 ? 4 : 2);
      else FHIP_I8_LAUNCH(true, false, kXSpread, 2);
    } else {
      FHIP_I8_LAUNCH(true, false, kXLate, 2);
    }
  } else {
    if (swiglu) FHIP_I8_LAUNCH(false, true, kXLate, 2);
    else FHIP_I8_LAUNCH(false, false, kXLate, 2);
  }
#undef FHIP_I8_LAUNCH
#undef FHIP_I8_LAUNCH_EX
  FHIP_CHECK_LAUNCH("q4k_gemv_i8_kernel");
  return FHIP_OK;
}

int launch_i8_any(const GemvGroup &g, const float *X, int K, int M, bool swiglu = false,
                  void *ws = nullptr) {
  if (M == 1) return launch_i8<1>(g, X, K, M, swiglu, ws);
  if (M == 2) return launch_i8<2>(g, X, K, M, swiglu, ws);
  if (M <= 4) return launch_i8<4>(g, X, K, M, swiglu, ws);
  return fail(FHIP_EINVAL, "q4k_gemv: the int8 kernel takes 1..4 tokens, not %d", M);
}

// First width on the 5..16-token kernel: 5, or 3 for K >= 24576, where the int8 kernel's
// four-token workgroups measured 36-37 us on a 5120 x 25600 matrix against 30-32 us (at K = 18944
// and at K = 5120 the int8 kernel stays 20-35% faster). FAK_HIP_GEMV16_FROM (1..5) overrides.
int gemv16_from(int K) {
  const int f = tuning().gemv16_from;
  return f ? f : K >= 24576 ? 3 : 5;
}

}  // namespace

void gemv_shape(int ntiles, int nblk, int max_waves, size_t lds_fixed, size_t lds_per_wave,
                int &TW, int &KW) {
  i8_shape(ntiles, nblk, max_waves, lds_fixed, lds_per_wave, TW, KW);
}

// Workspace bytes of a 1..4-token call over `ntiles` tiles with reduction dim K (see I8Plan).
size_t gemv_i8_ws_bytes(int ntiles, int K, int M, bool swiglu) {
  I8Plan p = M == 1 ? plan_i8<1>(ntiles, K, swiglu)
           : M == 2 ? plan_i8<2>(ntiles, K, swiglu)
                    : plan_i8<4>(ntiles, K, swiglu);
  return p.xop_bytes;
}

// The one-token launch shape (TW tiles x KW waves per workgroup) over `ntiles` tiles.
void q4k_gemv1_shape(int ntiles, int K, int &TW, int &KW) {
  const I8Plan p = plan_i8<1>(ntiles, K, false);
  TW = p.TW;
  KW = p.KW;
}

// Scratch bytes of a 1..16-token Q4_K matmul of an [N, K] weight (the route q4k_gemv takes).
size_t q4k_gemv_ws_bytes(int N, int K, int M) {
  if (M >= gemv16_from(K)) return gemv16_ws_bytes(0, N, K, M);
  return gemv_i8_ws_bytes(q4k_tiles(N), K, M, false);
}

// Small-M entry: 1..4 tokens on the int8 kernel, 5..16 (3..16 for K >= 24576) on the 32x32 MFMA
// kernel of q4k_gemv16.hip.
int q4k_gemv(const void *Wv, const float *X, float *Y, int N, int K, int M) {
  if (M < 1 || M > 16) return fail(FHIP_EINVAL, "q4k_gemv: M=%d outside 1..16", M);
  if (M >= gemv16_from(K)) return q4k_gemv16(Wv, X, Y, N, K, M);
  GemvGroup g = {};
  g.W[0] = (const uint8_t *)Wv;
  g.Y[0] = Y;
  g.N[0] = N;
  g.tile0[0] = 0;
  g.tile0[1] = q4k_tiles(N);
  g.count = 1;
  return launch_i8_any(g, X, K, M);
}

// A group (1..kMaxGroup members, one activation): one grid over all members' tiles for 1..4
// tokens; wider batches run the members one after another.
int q4k_gemv_group(const GemvGroup &g, const float *X, int K, int M) {
  if (M < 1 || M > 16) return fail(FHIP_EINVAL, "q4k_gemv_group: M=%d outside 1..16", M);
  if (M > 4) {
    for (int i = 0; i < g.count; ++i)
      if (int rc = q4k_gemv16(g.W[i], X, g.Y[i], g.N[i], K, M)) return rc;
    return FHIP_OK;
  }
  return launch_i8_any(g, X, K, M);
}

// The first stage of the fused decode MLP: inter[t][i] = silu(gate x_t)[i] * (up x_t)[i] for
// 1..4 tokens in one launch. ws: gemv_i8_ws_bytes(2 * q4k_tiles(I), K, M, true) bytes.
int q4k_gemv_swiglu(const void *gate, const void *up, const float *X, float *inter, int I, int K,
                    int M, void *ws) {
  if (M < 1 || M > 4) return fail(FHIP_EINVAL, "q4k_gemv_swiglu: M=%d outside 1..4", M);
  GemvGroup g = {};
  g.W[0] = (const uint8_t *)gate;
  g.W[1] = (const uint8_t *)up;
  g.Y[0] = g.Y[1] = inter;
  g.N[0] = g.N[1] = I;
  g.tile0[0] = 0;
  g.tile0[1] = q4k_tiles(I);
  g.tile0[2] = 2 * q4k_tiles(I);
  g.count = 2;
  return launch_i8_any(g, X, K, M, true, ws);
}

}  // namespace fhip
