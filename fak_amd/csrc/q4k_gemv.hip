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
//   * activation operand: every 32-value sub-block of a token is quantized to two int8 digits,
//     x ~= e * (q1 + q2 / 256) = e * T / 256 with e the smallest power of two >= max|x| / 127
//     and T = rint(256 x / e). The error is at most e / 512 per value (< 3.1e-5 of the block's
//     largest magnitude), integer activations are exact, and the int32 products of both digits
//     are exact. S_s is the f32 sum of the unquantized values.
//
// Accumulator layout. One MFMA covers one 32-byte chunk c of a row's nibbles (sub-block 2c in
// the low nibbles, 2c + 1 in the high nibbles) for the 16 rows of a tile. Its 16 operand rows
// stand for (sub-block, token, digit) triples, so the four chunks of a super-block accumulate
// into the SAME result: each lane loads its activation digits only into the operand of the MFMA
// whose sub-block owns the lane's row (an exec-masked LDS read) and the other operands keep
// zeros in that lane. For one token the 16 rows are the 8 sub-blocks x 2 digits, every result
// lane is useful, and result lane group g holds sub-blocks g and g + 4 of the 16 output rows.
// Two tokens use two results (sub-blocks 0-3, 4-7), four tokens one result per chunk.
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
#include "gemv_common.hpp"

namespace fhip {
namespace {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

// ---- Activation operand layout for MP (1, 2, 4) token rows --------------------------------
// Per super-block: MP result blocks of 16 rows x 4 lane groups x 16 bytes (entry index
// ((bl * MP + blk) * 16 + row) * 4 + g), then per (sub-block, token) a float2 {e, S}.
// Row `row` of block `blk` holds digit k of token t for sub-block sig (positions 8g..8g+7 of
// the sub-block in bytes 0-7 when sig is even, bytes 8-15 when odd; the other half is zero).
template <int MP>
__host__ __device__ constexpr int blk_of(int sig) {
  return MP == 1 ? 0 : MP == 2 ? sig >> 2 : sig >> 1;
}
template <int MP>
__host__ __device__ constexpr int row_of(int sig, int t, int k) {
  return MP == 1 ? 4 * (sig & 3) + 2 * (sig >> 2) + k
       : MP == 2 ? 4 * (sig & 3) + 2 * t + k
                 : 8 * (sig & 1) + 2 * t + k;
}
// Inverse: result block `blk`, lane group gq, pair p (result elements 2p, 2p + 1 = digits 0, 1)
// hold sub-block 4 * sig_hi + sig_q and token tok_of.
template <int MP>
__host__ __device__ constexpr bool sig_hi(int blk, int p) {
  return MP == 1 ? p == 1 : MP == 2 ? blk == 1 : blk >= 2;
}
template <int MP>
__host__ __device__ constexpr int sig_q(int blk, int gq) {
  return MP == 4 ? 2 * (blk & 1) + (gq >> 1) : gq;
}
template <int MP>
__host__ __device__ constexpr int tok_of(int gq, int p) {
  return MP == 1 ? 0 : MP == 2 ? p : 2 * (gq & 1) + p;
}
// Index of the {e, S} pair of (sub-block, token); the two pairs a lane reads for one result
// block are adjacent, the first at an even index.
template <int MP>
__host__ __device__ constexpr int es_of(int sig, int t) {
  return MP == 1 ? 2 * (sig & 3) + (sig >> 2) : sig * MP + t;
}
// Bytes of the operands of one super-block.
template <int MP>
__host__ __device__ constexpr size_t op_bytes() { return (size_t)MP * 1024 + (size_t)MP * 64; }


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

// Quantize the 32 values v of sub-block sig of token t into the layout above.
// A: operand entries of super-block slot bl; ES: its {e, S} pairs.
template <int MP>
__device__ __forceinline__ void quant_vals(const float (&v)[32], int sig, int t,
                                           uint4 *__restrict__ A, float2 *__restrict__ ES) {
  uint32_t mb = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i)
    mb = max(mb, absmax4_bits(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]));
  const float amax = __uint_as_float(mb);  // a NaN when the block holds one
  const float s = block_sum(v);
  // e = 2^k, the smallest power of two with 127 e >= amax (amax = f 2^E, f in [0.5, 1)), so
  // x / e is exact and integer activations quantize without error. Non-finite blocks get
  // e = NaN, which carries into every output that uses them.
  int E;
  const float f = frexpf(amax, &E);
  const int k = E - 7 + (f > 127.f / 128.f ? 1 : 0);
  float e = amax > 0.f ? ldexpf(1.f, k) : 0.f;
  if (!(amax <= 3.4e38f)) e = __builtin_nanf("");
  ES[es_of<MP>(sig, t)] = make_float2(e, s);

  // T = rint(256 x / e), |T| <= 32512, so x ~= e T / 256 to within e / 512. The digits are
  // q1 = (T + 128) >> 8 (byte 1 of T + 128) and q2 = T - 256 q1 in [-128, 127] (the low byte
  // of T), as two's complement bytes: q1 + q2 / 256 = T / 256 exactly (digits4). Each lane
  // group's eight values are written as soon as they are packed.
  const int sh = 8 - k;
  const int blk = blk_of<MP>(sig);
  uint4 *row0 = A + ((size_t)blk * 16 + row_of<MP>(sig, t, 0)) * 4;
  uint4 *row1 = A + ((size_t)blk * 16 + row_of<MP>(sig, t, 1)) * 4;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    uint32_t a0, a1, c0, c1;
    digits4(v[8 * g], v[8 * g + 1], v[8 * g + 2], v[8 * g + 3], sh, a0, c0);
    digits4(v[8 * g + 4], v[8 * g + 5], v[8 * g + 6], v[8 * g + 7], sh, a1, c1);
    row0[g] = (sig & 1) ? make_uint4(0, 0, a0, a1) : make_uint4(a0, a1, 0, 0);
    row1[g] = (sig & 1) ? make_uint4(0, 0, c0, c1) : make_uint4(c0, c1, 0, 0);
  }
}

// Quantize one 32-value sub-block of one token (zeros when !valid) into the layout above.
template <int MP>
__device__ __forceinline__ void quant_block(const float *__restrict__ x, bool valid, int sig,
                                            int t, uint4 *__restrict__ A,
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
// (digits4s) unless a lane's scale 2^(8 - k) is not a normal float (blocks below ~2^-120, where
// the wave takes ldexpf).
template <int MP>
__device__ __forceinline__ void quant_lanes(const float4 v, int lane, int t,
                                            uint4 *__restrict__ A, float2 *__restrict__ ES) {
  const int sig = lane >> 3, p = lane & 7;
  uint32_t mb = absmax4_bits(v.x, v.y, v.z, v.w);
  mb = max(mb, FHIP_DPP_U(mb, 0xB1));   // quad_perm [1,0,3,2]: lane ^ 1
  mb = max(mb, FHIP_DPP_U(mb, 0x4E));   // quad_perm [2,3,0,1]: lane ^ 2
  mb = max(mb, FHIP_DPP_U(mb, 0x141));  // row_half_mirror: the other quad of the eight
  const float amax = __uint_as_float(mb);  // a NaN when the block holds one
  float sum = quad_sum(v.x, v.y, v.z, v.w);
  sum = sum + FHIP_DPP(sum, 0xB1);
  sum = sum + FHIP_DPP(sum, 0x4E);
  sum = sum + FHIP_DPP(sum, 0x141);
  int E;
  const float f = frexpf(amax, &E);
  const int k = E - 7 + (f > 127.f / 128.f ? 1 : 0);
  float e = amax > 0.f ? ldexpf(1.f, k) : 0.f;
  if (!(amax <= 3.4e38f)) e = __builtin_nanf("");
  if (p == 0) ES[es_of<MP>(sig, t)] = make_float2(e, sum);
  uint32_t a, c;
  const int sh = 8 - k;
  if (__builtin_expect(__builtin_amdgcn_ballot_w64(sh > 127) == 0, 1))
    digits4s(v.x, v.y, v.z, v.w, ldexpf(1.f, sh), a, c);
  else
    digits4(v.x, v.y, v.z, v.w, sh, a, c);
  const int blk = blk_of<MP>(sig), g = p >> 1, half = p & 1;
  uint32_t *row0 = reinterpret_cast<uint32_t *>(A + ((size_t)blk * 16 + row_of<MP>(sig, t, 0)) * 4 + g);
  uint32_t *row1 = reinterpret_cast<uint32_t *>(A + ((size_t)blk * 16 + row_of<MP>(sig, t, 1)) * 4 + g);
  const int dw = 2 * (sig & 1) + half, dz = 2 * ((sig & 1) ^ 1) + half;
  row0[dw] = a;
  row0[dz] = 0u;
  row1[dw] = c;
  row1[dz] = 0u;
}

// Quantize super-blocks [s0, s0 + nb) of M tokens (tokens M..MP-1 zero) into slots 0..nb-1 of
// the operand buffers, `lane` of `nlanes` threads sharing the work.
template <int MP>
__device__ __forceinline__ void quant_range(const float *__restrict__ X, int K, int M, int s0,
                                            int nb, uint4 *__restrict__ A, float2 *__restrict__ ES,
                                            int lane, int nlanes) {
  const int per_t = nb * 8;
  for (int task = lane; task < per_t * MP; task += nlanes) {
    const int t = task / per_t, rest = task - t * per_t;
    const int bl = rest >> 3, sig = rest & 7;
    const bool valid = t < M;
    quant_block<MP>(X + (valid ? (size_t)t * K + 256 * (size_t)(s0 + bl) + 32 * sig : 0), valid,
                    sig, t, A + (size_t)bl * MP * 64, ES + (size_t)bl * 8 * MP);
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

// silu(z) = z / (1 + e^-z) with e^-z evaluated in double and rounded to f32, the operation
// order of internal/model/forward.go:452.
__device__ __forceinline__ float silu_f32(float z) {
  return z / (1.f + (float)exp(-(double)z));
}

// Weight records each wave keeps in flight (LDS path) and the widest workgroup (waves) for one
// token. Measured at the 7B FFN shapes: an 8-record ring with 8-wave workgroups, the
// activation loads issued ahead of the ring, and lane-parallel coalesced quantization were all
// slower (11.9-12 us gate/up, 14.7-15.1 us down, against 10.6 and 13.8 us here).
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
    const GemvGroup grp, const float *__restrict__ X, const uint4 *__restrict__ xg, int K, int M,
    int nblk, int TW, int KW) {
  constexpr int NT = MP == 1 ? 1 : 2;  // token slots per lane
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
  const unsigned char *opb = LX ? smem : reinterpret_cast<const unsigned char *>(xg);
  const uint4 *A = reinterpret_cast<const uint4 *>(opb);
  const float2 *ES = reinterpret_cast<const float2 *>(opb + (size_t)nblk * MP * 1024);
  float *red = reinterpret_cast<float *>(smem + (LX ? (size_t)nblk * op_bytes<MP>() : 0));

  // A lane's operand row belongs to one chunk per result block; with one or two tokens the
  // lane loads only for the MFMA of that chunk.
  auto lane_chunk = [&](int blk) {
    const int p = (r >> 1) & 1;
    const int sig = 4 * (sig_hi<MP>(blk, p) ? 1 : 0) + sig_q<MP>(blk, r >> 2);
    return sig >> 1;
  };
  auto a_index = [&](int slot, int m) {  // this lane's entry for the MFMA of chunk m
    const int blk = m * MP / 4;
    return ((size_t)(slot * MP + blk) * 16 + r) * 4 + gq;
  };
  auto es_index = [&](int slot, int blk) {  // float4 holding this lane's two {e, S} pairs
    return ((size_t)slot * 8 * MP +
            es_of<MP>(4 * (sig_hi<MP>(blk, 0) ? 1 : 0) + sig_q<MP>(blk, gq), tok_of<MP>(gq, 0))) /
           2;
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
#pragma unroll
      for (int m = 0; m < 4; ++m) o.a[m] = __builtin_bit_cast(i32x4, A[a_index(b, m)]);
#pragma unroll
      for (int blk = 0; blk < MP; ++blk)
        o.es[blk] = reinterpret_cast<const float4 *>(ES)[es_index(b, blk)];
    }
  };

  constexpr int PF = LX ? (MP == 1 ? kPF1 : 4) : 2;
  Ops ring[PF];
#pragma unroll
  for (int u = 0; u < PF; ++u) {
    if (!LX)
#pragma unroll
      for (int m = 0; m < 4; ++m) ring[u].a[m] = i32x4{0, 0, 0, 0};
    if (!xpre || u < PF0) load(min(b0 + u, b1 - 1), ring[u]);  // a repeat is never used
  }
  // With the first records in flight, the workgroup quantizes the activations of its K range.
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
                            const_cast<uint4 *>(A) + (size_t)(ob0 + i) * MP * 64,
                            const_cast<float2 *>(ES) + (size_t)(ob0 + i) * 8 * MP);
    } else if (xpre) {
#pragma unroll
      for (int j = 0; j < kXPre; ++j) {
        const int c = wave + j * nwaves;
        if (c < nchunk) {
          const int t = chunk_tok(c), bl = c - t * nblk;
          const float4 z = {0.f, 0.f, 0.f, 0.f};
          quant_lanes<MP>(MP == 1 || t < M ? xv[j] : z, lane, t, const_cast<uint4 *>(A) + (size_t)bl * MP * 64,
                          const_cast<float2 *>(ES) + (size_t)bl * 8 * MP);
        }
      }
    } else {
      quant_range<MP>(X, K, M, 0, nblk, const_cast<uint4 *>(A), const_cast<float2 *>(ES),
                      threadIdx.x, blockDim.x);
    }
    if (!xown) __syncthreads();
    if (xpre)
#pragma unroll
      for (int u = PF0; u < PF; ++u) load(min(b0 + u, b1 - 1), ring[u]);
  }
  const uint32_t k0F = 0x0F0F0F0Fu;

  // LDS path: the activation operands of the current super-block. Lanes that a given MFMA does
  // not load for keep zeros there for the whole kernel.
  i32x4 areg[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) areg[m] = i32x4{0, 0, 0, 0};

  float acc[NT];
#pragma unroll
  for (int s = 0; s < NT; ++s) acc[s] = 0.f;

  for (int bb = b0; bb < b1; bb += PF) {
#pragma unroll
    for (int u = 0; u < PF; ++u) {
      const int b = bb + u;
      if (b >= b1) break;
      // This slot's three loads are older than the other slots' refills: saying so lets the
      // compiler wait for just this record instead of draining the ring at the top of a pass.
      if (LX) __builtin_amdgcn_s_waitcnt(0x0F70 | (3 * (PF - 1)));
      else __builtin_amdgcn_s_waitcnt(0x0F70 | ((7 + MP) * (PF - 1)));  // < 16 loads: PF = 2
      Ops &cur = ring[u];

      float4 es[MP];
      if (LX) {
#pragma unroll
        for (int m = 0; m < 4; ++m)
          if (MP == 4 || lane_chunk(m * MP / 4) == m)
            areg[m] = __builtin_bit_cast(i32x4, A[a_index(b, m)]);
#pragma unroll
        for (int blk = 0; blk < MP; ++blk)
          es[blk] = reinterpret_cast<const float4 *>(ES)[es_index(b, blk)];
      } else {
#pragma unroll
        for (int m = 0; m < 4; ++m)
          areg[m] = MP == 4 || lane_chunk(m * MP / 4) == m ? cur.a[m] : i32x4{0, 0, 0, 0};
#pragma unroll
        for (int blk = 0; blk < MP; ++blk) es[blk] = cur.es[blk];
      }

      // Weight operands: chunk c = words 2c, 2c+1 of the lane's 32 bytes (8 nibble positions
      // of the chunk), low nibbles -> slots 0-7 (sub-block 2c), high -> slots 8-15 (2c + 1).
      const uint32_t q[8] = {cur.qa.x, cur.qa.y, cur.qa.z, cur.qa.w,
                             cur.qb.x, cur.qb.y, cur.qb.z, cur.qb.w};
      i32x4 D[MP];
#pragma unroll
      for (int blk = 0; blk < MP; ++blk) D[blk] = i32x4{0, 0, 0, 0};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const i32x4 B = {(int)(q[2 * c] & k0F), (int)(q[2 * c + 1] & k0F),
                         (int)((q[2 * c] >> 4) & k0F), (int)((q[2 * c + 1] >> 4) & k0F)};
        const int blk = c * MP / 4;
        D[blk] = __builtin_amdgcn_mfma_i32_16x16x64_i8(areg[c], B, D[blk], 0, 0, 0);
      }
      // The slot is refilled with the record PF ahead as soon as its operands are consumed;
      // the header words are kept for the scaling below.
      const uint4 h = cur.h;
      if (EX)
        load(min(b + PF, b1 - 1), cur);
      else if (b + PF < b1)
        load(b + PF, cur);

      const float dd = (float)__builtin_bit_cast(_Float16, (uint16_t)(h.x & 0xffffu));
      const float dmn = (float)__builtin_bit_cast(_Float16, (uint16_t)(h.x >> 16));
      float xs[NT], vs[NT];
#pragma unroll
      for (int s = 0; s < NT; ++s) xs[s] = vs[s] = 0.f;
#pragma unroll
      for (int blk = 0; blk < MP; ++blk)
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          float sc, mn;
          scale_min(h.y, h.z, h.w, sig_hi<MP>(blk, p), sig_q<MP>(blk, gq), sc, mn);
          const float val = fmaf((float)D[blk][2 * p + 1], 1.f / 256.f, (float)D[blk][2 * p]);
          const float e = p ? es[blk].z : es[blk].x;
          const float S = p ? es[blk].w : es[blk].y;
          const int s = MP == 1 ? 0 : p;
          xs[s] = fmaf(sc, e * val, xs[s]);
          vs[s] = fmaf(mn, S, vs[s]);
        }
#pragma unroll
      for (int s = 0; s < NT; ++s) acc[s] = fmaf(dd, xs[s], fmaf(-dmn, vs[s], acc[s]));
    }
  }

  // Partials of the KW parts go through LDS; part 0 sums them in part order (deterministic),
  // then adds the lane groups that hold the same (token, row): all four (one or two tokens)
  // or g and g ^ 2 (four tokens).
#pragma unroll
  for (int s = 0; s < NT; ++s) red[((tile * KW + part) * NT + s) * 64 + lane] = acc[s];
  __syncthreads();
  const int row = T * 16 + r;
  const bool fin = part == 0 && tvalid;
  if (!SWIGLU && !fin) return;
  float v[NT];
#pragma unroll
  for (int s = 0; s < NT; ++s) {
    v[s] = acc[s];
    for (int q = 1; q < KW; ++q) v[s] += red[((tile * KW + q) * NT + s) * 64 + lane];
    v[s] += __shfl_xor(v[s], 32);
    if (MP <= 2) v[s] += __shfl_xor(v[s], 16);
  }
  if (SWIGLU) {
    // Every wave reaches this barrier; the up tile's final values go through LDS to its gate
    // partner (tile + 1 holds up tile T when tile holds gate tile T).
    float *xch = red + (size_t)blockDim.x / 64 * NT * 64;
    if (fin)
#pragma unroll
      for (int s = 0; s < NT; ++s) xch[(tile * NT + s) * 64 + lane] = v[s];
    __syncthreads();
    if (!fin || mem != 0) return;
    if (row < N && gq < (MP == 4 ? 2 : 1)) {
#pragma unroll
      for (int s = 0; s < NT; ++s) {
        const int t = tok_of<MP>(gq, s);
        if (t < M) Y[(size_t)t * N + row] = silu_f32(v[s]) * xch[((tile + 1) * NT + s) * 64 + lane];
      }
    }
    return;
  }
  if (row < N && gq < (MP == 4 ? 2 : 1)) {
#pragma unroll
    for (int s = 0; s < NT; ++s) {
      const int t = tok_of<MP>(gq, s);
      if (t < M) Y[(size_t)t * N + row] = v[s];
    }
  }
}

// Global-path operand writer: one thread per (token, 32-value sub-block) of all of K.
template <int MP>
__global__ void gemv_i8_prep_kernel(const float *__restrict__ X, int K, int M, int nblk,
                                    uint4 *__restrict__ A) {
  const int id = blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= MP * nblk * 8) return;
  const int per_t = nblk * 8;
  const int t = id / per_t, rest = id - t * per_t;
  const int b = rest >> 3, sig = rest & 7;
  float2 *ES = reinterpret_cast<float2 *>(reinterpret_cast<unsigned char *>(A) +
                                          (size_t)nblk * MP * 1024);
  const bool valid = t < M;
  quant_block<MP>(X + (valid ? (size_t)t * K + 256 * (size_t)b + 32 * sig : 0), valid, sig, t,
                  A + (size_t)b * MP * 64, ES + (size_t)b * 8 * MP);
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
  constexpr int NT = MP == 1 ? 1 : 2;
  const int nblk = K / 256;
  const int max_waves = MP == 1 ? kMaxWaves1 : 8;
  I8Plan p{};
  const size_t ldsx = (size_t)nblk * op_bytes<MP>();
  i8_shape(ntiles, nblk, max_waves, ldsx, (size_t)64 * NT * 4, p.TW, p.KW);
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
      (size_t)p.TW * p.KW * 64 * NT * 4 + (swiglu ? (size_t)p.TW * 64 * NT * 4 : 0);
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
  const uint4 *xg = nullptr;
  if (!p.lds_x) {
    const int nprep = MP * nblk * 8;
    gemv_i8_prep_kernel<MP><<<ceil_div(nprep, 128), 128, 0, stream()>>>(X, K, M, nblk,
                                                                        (uint4 *)xop);
    FHIP_CHECK_LAUNCH("gemv_i8_prep_kernel");
    xg = (const uint4 *)xop;
  }
#define FHIP_I8_LAUNCH_EX(LXV, SWV, XMV, PF0V, EXV)                                          \
  q4k_gemv_i8_kernel<MP, LXV, SWV, XMV, PF0V, EXV><<<grid, threads, p.lds_bytes, stream()>>>( \
      g, X, xg, K, M, nblk, p.TW, p.KW)
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
