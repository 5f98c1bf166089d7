// q6k.hip — GGUF Q6_K weights on the device: the tiled upload, the bit-exact dequantizer and
// the int8-MFMA GEMV.
//
// Q6_K super-block (256 weights, 210 bytes; internal/model/quant_kquant.go:45,139-163):
//   [0, 128)    ql: low 4 bits; [128, 192) qh: high 2 bits; [192, 208) 16 int8 scales;
//   [208, 210)  f16 d.
// Weight n + l + 32 i (half n in {0, 128}, l < 32, i < 4) takes the low (i < 2) or high
// (i >= 2) nibble of ql[n/2 + l + 32 (i & 1)], bits 2i..2i+1 of qh[n/4 + l] as bits 4-5, and
// scale sc[n/16 + l/16 + 2i]: w = (d * f32(sc)) * f32(q - 32).
//
// The upload repacks the rows into the tiled layout of tiled.hpp (a byte permutation). The
// GEMV follows the Q4_K int8 GEMV (q4k_gemv.hip): per group j of 16 weights,
//   sum_k w x = d sc_j (sum_k q x - 32 S_j),    S_j = sum_k x,
// with sum_k q x on v_mfma_i32_16x16x64_i8. The weight operand is the 6-bit code q (0..63) as
// an int8, rebuilt per lane from its 16 ql bytes (a nibble) and 16 qh bytes (a 2-bit field);
// the activation operand is every 16-value group quantized to two int8 digits, x ~= e T / 256
// with e the smallest power of two >= max|x| / 127 and T = rint(256 x / e) (error <= e / 512).
// The 16 rows of an activation operand are (group, digit) pairs of 8 groups, so one result
// block holds 8 groups of the 16 rows of a tile: two result blocks (halves h = 0, 1) per
// super-block, each the sum of two MFMAs (k = 0, 1: group 8h + 4k + g in lane group g).
#include "f16bits.hpp"
#include "kernels.hpp"

namespace fhip {
namespace {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

// Activation operands per super-block: 16 groups x 2 digit rows x 16 bytes, then 16 {e, S}.
constexpr int kQ6Op = 16 * 2 * 16 + 16 * 8;  // 640

__device__ __forceinline__ int q6_code(uint32_t ql, uint32_t qh, int i) {
  const uint32_t lo = (i >= 2 ? ql >> 4 : ql) & 0x0fu;
  return (int)(lo | (((qh >> (2 * i)) & 3u) << 4)) - 32;
}

// Tiled record byte o (0 .. 3359) holds byte `src` of row r's 210-byte super-block.
__device__ __forceinline__ void q6_tiled_source(int o, int &r, int &src) {
  if (o < kQ6kD) {  // scales
    r = o >> 4;
    src = 192 + (o & 15);
  } else if (o < kQ6kQl) {  // d
    r = (o - kQ6kD) >> 1;
    src = 208 + ((o - kQ6kD) & 1);
  } else if (o < kQ6kQh) {  // ql: (h, lane = 16 g + r, pos)
    const int u = o - kQ6kQl, h = u >> 10, l = (u >> 4) & 63, pos = u & 15;
    r = l & 15;
    src = 64 * h + 16 * (l >> 4) + pos;
  } else {  // qh: (h, g1, r, pos)
    const int u = o - kQ6kQh, h = u >> 9, g1 = (u >> 8) & 1, pos = u & 15;
    r = (u >> 4) & 15;
    src = 128 + 32 * h + 16 * g1 + pos;
  }
}

// One thread per 16-byte unit of the tiled buffer (210 units per record).
__global__ void q6k_repack_kernel(uint8_t *__restrict__ dst, const uint8_t *__restrict__ raw,
                                  int N, int nblk, long long units) {
  const long long id = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= units) return;
  const long long rec = id / (kQ6kRecord / 16);
  const int u = (int)(id - rec * (kQ6kRecord / 16));
  const int T = (int)(rec / nblk), b = (int)(rec - (long long)T * nblk);
  uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    int r, src;
    q6_tiled_source(16 * u + i, r, src);
    const int row = 16 * T + r;
    const uint32_t v = row < N ? raw[((size_t)row * nblk + b) * kQ6kBlock + src] : 0u;
    w[i >> 2] |= v << (8 * (i & 3));
  }
  reinterpret_cast<uint4 *>(dst)[id] = make_uint4(w[0], w[1], w[2], w[3]);
}

// The inverse: one thread per byte of the raw rows.
__global__ void q6k_unpack_kernel(uint8_t *__restrict__ raw, const uint8_t *__restrict__ tiled,
                                  int nblk, long long bytes) {
  const long long id = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= bytes) return;
  const long long blk = id / kQ6kBlock;
  const int src = (int)(id - blk * kQ6kBlock);
  const int row = (int)(blk / nblk), b = (int)(blk - (long long)row * nblk);
  const int T = row >> 4, r = row & 15;
  int o;
  if (src < 128) {  // ql byte 64 h + 16 g + pos
    const int h = src >> 6, g = (src >> 4) & 3, pos = src & 15;
    o = kQ6kQl + 1024 * h + 16 * (16 * g + r) + pos;
  } else if (src < 192) {  // qh byte 32 h + 16 g1 + pos
    const int q = src - 128, h = q >> 5, g1 = (q >> 4) & 1, pos = q & 15;
    o = kQ6kQh + 512 * h + 256 * g1 + 16 * r + pos;
  } else if (src < 208) {
    o = 16 * r + (src - 192);
  } else {
    o = kQ6kD + 2 * r + (src - 208);
  }
  raw[id] = tiled[((size_t)T * nblk + b) * kQ6kRecord + o];
}

// One thread per (row, super-block): the 256 weights exactly as q6kDequantSuperBlock computes
// them, read from the tiled record.
__global__ void q6k_dequant_kernel(float *__restrict__ dw, const uint8_t *__restrict__ W, int N,
                                   int nblk) {
  const long long id = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= (long long)N * nblk) return;
  const int row = (int)(id / nblk), b = (int)(id - (long long)row * nblk);
  const int r = row & 15;
  const uint8_t *rec = W + ((size_t)(row >> 4) * nblk + b) * kQ6kRecord;
  const int8_t *sc = reinterpret_cast<const int8_t *>(rec + 16 * r);
  const float d = f16_bits_to_f32(rec[kQ6kD + 2 * r] | (rec[kQ6kD + 2 * r + 1] << 8));
  float *o = dw + (size_t)row * nblk * 256 + (size_t)b * 256;
  for (int h = 0; h < 2; ++h)
    for (int l = 0; l < 32; ++l) {
      // ql bytes 64 h + l and 64 h + 32 + l, qh byte 32 h + l, at their tiled places
      const int x0 = l, x1 = l + 32;
      const uint32_t q0 = rec[kQ6kQl + 1024 * h + 16 * (16 * (x0 >> 4) + r) + (x0 & 15)];
      const uint32_t q1 = rec[kQ6kQl + 1024 * h + 16 * (16 * (x1 >> 4) + r) + (x1 & 15)];
      const uint32_t hh = rec[kQ6kQh + 512 * h + 256 * (l >> 4) + 16 * r + (l & 15)];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int q = q6_code(i & 1 ? q1 : q0, hh, i);
        o[128 * h + l + 32 * i] = __fmul_rn(__fmul_rn(d, (float)sc[8 * h + l / 16 + 2 * i]),
                                           (float)q);
      }
    }
}

// Quantize group j (16 values at x) of one super-block into its operand slot `op`.
__device__ __forceinline__ void q6_quant_group(const float *__restrict__ x, int j,
                                               unsigned char *__restrict__ op) {
  float v[16];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float4 f = *reinterpret_cast<const float4 *>(x + 4 * i);
    v[4 * i] = f.x; v[4 * i + 1] = f.y; v[4 * i + 2] = f.z; v[4 * i + 3] = f.w;
  }
  float amax = 0.f, s = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    amax = fmaxf(amax, fabsf(v[i]));
    s += v[i];
  }
  int E;
  const float f = frexpf(amax, &E);
  const int k = E - 7 + (f > 127.f / 128.f ? 1 : 0);
  float e = amax > 0.f ? ldexpf(1.f, k) : 0.f;
  if (!(amax <= 3.4e38f)) e = __builtin_nanf("");
  reinterpret_cast<float2 *>(op + 512)[j] = make_float2(e, s);
  uint4 hi, lo;
  digits4(v[0], v[1], v[2], v[3], 8 - k, hi.x, lo.x);
  digits4(v[4], v[5], v[6], v[7], 8 - k, hi.y, lo.y);
  digits4(v[8], v[9], v[10], v[11], 8 - k, hi.z, lo.z);
  digits4(v[12], v[13], v[14], v[15], 8 - k, hi.w, lo.w);
  reinterpret_cast<uint4 *>(op)[2 * j] = hi;
  reinterpret_cast<uint4 *>(op)[2 * j + 1] = lo;
}

// Global-path operand writer: one thread per group of all of K.
__global__ void q6k_xprep_kernel(const float *__restrict__ x, int nblk,
                                 unsigned char *__restrict__ ops) {
  const int id = blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= nblk * 16) return;
  q6_quant_group(x + 16 * (size_t)id, id & 15, ops + (size_t)(id >> 4) * kQ6Op);
}

// One token: workgroup = TW tiles x KW waves, wave (tile, part) streams super-blocks
// [part nblk / KW, (part + 1) nblk / KW) of its tile with two records in flight. Two keep the
// kernel at 92 VGPRs, five waves per SIMD; three records (112 VGPRs, four waves) measured 4%
// slower and four (134, three waves: one 8-wave workgroup per CU) 8-20% slower (default shapes,
// us for 2 / 3 / 4 records: 18944 x 3584 14.8 / 15.5 / 18.1, 25600 x 5120 20.9 / 21.9 / 25.4,
// 14336 x 4096 10.7 / 11.2 / 11.4, 152064 x 3584 67.6 / 68.7 / 71.3).
template <bool LX>
__global__ __launch_bounds__(512) void q6k_gemv_kernel(const uint8_t *__restrict__ W,
                                                      const float *__restrict__ X,
                                                      const unsigned char *__restrict__ xg,
                                                      float *__restrict__ Y, int N, int nblk,
                                                      int TW, int KW) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int gq = lane >> 4, r = lane & 15;
  const int tile = wave / KW, part = wave - tile * KW;
  const int ntiles = (N + 15) >> 4;
  const int T = blockIdx.x * TW + tile;
  const bool tvalid = T < ntiles;
  const int b0 = part * nblk / KW, b1 = (part + 1) * nblk / KW;
  const int nb = b1 - b0;
  const uint8_t *base = W + (size_t)(tvalid ? T : 0) * nblk * kQ6kRecord;
  const unsigned char *opb = LX ? smem : xg;
  float *red = reinterpret_cast<float *>(smem + (LX ? (size_t)nblk * kQ6Op : 0));

  struct Rec {
    uint4 sc, ql0, ql1, qh0, qh1;
    uint32_t dd;
  };
  auto load = [&](int b, Rec &o) {
    const uint8_t *rec = base + (size_t)b * kQ6kRecord;
    o.sc = ld_stream(rec + 16 * r);
    o.dd = ld_stream32(rec + kQ6kD + 4 * (r >> 1));
    o.ql0 = ld_stream(rec + kQ6kQl + 16 * lane);
    o.ql1 = ld_stream(rec + kQ6kQl + 1024 + 16 * lane);
    o.qh0 = ld_stream(rec + kQ6kQh + 256 * (gq & 1) + 16 * r);
    o.qh1 = ld_stream(rec + kQ6kQh + 512 + 256 * (gq & 1) + 16 * r);
  };
  constexpr int PF = 2;
  Rec ring[PF];
#pragma unroll
  for (int u = 0; u < PF; ++u)
    if (u < nb) load(b0 + u, ring[u]);
  if (LX) {
    for (int t = threadIdx.x; t < nblk * 16; t += blockDim.x)
      q6_quant_group(X + 16 * (size_t)t, t & 15, smem + (size_t)(t >> 4) * kQ6Op);
    __syncthreads();
  }

  // Activation operand of this lane: row r = (group jj = r >> 1, digit r & 1) in lane group gq,
  // non-zero only in the MFMA k = jj >> 2 and only when jj & 3 == gq.
  const int jj = r >> 1, dig = r & 1;
  const bool a_on = (jj & 3) == gq;
  const int a_k = jj >> 2;
  const int sh2 = 2 * (gq >> 1);  // qh field of lane group gq: 4k + sh2
  const uint32_t m0F = in_reg(0x0F0F0F0Fu), m03 = in_reg(0x03030303u);
  float acc = 0.f;

  for (int bb = b0; bb < b1; bb += PF) {
#pragma unroll
    for (int u = 0; u < PF; ++u) {
      const int b = bb + u;
      if (b >= b1) break;
      Rec &cur = ring[u];
      const unsigned char *op = opb + (size_t)b * kQ6Op;
      i32x4 A0 = {0, 0, 0, 0}, A1 = {0, 0, 0, 0};
      if (a_on) {
        A0 = __builtin_bit_cast(i32x4, reinterpret_cast<const uint4 *>(op)[2 * jj + dig]);
        A1 = __builtin_bit_cast(i32x4, reinterpret_cast<const uint4 *>(op)[2 * (8 + jj) + dig]);
      }
      // {e, S} of the result groups of this lane: 8 h + 2 gq + t
      const float4 es0 = reinterpret_cast<const float4 *>(op + 512)[gq];
      const float4 es1 = reinterpret_cast<const float4 *>(op + 512)[4 + gq];
      i32x4 D[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint4 ql = h ? cur.ql1 : cur.ql0, qh = h ? cur.qh1 : cur.qh0;
        const i32x4 Ah = h ? A1 : A0;
        D[h] = i32x4{0, 0, 0, 0};
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          const int s = 4 * k + sh2;
          const uint32_t w[4] = {ql.x, ql.y, ql.z, ql.w}, v[4] = {qh.x, qh.y, qh.z, qh.w};
          i32x4 B;
#pragma unroll
          for (int m = 0; m < 4; ++m)
            B[m] = (int)(((w[m] >> (4 * k)) & m0F) | (((v[m] >> s) & m03) << 4));
          const i32x4 A = a_k == k ? Ah : i32x4{0, 0, 0, 0};
          D[h] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, B, D[h], 0, 0, 0);
        }
      }
      const uint4 sc = cur.sc;
      const uint32_t dd = cur.dd;
      if (b + PF < b1) load(b + PF, cur);

      const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)(dd >> (16 * (r & 1))));
      // scale of group 8 h + 2 gq + t: dword 2 h + (gq >> 1), byte 2 (gq & 1) + t
      float part_sum = 0.f;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint32_t scw = (gq >> 1) ? (h ? sc.w : sc.y) : (h ? sc.z : sc.x);
        const float4 es = h ? es1 : es0;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const int scv = (int8_t)(scw >> (8 * (2 * (gq & 1) + t)));
          const float val = fmaf((float)D[h][2 * t + 1], 1.f / 256.f, (float)D[h][2 * t]);
          const float e = t ? es.z : es.x, S = t ? es.w : es.y;
          part_sum = fmaf((float)scv, fmaf(e, val, -32.f * S), part_sum);
        }
      }
      acc = fmaf(d, part_sum, acc);
    }
  }

  red[(tile * KW + part) * 64 + lane] = acc;
  __syncthreads();
  if (part != 0 || !tvalid) return;
  float v = acc;
  for (int q = 1; q < KW; ++q) v += red[(tile * KW + q) * 64 + lane];
  v += __shfl_xor(v, 16);
  v += __shfl_xor(v, 32);
  const int row = T * 16 + r;
  if (gq == 0 && row < N) Y[row] = v;
}

int check_q6k_shape(const char *who, int out, int in) {
  if (out <= 0 || in <= 0 || in % 256 != 0)
    return fail(FHIP_EINVAL, "%s: need out > 0 and in a positive multiple of 256 (out=%d in=%d)",
                who, out, in);
  return FHIP_OK;
}

// Workgroup shape of the one-token GEMV and whether its activation operands fit in LDS.
struct Q6Plan {
  int TW, KW;
  size_t ldsx, redB;
  bool lds_x;
};

// Shape, measured one token at a time (us): up to one tile per CU, one tile of 8 waves (3584 x
// 3584 5.2 against 5.6 with 4 waves, 4096 x 4096 5.5 / 5.9, 512 x 3584 4.5 / 4.9), each wave
// streaming >= 1.5 records. Up to 8 tiles per CU: the workgroup of 1, 2 or 4 tiles (4, 4 or 2
// waves each) whose grid puts the fewest tiles on the busiest CU, the widest on a tie (its
// activation quantization serves more tiles): 18944 x 3584, 1184 tiles, 1 x 4 12.5 against
// 4 x 2 15.5 (5 against 8 tiles); 11008 x 4096 1 x 4 9.8 / 10.3 (3 against 4); 14336 x 4096, 4
// tiles each way, 4 x 2 / 2 x 4 11.1 against 1 x 4 11.6; 5120 x 25600 2 x 4 26.3 against 1 x 4
// 28.1. Taller matrices take the Q4_K GEMV's rule (152064 x 3584: 2 x 2 68.7, 1 x 4 69.6).
void q6_shape(int ntiles, int nblk, size_t ldsx, int &TW, int &KW) {
  const int cus = cu_count() > 0 ? cu_count() : 256;
  if (tuning().gemv_tw || tuning().gemv_kw || ntiles > 8 * cus) {
    gemv_shape(ntiles, nblk, 8, ldsx, 64 * 4, TW, KW);
    return;
  }
  if (ntiles <= cus) {
    TW = 1;
    KW = 8;
  } else {
    TW = 0;
    int best = 1 << 30;
    for (int tw = 1; tw <= 4; tw *= 2) {
      const int load = tw * ceil_div(ceil_div(ntiles, tw), cus);
      if (load <= best) {
        best = load;
        TW = tw;
      }
    }
    KW = TW == 4 ? 2 : 4;
  }
  while (KW > 1 && 2 * nblk < 3 * KW) KW /= 2;
}

Q6Plan plan_q6k(int N, int K) {
  Q6Plan p{};
  const int nblk = K / 256, ntiles = q4k_tiles(N);
  p.ldsx = (size_t)nblk * kQ6Op;
  q6_shape(ntiles, nblk, p.ldsx, p.TW, p.KW);
  p.redB = (size_t)p.TW * p.KW * 64 * 4;
  p.lds_x = p.ldsx + p.redB <= (size_t)lds_limit();
  return p;
}

int launch_q6k_gemv(const uint8_t *W, const float *x, float *y, int N, int K) {
  const int nblk = K / 256, ntiles = q4k_tiles(N);
  const Q6Plan p = plan_q6k(N, K);
  const int TW = p.TW, KW = p.KW;
  const size_t ldsx = p.ldsx, redB = p.redB;
  const bool lds_x = p.lds_x;
  const int grid = ceil_div(ntiles, TW), threads = 64 * TW * KW;
  if (lds_x) {
    q6k_gemv_kernel<true><<<grid, threads, ldsx + redB, stream()>>>(W, x, nullptr, y, N, nblk,
                                                                    TW, KW);
  } else {
    unsigned char *ops = (unsigned char *)workspace(ldsx);
    if (!ops) return FHIP_ENOMEM;
    if (int rc = check_disjoint("q6k_gemv", x, (size_t)K * 4, ops, ldsx)) return rc;
    q6k_xprep_kernel<<<ceil_div(nblk * 16, 128), 128, 0, stream()>>>(x, nblk, ops);
    FHIP_CHECK_LAUNCH("q6k_xprep_kernel");
    q6k_gemv_kernel<false><<<grid, threads, redB, stream()>>>(W, x, ops, y, N, nblk, TW, KW);
  }
  FHIP_CHECK_LAUNCH("q6k_gemv_kernel");
  return FHIP_OK;
}

}  // namespace

// Q6_K matmul on the tiled layout: one token on the int8 GEMV above, 2..16 tokens in one launch
// of the 32x32 MFMA kernel of q4k_gemv16.hip (max|dY|/RMS <= 1e-3), 17..32 on that kernel's f16
// form (one operand row per token) and more through the f16 MFMA prefill GEMM (q4k_gemm32.hip),
// both within the GEMM bound 1e-2.
size_t q6k_gemv_ws_bytes(int N, int K, int M) {
  if (M > 32) return gemm32_ws_bytes(1, N, K, M);
  if (M > 16) return gemv16_ws_bytes(1, N, K, M);
  if (M > 1) return gemv16_ws_bytes(1, N, K, M);
  const Q6Plan p = plan_q6k(N, K);
  return p.lds_x ? 0 : p.ldsx;
}

int q6k_gemv(const void *dW, const float *dX, float *dY, int out, int in, int P) {
  if (P > 32) return q6k_gemm32(dW, dX, dY, out, in, P);
  if (P > 16) return q6k_gemv32(dW, dX, dY, out, in, P);
  if (P > 1) return q6k_gemv16(dW, dX, dY, out, in, P);
  return launch_q6k_gemv((const uint8_t *)dW, dX, dY, out, in);
}

}  // namespace fhip

using namespace fhip;

extern "C" {

size_t fhip_q6k_bytes(int out, int in) {
  if (out <= 0 || in <= 0 || in % 256) return 0;
  return (size_t)out * (in / 256) * kQ6kBlock;
}

size_t fhip_q6k_packed_bytes(int out, int in) {
  if (out <= 0 || in <= 0 || in % 256) return 0;
  return q6k_packed_bytes(out, in);
}

int fhip_q6k_repack(void *dPacked, const uint8_t *dRaw, int out, int in) {
  clear_error();
  if (int rc = check_q6k_shape("fhip_q6k_repack", out, in)) return rc;
  if (!dPacked || !dRaw) return fail(FHIP_EINVAL, "fhip_q6k_repack: null pointer");
  const int nblk = in / 256;
  const long long units = (long long)q4k_tiles(out) * nblk * (kQ6kRecord / 16);
  untag_range(dPacked, q6k_packed_bytes(out, in));
  q6k_repack_kernel<<<(unsigned)((units + 255) / 256), 256, 0, stream()>>>(
      (uint8_t *)dPacked, dRaw, out, nblk, units);
  FHIP_CHECK_LAUNCH("q6k_repack_kernel");
  tag_weight(dPacked, q6k_packed_bytes(out, in), kWeightQ6K, out, in);
  return FHIP_OK;
}

int fhip_q6k_unpack(uint8_t *dRaw, const void *dPacked, int out, int in) {
  clear_error();
  if (int rc = check_q6k_shape("fhip_q6k_unpack", out, in)) return rc;
  if (!dPacked || !dRaw) return fail(FHIP_EINVAL, "fhip_q6k_unpack: null pointer");
  if (int rc = check_weight("fhip_q6k_unpack", dPacked, kWeightQ6K, out, in)) return rc;
  untag_range(dRaw, fhip_q6k_bytes(out, in));
  const int nblk = in / 256;
  const long long bytes = (long long)out * nblk * kQ6kBlock;
  q6k_unpack_kernel<<<(unsigned)((bytes + 255) / 256), 256, 0, stream()>>>(
      dRaw, (const uint8_t *)dPacked, nblk, bytes);
  FHIP_CHECK_LAUNCH("q6k_unpack_kernel");
  return FHIP_OK;
}

void *fhip_q6k_upload(const uint8_t *hRaw, int out, int in) {
  clear_error();
  if (check_q6k_shape("fhip_q6k_upload", out, in)) return nullptr;
  if (!hRaw) { fail(FHIP_EINVAL, "fhip_q6k_upload: null host pointer"); return nullptr; }
  const size_t raw_bytes = fhip_q6k_bytes(out, in);
  void *raw = fhip_malloc(raw_bytes);
  if (!raw) return nullptr;
  void *d = fhip_malloc(q6k_packed_bytes(out, in));
  if (!d) {
    fhip_free(raw);
    return nullptr;
  }
  const bool ok = fhip_h2d(raw, hRaw, raw_bytes) == FHIP_OK &&
                  fhip_q6k_repack(d, (const uint8_t *)raw, out, in) == FHIP_OK &&
                  hipStreamSynchronize(stream()) == hipSuccess;
  fhip_free(raw);  // the repack has finished (or failed) before the staging buffer is reused
  if (!ok) {
    fhip_free(d);
    return nullptr;
  }
  return d;
}

int fhip_q6k_dequant_f32(float *dW, const void *dPacked, int out, int in) {
  clear_error();
  if (int rc = check_q6k_shape("fhip_q6k_dequant_f32", out, in)) return rc;
  if (!dPacked || !dW) return fail(FHIP_EINVAL, "fhip_q6k_dequant_f32: null pointer");
  if (int rc = check_weight("fhip_q6k_dequant_f32", dPacked, kWeightQ6K, out, in)) return rc;
  untag_range(dW, (size_t)out * in * 4);
  const int nblk = in / 256;
  const long long n = (long long)out * nblk;
  q6k_dequant_kernel<<<(unsigned)((n + 255) / 256), 256, 0, stream()>>>(
      dW, (const uint8_t *)dPacked, out, nblk);
  FHIP_CHECK_LAUNCH("q6k_dequant_kernel");
  return FHIP_OK;
}

int fhip_q6k_matmul_f32(const void *dPacked, const float *dX, float *dY, int out, int in, int P) {
  clear_error();
  if (int rc = check_q6k_shape("fhip_q6k_matmul_f32", out, in)) return rc;
  if (P < 0) return fail(FHIP_EINVAL, "fhip_q6k_matmul_f32: P=%d < 0", P);
  if (P == 0) return FHIP_OK;
  if (!dPacked || !dX || !dY) return fail(FHIP_EINVAL, "fhip_q6k_matmul_f32: null pointer");
  if (((uintptr_t)dX & 15) || ((uintptr_t)dPacked & 15))
    return fail(FHIP_EINVAL, "fhip_q6k_matmul_f32: dX and dPacked must be 16-byte aligned");
  if (int rc = check_weight("fhip_q6k_matmul_f32", dPacked, kWeightQ6K, out, in)) return rc;
  untag_range(dY, (size_t)P * out * 4);
  return q6k_gemv(dPacked, dX, dY, out, in, P);
}

}  // extern "C"
