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
// Device plan. A workgroup owns TW 16-row tiles (tiled.hpp) and a group of up to 16 tokens: one
// tile whose KW waves each take a contiguous part of the super-blocks of a window of records,
// or (KW = 1) TW tiles of one wave each, which share the workgroup's staged activations.
//   * staging: the workgroup quantizes the window's activation blocks exactly as the reference
//     does (q8round.hpp) into LDS: int8 codes and per block {f32(S), dx}. The first weight
//     records of every wave are already in flight meanwhile.
//   * the integer sums run on the int8 MFMA v_mfma_i32_16x16x32_i8, whose K = 32 is exactly one
//     sub-block: A = 16 tokens x 32 codes, B = 32 nibbles x 16 rows, so D[t][row] = I_s. Lane
//     (g, r) feeds the nibbles of row r at positions 8g..8g+7 straight from its tiled 16-byte
//     pieces and the codes of token r at the same positions; result lane (g, r) holds I_s of
//     row r for tokens 4g..4g+3 and forms the two terms T1 = (f32(I) * ws) * dx and
//     T2 = (f32(S) * wm) * dx with the reference's roundings.
//   * the chain: a tile's first wave owns its (row, token) sums and adds the terms of its own
//     part as it makes them; with KW > 1 the other waves park theirs in LDS and the first wave
//     adds them after a barrier, in record order. A window's terms must fit in LDS; long rows or
//     many tokens take several windows, the sums carrying across.
// Weight records stream through a ring of PF in-flight loads per wave (three 16-byte loads per
// lane per record), as in the Q4_K GEMV.
#include "kernels.hpp"
#include "q8round.hpp"

namespace fhip {
namespace {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

constexpr int kTokGroup = 16;         // tokens per workgroup (the MFMA's A rows)

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

// LDS layout of one window of Wrec records for pg tokens:
//   codes  [pg][cstride] int8   (cstride = 256 Wrec + 16: the pad spreads token rows over banks)
//   sd     [pg][8 Wrec] float2  {f32(S), dx} per activation block
//   terms  [pg * 16][tstride] float2 {T1, T2}, (token, row)-major (tstride = 8 Wrec + 2),
//          then 64 float2 where lanes whose token is past the group put theirs; only with KW > 1
struct I8rLds {
  int cstride, tstride;
  size_t codes, sd, terms, dummy, total;
};
__host__ __device__ inline I8rLds i8r_lds(int pg, int Wrec, int KW) {
  I8rLds L;
  L.cstride = 256 * Wrec + 16;
  L.tstride = 8 * Wrec + 2;
  L.codes = 0;
  L.sd = (size_t)pg * L.cstride;
  L.terms = L.sd + (size_t)pg * 8 * Wrec * 8;
  L.dummy = L.terms + (size_t)pg * 16 * L.tstride * 8;
  L.total = KW > 1 ? L.dummy + 64 * 8 : L.terms;
  return L;
}

constexpr int kPF = 4;           // weight records in flight per wave
constexpr int kFusedTokens = 4;  // up to this many tokens each workgroup quantizes its window

// Many tokens: the activation is quantized once into global memory (codes [P][K] and
// {f32(S), dx} [P][K/32]) and each workgroup copies its window from there.
__global__ __launch_bounds__(256) void i8r_prep_kernel(const float *__restrict__ X, int P, int K,
                                                       int8_t *__restrict__ qx,
                                                       float2 *__restrict__ sdg) {
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
  __align__(16) int8_t q[32];
  int s = 0;
  const float d = q8_quant_block32(x, q, &s);
  uint4 *dst = reinterpret_cast<uint4 *>(qx + off);
  dst[0] = *reinterpret_cast<const uint4 *>(q);
  dst[1] = *reinterpret_cast<const uint4 *>(q + 16);
  sdg[id] = make_float2((float)s, d);
}

// fused: the workgroup quantizes its window from X itself (few tokens); otherwise it copies the
// window from qxg / sdg written by i8r_prep_kernel.
template <int NV>
__global__ __launch_bounds__(512) void q4k_i8route_kernel(
    const uint8_t *__restrict__ W, const float *__restrict__ X, const int8_t *__restrict__ qxg,
    const float2 *__restrict__ sdg, float *__restrict__ Y, int N, int K, int nblk, int P,
    int Wrec, int KW, int TW, int fused) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int t0 = blockIdx.y * kTokGroup;
  const int pg = min(kTokGroup, P - t0);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // This wave's tile and its part of the tile's records (TW > 1 only with KW = 1). A wave whose
  // tile is past the matrix streams the last tile and writes nothing.
  const int ntiles = (N + 15) / 16;
  const int tile = blockIdx.x * TW + wave / KW, kwave = wave - (wave / KW) * KW;
  const int gtile = min(tile, ntiles - 1);
  const int g = lane >> 4, r = lane & 15;
  const I8rLds L = i8r_lds(pg, Wrec, KW);
  int8_t *codes = reinterpret_cast<int8_t *>(smem + L.codes);
  float2 *sd = reinterpret_cast<float2 *>(smem + L.sd);
  float2 *terms = reinterpret_cast<float2 *>(smem + L.terms);
  const uint8_t *base = W + (size_t)gtile * nblk * kQ4kRecord;
  const bool arow = r < pg;  // this lane's A row (token r) exists
  // this lane's result tokens 4g + v, the sd row each reads (token 0 when past the group) and
  // where its terms go (a per-lane dummy slot when past the group)
  int tok[NV], tmask[NV];
  float2 *tdst[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int t = 4 * g + v;
    tok[v] = t < pg ? t : 0;
    tmask[v] = t < pg ? -1 : 0;
    tdst[v] = t < pg ? terms + (size_t)(t * 16 + r) * L.tstride
                     : reinterpret_cast<float2 *>(smem + L.dummy) + lane;
  }
  const uint32_t k0F = 0x0F0F0F0Fu;

  struct Rec {
    uint4 h, qa, qb;
  };
  // The nibbles are refilled as soon as the MFMAs have read them, the header after the terms:
  // refilling a slot only after its last use keeps it in the same registers from one pass to
  // the next (a copy of a slot still loading would wait for every load in flight).
  auto load_q = [&](int b, Rec &o) {
    const uint8_t *rec = base + (size_t)b * kQ4kRecord;
    o.qa = *reinterpret_cast<const uint4 *>(rec + kQ4kHdr + 16 * lane);
    o.qb = *reinterpret_cast<const uint4 *>(rec + kQ4kHdr + 1024 + 16 * lane);
  };
  auto load_h = [&](int b, Rec &o) {
    o.h = *reinterpret_cast<const uint4 *>(base + (size_t)b * kQ4kRecord + 16 * r);
  };

  float acc[NV];  // wave 0: (row r, token 4g + v)
#pragma unroll
  for (int v = 0; v < NV; ++v) acc[v] = 0.f;
  for (int wb = 0; wb < nblk; wb += Wrec) {
    const int we = min(nblk, wb + Wrec), nw = we - wb;
    const int per = (nw + KW - 1) / KW;
    const int b0 = min(we, wb + kwave * per), b1 = min(we, b0 + per);

    // Loads are unconditional, re-reading the wave's last record (or the window's, for a wave
    // without records) where the ring runs past it: no branches around loads keeps the
    // compiler's wait counts exact across the record loop.
    const int blast = max(b1, wb + 1) - 1;
    Rec ring[kPF];
#pragma unroll
    for (int u = 0; u < kPF; ++u) {
      load_h(min(b0 + u, blast), ring[u]);
      load_q(min(b0 + u, blast), ring[u]);
      __builtin_amdgcn_sched_barrier(kNoVmemAcross);
    }

    if (!fused) {
      for (int i = threadIdx.x; i < pg * nw * 16; i += blockDim.x) {  // codes, 16 B at a time
        const int t = i / (nw * 16), j = i - t * (nw * 16);
        reinterpret_cast<uint4 *>(codes + (size_t)t * L.cstride)[j] =
            reinterpret_cast<const uint4 *>(qxg + (size_t)(t0 + t) * K + (size_t)wb * 256)[j];
      }
      for (int i = threadIdx.x; i < pg * nw * 4; i += blockDim.x) {  // {S, dx}, two at a time
        const int t = i / (nw * 4), j = i - t * (nw * 4);
        reinterpret_cast<float4 *>(sd + (size_t)t * 8 * Wrec)[j] = reinterpret_cast<const float4 *>(
            sdg + (size_t)(t0 + t) * (K / 32) + (size_t)wb * 8)[j];
      }
    }
    // quantize the window's activation blocks: one thread per (token, block)
    for (int task = threadIdx.x; fused && task < pg * nw * 8; task += blockDim.x) {
      const int t = task / (nw * 8), lb = task - t * (nw * 8);
      const float *xp = X + (size_t)(t0 + t) * K + ((size_t)wb * 8 + lb) * 32;
      float x[32];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float4 v = reinterpret_cast<const float4 *>(xp)[i];
        x[4 * i] = v.x;
        x[4 * i + 1] = v.y;
        x[4 * i + 2] = v.z;
        x[4 * i + 3] = v.w;
      }
      __align__(16) int8_t q[32];
      int sum = 0;
      const float d = q8_quant_block32(x, q, &sum);
      uint4 *dst = reinterpret_cast<uint4 *>(codes + (size_t)t * L.cstride + 32 * lb);
      dst[0] = *reinterpret_cast<const uint4 *>(q);
      dst[1] = *reinterpret_cast<const uint4 *>(q + 16);
      sd[t * 8 * Wrec + lb] = make_float2((float)sum, d);
    }
    __syncthreads();

    // Rows of A past the group's tokens repeat token 0: their results are never read.
    const int8_t *arow_p = codes + (size_t)(arow ? r : 0) * L.cstride + 8 * g;
    const bool chain = kwave == 0;  // wave-uniform
    {
      // Every pass works kPF slots; slots past the wave's last record re-run that record (the
      // ring loads were clamped): their terms are rewritten with the same values and the chain
      // skips them. No branches in a pass, and each refill pinned after its slot's last use,
      // lets the compiler count the loads in flight exactly across the loop back-edge.
      for (int bb = b0; bb < b1; bb += kPF) {
#pragma unroll
        for (int u = 0; u < kPF; ++u) {
          const bool live = bb + u < b1;
          const int b = min(bb + u, blast);
          const int lb = b - wb;
          const uint32_t q[8] = {ring[u].qa.x, ring[u].qa.y, ring[u].qa.z, ring[u].qa.w,
                                 ring[u].qb.x, ring[u].qb.y, ring[u].qb.z, ring[u].qb.w};
          i32x4 D[8];
#pragma unroll
          for (int s = 0; s < 8; ++s) {
            // chunk s/2 = words q[2 (s/2)], q[2 (s/2) + 1]: low nibbles for even s, high for odd
            const uint32_t w0 = q[2 * (s >> 1)], w1 = q[2 * (s >> 1) + 1];
            const uint32_t n0 = (s & 1) ? (w0 >> 4) & k0F : w0 & k0F;
            const uint32_t n1 = (s & 1) ? (w1 >> 4) & k0F : w1 & k0F;
            const long B = (long)(((unsigned long)n1 << 32) | n0);
            const long A = *reinterpret_cast<const long *>(arow_p + 256 * lb + 32 * s);
            D[s] = __builtin_amdgcn_mfma_i32_16x16x32_i8(A, B, i32x4{0, 0, 0, 0}, 0, 0, 0);
          }
          const int bnext = min(bb + u + kPF, blast);
          load_q(bnext, ring[u]);  // operands consumed: refill
          __builtin_amdgcn_sched_barrier(kNoVmemAcross);
          const uint4 h = ring[u].h;
          const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)(h.x & 0xffffu));
          const float dmin = (float)__builtin_bit_cast(_Float16, (uint16_t)(h.x >> 16));
#pragma unroll
          for (int s = 0; s < 8; ++s) {
            uint32_t sc, m;
            scale_min_s(h.y, h.z, h.w, s, sc, m);
            const float ws = __fmul_rn(d, (float)sc), wm = __fmul_rn(dmin, (float)m);
#pragma unroll
            for (int v = 0; v < NV; ++v) {
              // lanes whose token 4g + v is past the group compute on token 0 and discard
              const float2 e = sd[tok[v] * 8 * Wrec + 8 * lb + s];  // {f32(S), dx}
              const float T1 = __fmul_rn(__fmul_rn((float)D[s][v], ws), e.y);
              const float T2 = __fmul_rn(__fmul_rn(e.x, wm), e.y);
              if (chain) {
                const float a = __fsub_rn(__fadd_rn(acc[v], T1), T2);
                acc[v] = live ? a : acc[v];
              } else {
                tdst[v][(8 * lb + s) & tmask[v]] = make_float2(T1, T2);
              }
            }
          }
          load_h(bnext, ring[u]);
          __builtin_amdgcn_sched_barrier(kNoVmemAcross);
        }
      }
    }
    __syncthreads();
    if (KW > 1 && kwave == 0) {
      // the other waves' records of this window, in order: local records per .. nw - 1. Eight
      // pairs of sub-blocks are read before any is added, so the LDS latency is paid once per
      // eight steps of the chain, not once per step (3584 x 18944 at one token: 31.6 -> 25.1 us).
      auto step = [&](int v, const float4 p) {
        acc[v] = __fadd_rn(acc[v], p.x);
        acc[v] = __fsub_rn(acc[v], p.y);
        acc[v] = __fadd_rn(acc[v], p.z);
        acc[v] = __fsub_rn(acc[v], p.w);
      };
      int k = 4 * min(per, nw);
      const int kend = 4 * nw;
      for (; k + 8 <= kend; k += 8) {
        float4 p[8][NV];
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
          for (int v = 0; v < NV; ++v) p[j][v] = reinterpret_cast<const float4 *>(tdst[v])[k + j];
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
          for (int v = 0; v < NV; ++v) step(v, p[j][v]);
      }
      for (; k < kend; ++k)
#pragma unroll
        for (int v = 0; v < NV; ++v) step(v, reinterpret_cast<const float4 *>(tdst[v])[k]);
    }
    __syncthreads();
  }
  if (kwave == 0 && tile < ntiles) {
    const int row = tile * 16 + r;
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const int t = 4 * g + v;
      if (t < pg && row < N) Y[(size_t)(t0 + t) * N + row] = acc[v];
    }
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
  if (int rc = check_weight("fhip_q4k_matmul_int8_f32", dPacked, kWeightQ4K, out, in)) return rc;
  untag_range(dY, (size_t)P * out * 4);
  const int nblk = in / 256;
  const bool fused = P <= kFusedTokens;
  int8_t *qx = nullptr;
  float2 *sdg = nullptr;
  if (!fused) {
    const size_t qbytes = ((size_t)P * in + 255) & ~(size_t)255;
    unsigned char *ws = (unsigned char *)workspace(qbytes + (size_t)P * (in / 32) * sizeof(float2));
    if (!ws) return FHIP_ENOMEM;
    if (int rc = check_disjoint("fhip_q4k_matmul_int8_f32", dX, (size_t)P * in * 4, ws,
                                qbytes + (size_t)P * (in / 32) * sizeof(float2)))
      return rc;
    qx = reinterpret_cast<int8_t *>(ws);
    sdg = reinterpret_cast<float2 *>(ws + qbytes);
    const long long nq = (long long)P * (in / 32);
    i8r_prep_kernel<<<(unsigned)((nq + 255) / 256), 256, 0, stream()>>>(dX, P, in, qx, sdg);
    FHIP_CHECK_LAUNCH("i8r_prep_kernel");
  }
  // Shape: a 16-row tile per workgroup whose records are split over up to 8 waves until the grid
  // has ~16 waves per CU (~8 for one token), each wave keeping >= 2 records; a window of records
  // whose LDS fits the device. (One token with ~16 waves per CU put 4 waves on each 18944 x 3584
  // tile: 26.2 us against 21.4 with 2; the 3584 x 18944 down projection keeps 8 either way.
  // Eight tokens on 18944 x 3584 want 4: 91 us, 130 with 2.)
  const int ntiles = q4k_tiles(out);
  const int groups = ceil_div(P, kTokGroup);
  const int pg = P < kTokGroup ? P : kTokGroup;
  int KW = tuning().i8r_kw, TW = 1;
  if (KW <= 0) {
    KW = 1;
    const long long fill = (P == 1 ? 8LL : 16LL) * cu_count();
    while (KW < 8 && (long long)ntiles * groups * KW < fill && nblk >= 2 * KW)
      KW *= 2;
  }
  if (KW > 8) KW = 8;
  // Wide matrices: one wave per tile and eight tiles per workgroup. The staged window (the
  // tokens' codes) is quantized or copied once for the eight tiles and, with KW = 1, no terms are
  // parked in LDS (18944 x 3584 at 1 / 4 / 8 / 16 tokens 18.8 / 41.0 / 43.3 / 45.4 us, against
  // 21.3 / 76.1 / 91.1 / 144 with a tile of 2-4 waves per workgroup, whose parked terms held up to
  // 155 KB of LDS, one workgroup per CU; 4 tiles per workgroup 20.7 / 44.7 / 44.7 / 48.1).
  if (tuning().i8r_tw > 0) {
    TW = tuning().i8r_tw;
    KW = 1;
  } else if (tuning().i8r_kw <= 0 && ntiles >= 4 * cu_count()) {
    TW = 8;
    KW = 1;
  }
  if (TW > 8) TW = 8;  // 512 threads per workgroup at most
  const size_t budget = (size_t)lds_limit();
  int wmax = nblk;
  while (wmax > 1 && i8r_lds(pg, wmax, KW).total > budget) --wmax;
  const int nwin = ceil_div(nblk, wmax);
  const int Wrec = ceil_div(nblk, nwin);
  const size_t lds = i8r_lds(pg, Wrec, KW).total;
  if (lds > budget)
    return fail(FHIP_EINVAL, "fhip_q4k_matmul_int8_f32: %zu B of LDS exceeds the device limit",
                lds);
  dim3 grid(ceil_div(ntiles, TW), groups);
  // result tokens per lane: lane group g holds tokens 4g .. 4g + 3 of the group
  auto launch = [&](auto kern) {
    kern<<<grid, 64 * KW * TW, lds, stream()>>>(reinterpret_cast<const uint8_t *>(dPacked), dX, qx,
                                                sdg, dY, out, in, nblk, P, Wrec, KW, TW,
                                                fused ? 1 : 0);
  };
  if (pg == 1)
    launch(q4k_i8route_kernel<1>);
  else if (pg == 2)
    launch(q4k_i8route_kernel<2>);
  else
    launch(q4k_i8route_kernel<4>);
  FHIP_CHECK_LAUNCH("q4k_i8route_kernel");
  return FHIP_OK;
}
