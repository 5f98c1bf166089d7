// gemv_common.hpp — pieces of the small-M Q8_0 matmul: the activation operand layout (a
// power-of-two block scale and a hi/lo f16 split), its staging into LDS or a global buffer, and
// the workgroup-level split-K reduction.
#pragma once

#include "kernels.hpp"

namespace fhip {

// Activation operands for 32-wide K slices. For slice s, lane group g (0..3) and operand row
// rho = 2t + h (token t, h = 0 hi / 1 lo):
//   A[(s * 4 + g) * 2M + rho] = 8 f16 values split_h(X[t][32 s + 8 g + perm8(j)] / e), j = 0..7
//   E[(s >> 3) * M * 8 + t * 8 + (s & 7)] = {sum over the slice of (hi + lo), e}   (f32 pair)
// with e = 2^k chosen per (slice, token) so that the slice's largest magnitude lands in
// [2^13, 2^14): any finite f32 activation block, however large or small, becomes f16 values
// without overflow and with 11-bit relative precision down to 2^-28 of the block maximum, and
// the block's product is scaled back by e exactly (a power of two). split_0(v) = f16(v),
// split_1(v) = f16(v - f16(v)): two f16 MFMA rows carry v to ~22 bits. A block holding a NaN or
// an infinity gets e = NaN, which reaches every output that uses it.
// The same layout is used in LDS (staged by the matmul workgroup itself) and in global memory
// (written by q8_xprep_kernel when the operands do not fit in LDS).

// One (slice, token) task: 32 activations -> 8 operand rows + {sum, e}.
template <int M>
__device__ __forceinline__ void split_slice(const float *__restrict__ x, bool valid, int sl,
                                            int t, uint4 *__restrict__ A,
                                            float2 *__restrict__ E) {
  constexpr int R2 = 2 * M;
  float sum = 0.f, e = 0.f;
  if (valid) {
    float4 v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = *reinterpret_cast<const float4 *>(x + 4 * i);
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i)
      amax = fmaxf(fmaxf(fmaxf(amax, fabsf(v[i].x)), fabsf(v[i].y)),
                   fmaxf(fabsf(v[i].z), fabsf(v[i].w)));
    // amax = f 2^E with f in [0.5, 1): k = E - 14 puts amax / 2^k in [2^13, 2^14).
    int E2 = 0;
    (void)frexpf(amax, &E2);
    const int k = E2 - 14;
    const bool finite = amax <= 3.4028235e38f;  // false for Inf and NaN
    e = amax > 0.f ? (finite ? ldexpf(1.f, k) : __builtin_nanf("")) : 0.f;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const float el[8] = {v[2 * g].x, v[2 * g].y, v[2 * g].z, v[2 * g].w,
                           v[2 * g + 1].x, v[2 * g + 1].y, v[2 * g + 1].z, v[2 * g + 1].w};
      f16x8 hi, lo;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float xv = finite ? ldexpf(el[perm8(j)], -k) : 0.f;
        const _Float16 h = (_Float16)xv;
        const _Float16 l = (_Float16)(xv - (float)h);
        hi[j] = h;
        lo[j] = l;
        sum += (float)h + (float)l;
      }
      A[(sl * 4 + g) * R2 + 2 * t] = __builtin_bit_cast(uint4, hi);
      A[(sl * 4 + g) * R2 + 2 * t + 1] = __builtin_bit_cast(uint4, lo);
    }
  } else {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      A[(sl * 4 + g) * R2 + 2 * t] = make_uint4(0, 0, 0, 0);
      A[(sl * 4 + g) * R2 + 2 * t + 1] = make_uint4(0, 0, 0, 0);
    }
  }
  E[(sl >> 3) * M * 8 + t * 8 + (sl & 7)] = make_float2(sum, e);
}

// Stage slices [s0, s0 + ns) of M tokens (global slices >= ns_valid are zero) into A/E, whose
// slice 0 is global slice s0. `lane`/`nlanes` pick the threads that share the work: the whole
// workgroup (then __syncthreads before use) or one wave (then only a wave fence).
template <int M>
__device__ __forceinline__ void stage_x(const float *__restrict__ X, int K, int s0, int ns,
                                        int ns_valid, uint4 *__restrict__ A,
                                        float2 *__restrict__ E, int lane, int nlanes) {
  for (int task = lane; task < ns * M; task += nlanes) {
    const int t = task / ns, sl = task - t * ns;
    const bool valid = s0 + sl < ns_valid;
    split_slice<M>(X + (size_t)t * K + 32 * (valid ? s0 + sl : 0), valid, sl, t, A, E);
  }
}

// Bytes of the operand layout for `ns` slices (E padded to whole groups of 8 slices).
__host__ __device__ inline size_t xop_a_bytes(int M, int ns) { return (size_t)ns * 4 * 2 * M * 16; }
__host__ __device__ inline size_t xop_bytes(int M, int ns) {
  return xop_a_bytes(M, ns) + (size_t)((ns + 7) / 8) * M * 8 * 8;
}

// Workgroup split-K: the KW waves of a 16-row tile each hold a partial over their own K part.
// Partials go through LDS and part 0 sums them in part order, so results are deterministic.
// red: LDS scratch of TW * KW * 64 * VALS floats; vals: the wave's VALS accumulators per lane.
template <int VALS>
__device__ __forceinline__ void wg_reduce(float *__restrict__ red, int tile, int part, int KW,
                                          int lane, float (&vals)[VALS]) {
  if (KW > 1) {
#pragma unroll
    for (int v = 0; v < VALS; ++v) red[((tile * KW + part) * VALS + v) * 64 + lane] = vals[v];
  }
  __syncthreads();
  if (KW > 1 && part == 0) {
    for (int q = 1; q < KW; ++q)
#pragma unroll
      for (int v = 0; v < VALS; ++v) vals[v] += red[((tile * KW + q) * VALS + v) * 64 + lane];
  }
}

}  // namespace fhip
