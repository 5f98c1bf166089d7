// gemv_common.hpp — pieces shared by the small-M Q4_K and Q8_0 matmul kernels: the activation
// operand layout (hi/lo f16 split), its staging into LDS or a global buffer, and the
// workgroup-level split-K reduction.
#pragma once

#include "kernels.hpp"

namespace fhip {

// Activation operands for 32-wide K slices. For slice s, lane group g (0..3) and operand row
// rho = 2t + h (token t, h = 0 hi / 1 lo):
//   A[(s * 4 + g) * 2M + rho] = 8 f16 values split_h(X[t][32 s + 8 g + perm8(j)]), j = 0..7
//   S[(s >> 3) * M * 8 + t * 8 + (s & 7)] = sum over the slice of (hi + lo)   (f32)
// split_0(x) = f16(x), split_1(x) = f16(x - f16(x)): two f16 MFMA rows carry x to ~22 bits.
// The same layout is used in LDS (staged by the matmul workgroup itself) and in global memory
// (written by gemv_xprep_kernel when the operands do not fit in LDS).

// One (slice, token) task: 32 activations -> 8 operand rows + one sum.
template <int M>
__device__ __forceinline__ void split_slice(const float *__restrict__ x, bool valid, int sl,
                                            int t, uint4 *__restrict__ A, float *__restrict__ S) {
  constexpr int R2 = 2 * M;
  float sum = 0.f;
  if (valid) {
    float4 v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = *reinterpret_cast<const float4 *>(x + 4 * i);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const float e[8] = {v[2 * g].x, v[2 * g].y, v[2 * g].z, v[2 * g].w,
                          v[2 * g + 1].x, v[2 * g + 1].y, v[2 * g + 1].z, v[2 * g + 1].w};
      f16x8 hi, lo;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float xv = e[perm8(j)];
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
  S[(sl >> 3) * M * 8 + t * 8 + (sl & 7)] = sum;
}

// Stage slices [s0, s0 + ns) of M tokens (global slices >= ns_valid are zero) into A/S, whose
// slice 0 is global slice s0. `lane`/`nlanes` pick the threads that share the work: the whole
// workgroup (then __syncthreads before use) or one wave (then only a wave fence).
template <int M>
__device__ __forceinline__ void stage_x(const float *__restrict__ X, int K, int s0, int ns,
                                        int ns_valid, uint4 *__restrict__ A,
                                        float *__restrict__ S, int lane, int nlanes) {
  for (int task = lane; task < ns * M; task += nlanes) {
    const int t = task / ns, sl = task - t * ns;
    const bool valid = s0 + sl < ns_valid;
    split_slice<M>(X + (size_t)t * K + 32 * (valid ? s0 + sl : 0), valid, sl, t, A, S);
  }
}

// Bytes of the operand layout for `ns` slices (S padded to whole groups of 8 slices).
__host__ __device__ inline size_t xop_a_bytes(int M, int ns) { return (size_t)ns * 4 * 2 * M * 16; }
__host__ __device__ inline size_t xop_bytes(int M, int ns) {
  return xop_a_bytes(M, ns) + (size_t)((ns + 7) / 8) * M * 8 * 4;
}

// Launch the standalone operand writer into global memory (layout above, S after A).
int launch_gemv_xprep(const float *X, int M, int K, int ns, void *xop);

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
