// kernels.hpp — device helpers and launchers shared by the Q4_K / Q8_0 matmul kernels.
#pragma once

#include "common.hpp"
#include "tiled.hpp"

namespace fhip {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// The order in which a lane's 8 K-elements sit in its MFMA operand: element j holds the value
// at K offset kPerm[j] within the lane's 8-run. It is the order the nibble unpack produces
// (bytes 0,2 then 1,3 of each dword); the activation operands are built in the same order, so
// every product pairs a weight with its own activation.
__host__ __device__ constexpr int perm8(int j) { return (j & 4) | ((j & 1) << 1) | ((j >> 1) & 1); }

// A checked Q4_K matmul of P tokens (the route of fhip_q4k_matmul_f32) and the scratch bytes
// (workspace()) it needs.
int q4k_matmul_run(const void *W, const float *X, float *Y, int N, int K, int P);
size_t q4k_matmul_ws_bytes(int N, int K, int P);

int q4k_gemv(const void *W, const float *X, float *Y, int N, int K, int M);
// Scratch bytes (workspace()) of one q4k_gemv call.
size_t q4k_gemv_ws_bytes(int N, int K, int M);
// Matrices sharing one activation, run as one grid (the group dispatch of
// internal/model/metal_q4k_on.go:139-190). Members are concatenated by 16-row tiles.
constexpr int kMaxGroup = 8;
struct GemvGroup {
  const uint8_t *W[kMaxGroup];
  float *Y[kMaxGroup];
  int N[kMaxGroup];
  int tile0[kMaxGroup + 1];  // first tile of each member; tile0[count] = total tiles
  int count;
};
int q4k_gemv_group(const GemvGroup &g, const float *X, int K, int M);
// 5..16 tokens (3..16 for K >= 24576) on the 32x32x16 MFMA with exact weight operands (q4k_gemv16.hip).
int q4k_gemv16(const void *W, const float *X, float *Y, int N, int K, int M);
// Scratch bytes of a q4k_gemv16 (fmt 0) / q6k_gemv16 (fmt 1) / q4k_gemv32 call.
size_t gemv16_ws_bytes(int fmt, int N, int K, int M);
// 17..32 tokens on the same kernel with one f16 operand row per token (q4k_gemv16.hip).
int q4k_gemv32(const void *W, const float *X, float *Y, int N, int K, int M);
int q6k_gemv32(const void *W, const float *X, float *Y, int N, int K, int M);
// The same for a tiled Q6_K weight.
int q6k_gemv16(const void *W, const float *X, float *Y, int N, int K, int M);
// Fused decode MLP pieces (1..4 tokens): the workspace a small-M call over `ntiles` tiles
// needs, the SwiGLU stage over {gate, up}, and the Q6_K GEMV.
size_t gemv_i8_ws_bytes(int ntiles, int K, int M, bool swiglu);
// The one-token GEMV's workgroup shape over `ntiles` 16-row tiles of reduction dim K.
void q4k_gemv1_shape(int ntiles, int K, int &TW, int &KW);
int q4k_gemv_swiglu(const void *gate, const void *up, const float *X, float *inter, int I, int K,
                    int M, void *ws);
int q6k_gemv(const void *W, const float *X, float *Y, int N, int K, int M);
// Scratch bytes of one q6k_gemv call.
size_t q6k_gemv_ws_bytes(int N, int K, int M);
int q4k_gemm32(const void *W, const float *X, float *Y, int N, int K, int M);
// Scratch bytes of a q4k_gemm32 (fmt 0) / q6k_gemm32 (fmt 1) call.
size_t gemm32_ws_bytes(int fmt, int N, int K, int M);
// The same GEMM over a tiled Q6_K weight (prefill of the q4_k_m Q6_K tensors).
int q6k_gemm32(const void *W, const float *X, float *Y, int N, int K, int M);
int q8_0_gemv(const void *W, const float *X, float *Y, int N, int K, int M);

// __builtin_amdgcn_sched_barrier mask: every instruction class except vector-memory ones may be
// scheduled across (ALU 0x1, VALU 0x2, SALU 0x4, MFMA 0x8, LDS 0x80). Placed after a ring
// refill, it keeps the refill loads where the source puts them.
constexpr int kNoVmemAcross = 0x0;

// gfx9 VOP3 instructions cannot encode literal constants, so (q & mask) | magic with literal
// operands compiles to two instructions. Holding the constants in registers (opaque to constant
// folding) lets each nibble pair become one v_and_or_b32.
__device__ __forceinline__ uint32_t in_reg(uint32_t x) {
  asm volatile("" : "+v"(x));
  return x;
}

// Loads of weight records, which every call reads exactly once: non-temporal, so the weight
// stream does not evict what is reused from the L2 (the activations). Used by the 1..4-token
// Q4_K, the Q6_K and the Q8_0 GEMVs; the 5..16-token kernel keeps cached loads (measured 8%
// slower with these on a 25600 x 5120 matrix at 16 tokens).
__device__ __forceinline__ uint4 ld_stream(const void *p) {
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 ld_stream2(const void *p) {
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  const u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const u32x2 *>(p));
  return make_uint2(v.x, v.y);
}
__device__ __forceinline__ uint32_t ld_stream32(const void *p) {
  return __builtin_nontemporal_load(reinterpret_cast<const uint32_t *>(p));
}
__device__ __forceinline__ uint16_t ld_stream16(const void *p) {
  return __builtin_nontemporal_load(reinterpret_cast<const uint16_t *>(p));
}

// v + p[0] + p[stride] + ... + p[(N - 1) stride], in that order, every load issued first.
template <int N, typename T>
__device__ __forceinline__ T add_n(T v, const T *__restrict__ p, size_t stride) {
  T q[N];
#pragma unroll
  for (int j = 0; j < N; ++j) q[j] = p[(size_t)j * stride];
#pragma unroll
  for (int j = 0; j < N; ++j) v = v + q[j];
  return v;
}

// Ordered sum of K-range partial results: v (range 0) += p1[k * stride] for k = 0 .. count-1
// (ranges 1 .. count), in that order. The loads go out eight at a time, the last group in a
// straight-line block of exactly the remaining count (count is uniform over the launch, so the
// choice is a scalar branch): a loop of run-time length would wait for each load before issuing
// the next, and clamped indices re-issue the last range's load (6 repeats for two ranges).
template <typename T>
__device__ __forceinline__ T add_ranges(T v, const T *__restrict__ p1, size_t stride, int count) {
  int k = 0;
  for (; k + 8 <= count; k += 8) v = add_n<8>(v, p1 + (size_t)k * stride, stride);
  const T *p = p1 + (size_t)k * stride;
  switch (count - k) {
    case 1: return add_n<1>(v, p, stride);
    case 2: return add_n<2>(v, p, stride);
    case 3: return add_n<3>(v, p, stride);
    case 4: return add_n<4>(v, p, stride);
    case 5: return add_n<5>(v, p, stride);
    case 6: return add_n<6>(v, p, stride);
    case 7: return add_n<7>(v, p, stride);
    default: return v;
  }
}

// Two-digit int8 activations: the digits of four values x at scale 2^sh (|x| 2^sh <= 32512): y = x 2^sh + (1.5 2^23 + 128)
// lies in [2^23, 2^24), where floats are the integers, so the add rounds x 2^sh half to even
// exactly as rint and the low 23 bits of y hold 2^22 + T + 128. Byte 1 of y is then
// q1 = (T + 128) >> 8 and byte 0 is the low byte of T + 128, i.e. q2 ^ 0x80. a gathers the
// four q1, c the four q2 (value i in byte i).
__device__ __forceinline__ void digits4(float x0, float x1, float x2, float x3, int sh,
                                        uint32_t &a, uint32_t &c) {
  constexpr float kMagic = 12583040.f;  // 1.5 * 2^23 + 128
  const uint32_t y0 = __float_as_uint(ldexpf(x0, sh) + kMagic);
  const uint32_t y1 = __float_as_uint(ldexpf(x1, sh) + kMagic);
  const uint32_t y2 = __float_as_uint(ldexpf(x2, sh) + kMagic);
  const uint32_t y3 = __float_as_uint(ldexpf(x3, sh) + kMagic);
  a = __builtin_amdgcn_perm(y1, y0, 0x0C0C0501u) | __builtin_amdgcn_perm(y3, y2, 0x05010C0Cu);
  c = (__builtin_amdgcn_perm(y1, y0, 0x0C0C0400u) | __builtin_amdgcn_perm(y3, y2, 0x04000C0Cu)) ^
      0x80808080u;
}

// digits4 with the scale given as the float s = 2^sh, for sh in [-126, 127] (s normal): one fma
// per value. The product x s is exact in the fma, which then rounds x s + (1.5 2^23 + 128) once,
// as the add after ldexpf(x, sh) does (where x 2^sh would be subnormal, |x 2^sh| < 2^-126 and
// both round to the constant itself), so the digits are the same bits.
__device__ __forceinline__ void digits4s(float x0, float x1, float x2, float x3, float s,
                                         uint32_t &a, uint32_t &c) {
  constexpr float kMagic = 12583040.f;  // 1.5 * 2^23 + 128
  const uint32_t y0 = __float_as_uint(__builtin_fmaf(x0, s, kMagic));
  const uint32_t y1 = __float_as_uint(__builtin_fmaf(x1, s, kMagic));
  const uint32_t y2 = __float_as_uint(__builtin_fmaf(x2, s, kMagic));
  const uint32_t y3 = __float_as_uint(__builtin_fmaf(x3, s, kMagic));
  a = __builtin_amdgcn_perm(y1, y0, 0x0C0C0501u) | __builtin_amdgcn_perm(y3, y2, 0x05010C0Cu);
  c = (__builtin_amdgcn_perm(y1, y0, 0x0C0C0400u) | __builtin_amdgcn_perm(y3, y2, 0x04000C0Cu)) ^
      0x80808080u;
}

// Three-digit int8 activations: the digits of four values x at scale 2^sh with |x 2^sh| <=
// 63 * 2^16. y = x 2^sh + (1.5 2^23 + 32896) lies in [2^23, 2^24), where floats are the
// integers, so the add rounds x 2^sh half to even exactly as rint, giving T, and the low 23 bits
// of y hold 2^22 + T + 32896 = 2^22 + 65536 q1 + 256 (q2 + 128) + (q3 + 128) with q2, q3 in
// [-128, 127] and q1 in [-63, 63]. Byte 0 of y is q3 ^ 0x80, byte 1 q2 ^ 0x80 and byte 2 q1 + 64
// (in [1, 127]); q1 + q2 / 256 + q3 / 65536 = T / 65536 exactly. a gathers the four q1, b the
// four q2, c the four q3 (value i in byte i), each as a two's complement byte.
__device__ __forceinline__ void digits3_pack(uint32_t y0, uint32_t y1, uint32_t y2, uint32_t y3,
                                             uint32_t &a, uint32_t &b, uint32_t &c) {
  // Bytes 0 and 1 of the four words, transposed in two steps: t01 = {y0.0, y1.0, y0.1, y1.1},
  // t23 = {y2.0, y3.0, y2.1, y3.1}.
  const uint32_t t01 = __builtin_amdgcn_perm(y1, y0, 0x05010400u);
  const uint32_t t23 = __builtin_amdgcn_perm(y3, y2, 0x05010400u);
  c = __builtin_amdgcn_perm(t23, t01, 0x05040100u) ^ 0x80808080u;
  b = __builtin_amdgcn_perm(t23, t01, 0x07060302u) ^ 0x80808080u;
  // q1 + 64 -> q1: flipping bit 6 gives q1 for q1 >= 0 and q1 + 128 for q1 < 0 (bit 6 then set),
  // and copying bit 6 into bit 7 turns the latter into the byte q1 + 256.
  const uint32_t w =
      (__builtin_amdgcn_perm(y1, y0, 0x0C0C0602u) | __builtin_amdgcn_perm(y3, y2, 0x06020C0Cu)) ^
      0x40404040u;
  a = w | ((w << 1) & 0x80808080u);
}
constexpr float kMagic3 = 12615808.f;  // 1.5 * 2^23 + 32896

__device__ __forceinline__ void digits3(float x0, float x1, float x2, float x3, int sh,
                                        uint32_t &a, uint32_t &b, uint32_t &c) {
  digits3_pack(__float_as_uint(ldexpf(x0, sh) + kMagic3), __float_as_uint(ldexpf(x1, sh) + kMagic3),
               __float_as_uint(ldexpf(x2, sh) + kMagic3), __float_as_uint(ldexpf(x3, sh) + kMagic3),
               a, b, c);
}

// digits3 with the scale given as the float s = 2^sh (s normal): one fma per value, the same
// bits as digits3 (the fma rounds the exact product plus the constant once, as the add after
// ldexpf does).
__device__ __forceinline__ void digits3s(float x0, float x1, float x2, float x3, float s,
                                         uint32_t &a, uint32_t &b, uint32_t &c) {
  digits3_pack(__float_as_uint(__builtin_fmaf(x0, s, kMagic3)),
               __float_as_uint(__builtin_fmaf(x1, s, kMagic3)),
               __float_as_uint(__builtin_fmaf(x2, s, kMagic3)),
               __float_as_uint(__builtin_fmaf(x3, s, kMagic3)), a, b, c);
}

// Largest magnitude of four floats as a bit pattern: magnitudes order like their patterns, and a
// NaN or an infinity gives a pattern >= 0x7F800000, so the integer maximum needs no NaN quieting
// (fmaxf's) and the maximum of a block is order-free.
__device__ __forceinline__ uint32_t absmax4_bits(float x0, float x1, float x2, float x3) {
  const uint32_t m = 0x7FFFFFFFu;
  return max(max(__float_as_uint(x0) & m, __float_as_uint(x1) & m),
             max(__float_as_uint(x2) & m, __float_as_uint(x3) & m));
}

// Workgroup shape of the small-M GEMV kernels (TW tiles x KW waves; see q4k_gemv.hip).
void gemv_shape(int ntiles, int nblk, int max_waves, size_t lds_fixed, size_t lds_per_wave,
                int &TW, int &KW);

}  // namespace fhip
