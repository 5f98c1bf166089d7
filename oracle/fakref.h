/* fakref.h — the ORACLE: a plain-C restatement of fak's Go CPU path for the GGUF Q4_K / Q8_0
 * dequantize-and-multiply. TEST INFRASTRUCTURE ONLY: it is the parity reference for the HIP
 * backend and the CPU baseline timed beside it. Nothing in the product (fak_amd/, include/)
 * links, loads or calls it.
 *
 * Every function names the Go source it follows (paths relative to the fak repository). The
 * reference is Go and no Go toolchain exists here, so this file restates it operation for
 * operation: same operand order, same 4-accumulator reduction, no fused multiply-add (built
 * with -ffp-contract=off, matching amd64 Go codegen, internal/model/quant.go:80-86).
 *
 * Pinning status (what checks each function against something other than itself):
 *   fr_f16_bits_to_f32_bits   exhaustive 2^16 sweep vs numpy IEEE half->single (finite), NaN
 *                             payload rule by hand                         -> pinned
 *   fr_get_scale_min_k4       closed form + bijective packer round trip over all fields,
 *                             hand cases                                   -> pinned
 *   fr_q4k_dequant_superblock hand-derived blocks (closed form), independent numpy dequant
 *                             of random blocks (bit-exact)                 -> pinned
 *   fr_q4k_matrows_range      integer-exact fixtures (exact closed form), order-revealing
 *                             adversarial vectors with hand-computed sums, f64 brute force
 *                             tolerance                                    -> pinned
 *   fr_q4k_gemm_range         == fr_q4k_matrows_range per token bitwise (the reference's own
 *                             invariant, prefill_q4k_test.go:75-110) + the above -> pinned
 *   fr_q6k_dequant_superblock hand golden (quant_kquant_test.go:113-129: d=2, scales 1, codes 0
 *                             -> -64); an index-revealing block whose every weight has its own
 *                             (ql, qh, scale) combination, checked against an independent
 *                             vectorised numpy decode of the GGUF Q6_K layout        -> pinned
 *   fr_q6k_matrows_range      the reference's lcgBytes fixture (quant_kquant_test.go:51-88,
 *                             d = 1, x = (7i % 23) - 11) = exact integer dot; order-revealing
 *                             cancellation; f64 brute force                           -> pinned
 *   fr_q8_0_*                 hand golden (quant_kquant_test.go:154-167), integer-exact and
 *                             order-revealing fixtures                     -> pinned
 *   fr_q8round                vs round-half-away-from-zero over a dense sweep -> pinned
 *   fr_quantize_vec_q8, fr_qdot8, fr_qgemm8cell
 *                             closed forms on integer-exact inputs; order-revealing cases
 *                                                                          -> pinned
 *   fr_q4k_reduce_row         vs an independent vectorised numpy integer reduction (exact)
 *                                                                          -> pinned
 *   fr_q4k_combine_row, fr_q4k_matrows_int8
 *                             closed form on integer-exact inputs (d=1, dmin=0, amax=127 ->
 *                             dx=1, the sum is an exact integer); order-revealing cases whose
 *                             sequential result differs from a reassociated one; bounded
 *                             distance from fr_q4k_matrows_range (activation quantization)
 *                                                                          -> pinned
 *   fr_silu, fr_swiglu        special values (signed zeros, infinities, NaN, f32 overflow of
 *                             e^-z) and an independent 50-digit decimal evaluation of
 *                             e^-z rounded f64 -> f32, then 1 + t and z / s in IEEE f32 (numpy),
 *                             bit-exact over a dense sweep. glibc's exp stands in for Go's
 *                             math.Exp (both within 1 ulp in f64); the f32 rounding absorbs the
 *                             difference except where e^-z lies within 1 f64 ulp of an f32
 *                             rounding boundary                            -> pinned
 * The exact bits the Go compiler would produce for the same loops are not available (no Go
 * toolchain); equality is argued from identical operation order with no contraction.
 */
#ifndef FAK_ORACLE_FAKREF_H
#define FAK_ORACLE_FAKREF_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* internal/model/quantbits.go:15-36 */
uint32_t fr_f16_bits_to_f32_bits(uint16_t h);
/* internal/model/quantbits.go:42-47 */
void fr_get_scale_min_k4(int j, const uint8_t *q, uint8_t *scale, uint8_t *min);

/* internal/model/quant_q4k.go:90-111 (== internal/ggufload/gguf_dequant.go:709-731) */
void fr_q4k_dequant_superblock(float *dst, const uint8_t *blk);
/* dequantize `nblk` consecutive super-blocks (a row) into dst[nblk*256] */
void fr_q4k_dequant_row(float *dst, const uint8_t *raw, int nblk);
/* internal/model/quant_q4k.go:145-165 — y[lo:hi] for weight raw [out][in/256][144] */
void fr_q4k_matrows_range(const uint8_t *raw, int out, int in, const float *x, float *y,
                          int lo, int hi);
/* internal/model/quant_q4k.go:378-405 — Y[t*out+o] for o in [lo,hi), t in [0,P) */
void fr_q4k_gemm_range(const uint8_t *raw, int out, int in, const float *X, int P, float *Y,
                       int lo, int hi);

/* internal/model/quant_iquant.go:14-19 */
void fr_q8_0_dequant_block(float *dst, const uint8_t *blk);
/* internal/model/quant_kquant.go:139-163 */
void fr_q6k_dequant_superblock(float *dst, const uint8_t *blk);
/* internal/model/quant_kquant.go:210-232 with kind Q6_K (blockWeights 256, blockBytes 210) */
void fr_q6k_matrows_range(const uint8_t *raw, int out, int in, const float *x, float *y, int lo,
                          int hi);
/* internal/model/quant_kquant.go:210-232 with kind Q8_0 (blockWeights 32, blockBytes 34) */
void fr_q8_0_matrows_range(const uint8_t *raw, int out, int in, const float *x, float *y,
                           int lo, int hi);

/* The HAL Q8 lane (int8 codes + f32 per-block scales; the activation is quantized).
 * internal/compute/cpuref.go:486-501 (== internal/model/quant.go:89-104) */
int8_t fr_q8round(float x);
/* internal/model/forward.go:452 */
float fr_silu(float z);
/* g[i] = silu(g[i]) * u[i] (denseSwiGLU, internal/model/moe.go:111-136) */
void fr_swiglu(float *g, const float *u, int n);
/* internal/compute/cpuref.go:505-527 (== internal/model/quant_quantize.go:16-43) */
void fr_quantize_vec_q8(const float *x, int n, int block, int8_t *q, float *d);
/* internal/compute/cpuref.go:531-549 */
float fr_qdot8(const int8_t *qw, const float *dw, const int8_t *qx, const float *dx, int n,
               int block);
/* internal/compute/cpuref.go:553-577 */
float fr_qgemm8cell(const int8_t *qw, const float *dw, const int8_t *qx, const float *dx,
                    int nblk, int block);
/* cpuBackend.MatMul Q8_0 branch, internal/compute/cpuref.go:128-135 */
void fr_hal_q8_matmul(const int8_t *codes, const float *scales, const float *x, float *y,
                      int out, int in, int block);
/* cpuBackend.BatchedMatMul Q8_0 branch, internal/compute/cpuref.go:160-176 */
void fr_hal_q8_batched_matmul(const int8_t *codes, const float *scales, const float *X,
                              float *Y, int out, int in, int P, int block);

/* Row-parallel drivers, internal/model/parallel.go:266-330: [0,out) is cut into
 * ceil(out / (workers*4)) sized chunks grabbed dynamically by `workers` threads. Each row is
 * computed by exactly one thread with the serial arithmetic, so results are bit-identical to
 * the serial *_range call for any worker count. Return 0 on success. */
/* the int8 Q4_K decode route (FAK_KQ_INT8), internal/model/quant_q4k_int8.go:72-142 */
void fr_q4k_reduce_row(const uint8_t *row, int nblk, const int8_t *qx, int32_t *IS, int32_t *SS);
float fr_q4k_combine_row(const uint8_t *row, int nblk, const float *dx, const int32_t *IS,
                         const int32_t *SS);
void fr_q4k_matrows_int8(const uint8_t *raw, int out, int in, const float *x, float *y);

int fr_q4k_matrows_par(const uint8_t *raw, int out, int in, const float *x, float *y,
                       int workers);
int fr_q4k_gemm_par(const uint8_t *raw, int out, int in, const float *X, int P, float *Y,
                    int workers);
int fr_q8_0_matrows_par(const uint8_t *raw, int out, int in, const float *x, float *y,
                        int workers);

#ifdef __cplusplus
}
#endif
#endif
