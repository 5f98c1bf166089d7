/* fakref.c — ORACLE (test infrastructure only): C restatement of fak's Go CPU Q4_K / Q8_0
 * matmul path. See fakref.h for the per-function citations and pinning status.
 *
 * Build: gcc -O2 -ffp-contract=off -fno-fast-math -fPIC -shared (oracle/build.py). The
 * contraction switch is load-bearing: the reference dequant `d1*float32(nib) - m1` rounds the
 * product before the subtraction, and the 4-accumulator dot rounds every product before it is
 * added (amd64 Go never fuses; internal/model/quant.go:80-86 records why fusion breaks
 * determinism on arm64).
 */
#include "fakref.h"

#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>

#define QK_K 256
#define Q4K_BLOCK_BYTES 144 /* internal/model/quant_q4k.go:52 */
#define Q8_0_BLOCK_WEIGHTS 32
#define Q8_0_BLOCK_BYTES 34 /* internal/model/quant_kquant.go:48-49 */
#define Q6K_BLOCK_BYTES 210 /* internal/model/quant_kquant.go:45: 128 + 64 + 16 + 2 */

static inline float bits_f32(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static inline uint16_t le16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* internal/model/quantbits.go:15-36 */
uint32_t fr_f16_bits_to_f32_bits(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  int exp = (int)((h >> 10) & 0x1f);
  uint32_t frac = (uint32_t)(h & 0x03ffu);
  switch (exp) {
  case 0:
    if (frac == 0) return sign;
    exp = -14;
    while ((frac & 0x0400u) == 0) {
      frac <<= 1;
      exp--;
    }
    frac &= 0x03ffu;
    return sign | ((uint32_t)(exp + 127) << 23) | (frac << 13);
  case 0x1f:
    return sign | 0x7f800000u | (frac << 13);
  default:
    return sign | ((uint32_t)(exp - 15 + 127) << 23) | (frac << 13);
  }
}

/* internal/model/quantbits.go:42-47 */
void fr_get_scale_min_k4(int j, const uint8_t *q, uint8_t *scale, uint8_t *min) {
  if (j < 4) {
    *scale = q[j] & 63;
    *min = q[j + 4] & 63;
    return;
  }
  *scale = (uint8_t)((q[j + 4] & 0x0f) | ((q[j - 4] >> 6) << 4));
  *min = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
}

/* internal/model/quant_q4k.go:90-111 */
void fr_q4k_dequant_superblock(float *dst, const uint8_t *blk) {
  const float d = bits_f32(fr_f16_bits_to_f32_bits(le16(blk + 0)));
  const float mn = bits_f32(fr_f16_bits_to_f32_bits(le16(blk + 2)));
  const uint8_t *scales = blk + 4;
  const uint8_t *q = blk + 16;
  int qi = 0, is = 0;
  for (int j = 0; j < QK_K; j += 64) {
    uint8_t sc, m;
    fr_get_scale_min_k4(is, scales, &sc, &m);
    const float d1 = d * (float)sc, m1 = mn * (float)m;
    fr_get_scale_min_k4(is + 1, scales, &sc, &m);
    const float d2 = d * (float)sc, m2 = mn * (float)m;
    for (int l = 0; l < 32; l++) dst[j + l] = d1 * (float)(q[qi + l] & 0x0f) - m1;
    for (int l = 0; l < 32; l++) dst[j + 32 + l] = d2 * (float)(q[qi + l] >> 4) - m2;
    qi += 32;
    is += 2;
  }
}

void fr_q4k_dequant_row(float *dst, const uint8_t *raw, int nblk) {
  for (int b = 0; b < nblk; b++)
    fr_q4k_dequant_superblock(dst + (size_t)b * QK_K, raw + (size_t)b * Q4K_BLOCK_BYTES);
}

/* The per-super-block 4-accumulator dot, internal/model/quant_q4k.go:154-161. */
static inline float dot4_256(const float *buf, const float *xs) {
  float s0 = 0, s1 = 0, s2 = 0, s3 = 0;
  for (int i = 0; i < QK_K; i += 4) {
    s0 += buf[i] * xs[i];
    s1 += buf[i + 1] * xs[i + 1];
    s2 += buf[i + 2] * xs[i + 2];
    s3 += buf[i + 3] * xs[i + 3];
  }
  return (s0 + s1) + (s2 + s3);
}

/* internal/model/quant_q4k.go:145-165 */
void fr_q4k_matrows_range(const uint8_t *raw, int out, int in, const float *x, float *y,
                          int lo, int hi) {
  (void)out;
  const int nblk = in / QK_K;
  const size_t rowBytes = (size_t)nblk * Q4K_BLOCK_BYTES;
  float buf[QK_K];
  for (int o = lo; o < hi; o++) {
    const uint8_t *row = raw + (size_t)o * rowBytes;
    float acc = 0;
    for (int b = 0; b < nblk; b++) {
      fr_q4k_dequant_superblock(buf, row + (size_t)b * Q4K_BLOCK_BYTES);
      acc += dot4_256(buf, x + (size_t)b * QK_K);
    }
    y[o] = acc;
  }
}

/* internal/model/quant_q4k.go:378-405 */
void fr_q4k_gemm_range(const uint8_t *raw, int out, int in, const float *X, int P, float *Y,
                       int lo, int hi) {
  const int nblk = in / QK_K;
  const size_t rowBytes = (size_t)nblk * Q4K_BLOCK_BYTES;
  float buf[QK_K];
  float *acc = (float *)malloc(sizeof(float) * (size_t)(P > 0 ? P : 1));
  for (int o = lo; o < hi; o++) {
    const uint8_t *row = raw + (size_t)o * rowBytes;
    for (int t = 0; t < P; t++) acc[t] = 0;
    for (int b = 0; b < nblk; b++) {
      fr_q4k_dequant_superblock(buf, row + (size_t)b * Q4K_BLOCK_BYTES);
      for (int t = 0; t < P; t++) acc[t] += dot4_256(buf, X + (size_t)t * in + (size_t)b * QK_K);
    }
    for (int t = 0; t < P; t++) Y[(size_t)t * out + o] = acc[t];
  }
  free(acc);
}

/* internal/model/quant_iquant.go:14-19 */
void fr_q8_0_dequant_block(float *dst, const uint8_t *blk) {
  const float d = bits_f32(fr_f16_bits_to_f32_bits(le16(blk)));
  for (int j = 0; j < Q8_0_BLOCK_WEIGHTS; j++) dst[j] = (float)(int8_t)blk[2 + j] * d;
}

/* internal/model/quant_kquant.go:210-232, kind Q8_0 */
void fr_q8_0_matrows_range(const uint8_t *raw, int out, int in, const float *x, float *y,
                           int lo, int hi) {
  (void)out;
  const int nblk = in / Q8_0_BLOCK_WEIGHTS;
  const size_t rowBytes = (size_t)nblk * Q8_0_BLOCK_BYTES;
  float buf[Q8_0_BLOCK_WEIGHTS];
  for (int o = lo; o < hi; o++) {
    const uint8_t *row = raw + (size_t)o * rowBytes;
    float acc = 0;
    for (int b = 0; b < nblk; b++) {
      fr_q8_0_dequant_block(buf, row + (size_t)b * Q8_0_BLOCK_BYTES);
      const float *xs = x + (size_t)b * Q8_0_BLOCK_WEIGHTS;
      float s0 = 0, s1 = 0, s2 = 0, s3 = 0;
      for (int i = 0; i < Q8_0_BLOCK_WEIGHTS; i += 4) {
        s0 += buf[i] * xs[i];
        s1 += buf[i + 1] * xs[i + 1];
        s2 += buf[i + 2] * xs[i + 2];
        s3 += buf[i + 3] * xs[i + 3];
      }
      acc += (s0 + s1) + (s2 + s3);
    }
    y[o] = acc;
  }
}

/* internal/model/quant_kquant.go:139-163 (q6kDequantSuperBlock): 210-byte super-block, ql[128]
 * low nibbles, qh[64] high 2-bit pairs, 16 int8 scales, f16 d at byte 208;
 * w = (d * f32(int8 scale)) * f32(q - 32). */
void fr_q6k_dequant_superblock(float *dst, const uint8_t *blk) {
  const uint8_t *ql = blk, *qh = blk + 128, *sc = blk + 192;
  const float d = bits_f32(fr_f16_bits_to_f32_bits(le16(blk + Q6K_BLOCK_BYTES - 2)));
  int qlOff = 0, qhOff = 0, scOff = 0;
  for (int n = 0; n < QK_K; n += 128) {
    for (int l = 0; l < 32; l++) {
      const int is = l / 16;
      const int8_t q1 = (int8_t)((ql[qlOff + l] & 0x0f) | (((qh[qhOff + l] >> 0) & 3) << 4)) - 32;
      const int8_t q2 = (int8_t)((ql[qlOff + l + 32] & 0x0f) | (((qh[qhOff + l] >> 2) & 3) << 4)) - 32;
      const int8_t q3 = (int8_t)((ql[qlOff + l] >> 4) | (((qh[qhOff + l] >> 4) & 3) << 4)) - 32;
      const int8_t q4 = (int8_t)((ql[qlOff + l + 32] >> 4) | (((qh[qhOff + l] >> 6) & 3) << 4)) - 32;
      dst[n + l + 0] = d * (float)(int8_t)sc[scOff + is + 0] * (float)q1;
      dst[n + l + 32] = d * (float)(int8_t)sc[scOff + is + 2] * (float)q2;
      dst[n + l + 64] = d * (float)(int8_t)sc[scOff + is + 4] * (float)q3;
      dst[n + l + 96] = d * (float)(int8_t)sc[scOff + is + 6] * (float)q4;
    }
    qlOff += 64;
    qhOff += 32;
    scOff += 8;
  }
}

/* internal/model/quant_kquant.go:210-232 with kind Q6_K (blockWeights 256, blockBytes 210) */
void fr_q6k_matrows_range(const uint8_t *raw, int out, int in, const float *x, float *y, int lo,
                          int hi) {
  (void)out;
  const int nblk = in / QK_K;
  const size_t rowBytes = (size_t)nblk * Q6K_BLOCK_BYTES;
  float buf[QK_K];
  for (int o = lo; o < hi; o++) {
    const uint8_t *row = raw + (size_t)o * rowBytes;
    float acc = 0;
    for (int b = 0; b < nblk; b++) {
      fr_q6k_dequant_superblock(buf, row + (size_t)b * Q6K_BLOCK_BYTES);
      const float *xs = x + (size_t)b * QK_K;
      float s0 = 0, s1 = 0, s2 = 0, s3 = 0;
      for (int i = 0; i < QK_K; i += 4) {
        s0 += buf[i] * xs[i];
        s1 += buf[i + 1] * xs[i + 1];
        s2 += buf[i + 2] * xs[i + 2];
        s3 += buf[i + 3] * xs[i + 3];
      }
      acc += (s0 + s1) + (s2 + s3);
    }
    y[o] = acc;
  }
}

/* internal/model/forward.go:452: z / (1 + float32(math.Exp(float64(-z)))) */
float fr_silu(float z) { return z / (1.0f + (float)exp(-(double)z)); }

/* the SwiGLU step of denseSwiGLU (internal/model/moe.go:111-136; the same loop as
 * internal/model/profile.go:328): g[i] = silu(g[i]) * u[i] */
void fr_swiglu(float *g, const float *u, int n) {
  for (int i = 0; i < n; i++) g[i] = fr_silu(g[i]) * u[i];
}

/* internal/compute/cpuref.go:486-501 */
static inline float absf_(float v) { return v < 0 ? -v : v; }

int8_t fr_q8round(float x) {
  /* truncate toward zero; NaN and |x| >= 2^31 give amd64's CVTTSS2SI "integer indefinite", and
   * Go's int32 increment/decrement wrap (so -3e9 ends at +127) */
  int32_t t = absf_(x) < 2147483648.f ? (int32_t)x : INT32_MIN;
  float f = x - (float)t;
  if (f >= 0.5f)
    t = (int32_t)((uint32_t)t + 1u);
  else if (f <= -0.5f)
    t = (int32_t)((uint32_t)t - 1u);
  if (t > 127) return 127;
  if (t < -127) return -127;
  return (int8_t)t;
}

static inline float absf(float v) { return v < 0 ? -v : v; }

/* internal/compute/cpuref.go:505-527 */
void fr_quantize_vec_q8(const float *x, int n, int block, int8_t *q, float *d) {
  const int nblk = n / block;
  memset(q, 0, (size_t)n);
  for (int b = 0; b < nblk; b++) {
    const float *blk = x + (size_t)b * block;
    float amax = 0;
    for (int i = 0; i < block; i++) {
      const float a = absf(blk[i]);
      if (a > amax) amax = a;
    }
    const float dd = amax / 127.0f;
    d[b] = dd;
    if (dd == 0) continue;
    const float inv = 1.0f / dd;
    for (int i = 0; i < block; i++) q[(size_t)b * block + i] = fr_q8round(blk[i] * inv);
  }
}

/* internal/compute/cpuref.go:531-549 */
float fr_qdot8(const int8_t *qw, const float *dw, const int8_t *qx, const float *dx, int n,
               int block) {
  const int nblk = n / block;
  float acc = 0;
  for (int b = 0; b < nblk; b++) {
    const int8_t *wb = qw + (size_t)b * block;
    const int8_t *xb = qx + (size_t)b * block;
    int32_t s0 = 0, s1 = 0, s2 = 0, s3 = 0;
    for (int i = 0; i < block; i += 4) {
      s0 += (int32_t)wb[i] * (int32_t)xb[i];
      s1 += (int32_t)wb[i + 1] * (int32_t)xb[i + 1];
      s2 += (int32_t)wb[i + 2] * (int32_t)xb[i + 2];
      s3 += (int32_t)wb[i + 3] * (int32_t)xb[i + 3];
    }
    acc += (float)((s0 + s1) + (s2 + s3)) * dw[b] * dx[b];
  }
  return acc;
}

/* internal/compute/cpuref.go:553-577 (lanes = 16) */
float fr_qgemm8cell(const int8_t *qw, const float *dw, const int8_t *qx, const float *dx,
                    int nblk, int block) {
  float acc[16];
  for (int k = 0; k < 16; k++) acc[k] = 0;
  for (int b = 0; b < nblk; b++) {
    const int8_t *wb = qw + (size_t)b * block;
    const int8_t *xb = qx + (size_t)b * block;
    int32_t p[16];
    for (int kk = 0; kk < 16; kk++)
      p[kk] = (int32_t)wb[2 * kk] * (int32_t)xb[2 * kk] +
              (int32_t)wb[2 * kk + 1] * (int32_t)xb[2 * kk + 1];
    const float s = dw[b] * dx[b];
    for (int kk = 0; kk < 16; kk++) acc[kk] += (float)p[kk] * s;
  }
  for (int kk = 0; kk < 8; kk++) acc[kk] += acc[kk + 8];
  for (int kk = 0; kk < 4; kk++) acc[kk] += acc[kk + 4];
  acc[0] += acc[2];
  acc[1] += acc[3];
  return acc[0] + acc[1];
}

/* internal/compute/cpuref.go:128-135 */
void fr_hal_q8_matmul(const int8_t *codes, const float *scales, const float *x, float *y,
                      int out, int in, int block) {
  const int nblk = in / block;
  int8_t *qx = (int8_t *)malloc((size_t)in);
  float *dx = (float *)malloc(sizeof(float) * (size_t)(nblk > 0 ? nblk : 1));
  fr_quantize_vec_q8(x, in, block, qx, dx);
  for (int o = 0; o < out; o++)
    y[o] = fr_qdot8(codes + (size_t)o * in, scales + (size_t)o * nblk, qx, dx, in, block);
  free(qx);
  free(dx);
}

/* internal/compute/cpuref.go:160-176 */
void fr_hal_q8_batched_matmul(const int8_t *codes, const float *scales, const float *X,
                              float *Y, int out, int in, int P, int block) {
  const int nblk = in / block;
  int8_t *qx = (int8_t *)malloc((size_t)P * in + 1);
  float *dx = (float *)malloc(sizeof(float) * ((size_t)P * nblk + 1));
  for (int t = 0; t < P; t++)
    fr_quantize_vec_q8(X + (size_t)t * in, in, block, qx + (size_t)t * in, dx + (size_t)t * nblk);
  for (int o = 0; o < out; o++)
    for (int t = 0; t < P; t++)
      Y[(size_t)t * out + o] =
          fr_qgemm8cell(codes + (size_t)o * in, scales + (size_t)o * nblk, qx + (size_t)t * in,
                        dx + (size_t)t * nblk, nblk, block);
  free(qx);
  free(dx);
}

/* ---- the int8 Q4_K decode route (FAK_KQ_INT8), internal/model/quant_q4k_int8.go --------- */

/* internal/model/quant_q4k_int8.go:72-100: per sub-block s of super-block b,
 * IS[b*8+s] = sum(nibble * qx), SS[b*8+s] = sum(qx) over the sub-block's 32 values (int32). */
void fr_q4k_reduce_row(const uint8_t *row, int nblk, const int8_t *qx, int32_t *IS, int32_t *SS) {
  for (int b = 0; b < nblk; b++) {
    const uint8_t *q = row + (size_t)b * Q4K_BLOCK_BYTES + 16;
    const int base = b * 8;
    int qi = 0;
    for (int k = 0; k < 4; k++) {
      const int8_t *qxA = qx + (size_t)(base + 2 * k) * 32;
      int32_t IA = 0, SA = 0;
      for (int l = 0; l < 32; l++) {
        IA += (int32_t)(q[qi + l] & 0x0f) * (int32_t)qxA[l];
        SA += (int32_t)qxA[l];
      }
      IS[base + 2 * k] = IA;
      SS[base + 2 * k] = SA;
      const int8_t *qxB = qx + (size_t)(base + 2 * k + 1) * 32;
      int32_t IB = 0, SB = 0;
      for (int l = 0; l < 32; l++) {
        IB += (int32_t)(q[qi + l] >> 4) * (int32_t)qxB[l];
        SB += (int32_t)qxB[l];
      }
      IS[base + 2 * k + 1] = IB;
      SS[base + 2 * k + 1] = SB;
      qi += 32;
    }
  }
}

/* internal/model/quant_q4k_int8.go:110-130: acc += (f32(I)*ws)*dxs; acc -= (f32(S)*wm)*dxs,
 * ws = d*f32(sc), wm = min*f32(m), sub-block 0..7 within each super-block, blocks in order. */
float fr_q4k_combine_row(const uint8_t *row, int nblk, const float *dx, const int32_t *IS,
                         const int32_t *SS) {
  float acc = 0;
  for (int b = 0; b < nblk; b++) {
    const uint8_t *blk = row + (size_t)b * Q4K_BLOCK_BYTES;
    const float d = bits_f32(fr_f16_bits_to_f32_bits(le16(blk + 0)));
    const float mn = bits_f32(fr_f16_bits_to_f32_bits(le16(blk + 2)));
    const int base = b * 8;
    for (int s = 0; s < 8; s++) {
      uint8_t sc, m;
      fr_get_scale_min_k4(s, blk + 4, &sc, &m);
      const float ws = d * (float)sc, wm = mn * (float)m;
      const float dxs = dx[base + s];
      acc += ((float)IS[base + s] * ws) * dxs;
      acc -= ((float)SS[base + s] * wm) * dxs;
    }
  }
  return acc;
}

/* internal/model/quant_q4k_int8.go:135-142 with the activation quantized once by
 * quantizeRowQ8scalar (internal/model/quant_quantize.go:16-43, == fr_quantize_vec_q8, block 32):
 * the int8 decode GEMV of one token. */
void fr_q4k_matrows_int8(const uint8_t *raw, int out, int in, const float *x, float *y) {
  const int nblk = in / QK_K;
  int8_t *qx = (int8_t *)malloc((size_t)in + 1);
  float *dx = (float *)malloc(sizeof(float) * ((size_t)in / 32 + 1));
  int32_t *IS = (int32_t *)malloc(sizeof(int32_t) * ((size_t)nblk * 8 + 1));
  int32_t *SS = (int32_t *)malloc(sizeof(int32_t) * ((size_t)nblk * 8 + 1));
  fr_quantize_vec_q8(x, in, 32, qx, dx);
  const size_t rb = (size_t)nblk * Q4K_BLOCK_BYTES;
  for (int o = 0; o < out; o++) {
    fr_q4k_reduce_row(raw + (size_t)o * rb, nblk, qx, IS, SS);
    y[o] = fr_q4k_combine_row(raw + (size_t)o * rb, nblk, dx, IS, SS);
  }
  free(qx);
  free(dx);
  free(IS);
  free(SS);
}

/* ---- row-parallel drivers: internal/model/parallel.go:266-330 ---------------------------- */

typedef struct {
  int kind; /* 0 q4k gemv, 1 q4k gemm, 2 q8_0 gemv */
  const uint8_t *raw;
  int out, in, P;
  const float *x;
  float *y;
  int chunk;
  int nchunks;
  atomic_int next;
} par_job;

static void run_range(par_job *j, int lo, int hi) {
  switch (j->kind) {
  case 0: fr_q4k_matrows_range(j->raw, j->out, j->in, j->x, j->y, lo, hi); break;
  case 1: fr_q4k_gemm_range(j->raw, j->out, j->in, j->x, j->P, j->y, lo, hi); break;
  default: fr_q8_0_matrows_range(j->raw, j->out, j->in, j->x, j->y, lo, hi); break;
  }
}

static void *par_worker(void *arg) {
  par_job *j = (par_job *)arg;
  for (;;) {
    const int c = atomic_fetch_add(&j->next, 1);
    if (c >= j->nchunks) break;
    const int lo = c * j->chunk;
    int hi = lo + j->chunk;
    if (hi > j->out) hi = j->out;
    run_range(j, lo, hi);
  }
  return NULL;
}

#define PAR_GRANULARITY 4 /* parChunkGranularity, internal/model/parallel.go */

static int par_run(par_job *j, int workers) {
  const int n = j->out;
  if (workers <= 1 || n <= 1) {
    run_range(j, 0, n);
    return 0;
  }
  if (workers > n) workers = n;
  int chunk = (n + workers * PAR_GRANULARITY - 1) / (workers * PAR_GRANULARITY);
  if (chunk < 1) chunk = 1;
  j->chunk = chunk;
  j->nchunks = (n + chunk - 1) / chunk;
  atomic_store(&j->next, 0);
  pthread_t *th = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)workers);
  if (!th) return -1;
  int started = 0;
  for (int w = 0; w < workers - 1; w++) {
    if (pthread_create(&th[w], NULL, par_worker, j) != 0) break;
    started++;
  }
  par_worker(j); /* the caller is the last worker, like parFor */
  for (int w = 0; w < started; w++) pthread_join(th[w], NULL);
  free(th);
  return 0;
}

int fr_q4k_matrows_par(const uint8_t *raw, int out, int in, const float *x, float *y,
                       int workers) {
  par_job j = {.kind = 0, .raw = raw, .out = out, .in = in, .P = 1, .x = x, .y = y};
  return par_run(&j, workers);
}

int fr_q4k_gemm_par(const uint8_t *raw, int out, int in, const float *X, int P, float *Y,
                    int workers) {
  par_job j = {.kind = 1, .raw = raw, .out = out, .in = in, .P = P, .x = X, .y = Y};
  return par_run(&j, workers);
}

int fr_q8_0_matrows_par(const uint8_t *raw, int out, int in, const float *x, float *y,
                        int workers) {
  par_job j = {.kind = 2, .raw = raw, .out = out, .in = in, .P = 1, .x = x, .y = y};
  return par_run(&j, workers);
}
