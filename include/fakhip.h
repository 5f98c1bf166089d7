/* fakhip.h — the flat C ABI of the MI355X (gfx950) HIP backend for fak's GGUF Q4_K / Q8_0
 * dequantize-and-multiply hot path.
 *
 * It is the ROCm twin of the CUDA tenant's flat ABI (internal/compute/cuda_backend.h): a host
 * binding (the Go cgo wrapper, a ctypes stub, a C++ harness) owns shapes, residency policy and
 * tensor types; this header carries only device pointers, sizes and integer status codes. It
 * includes nothing but <stddef.h>/<stdint.h>, so a plain host compiler (cgo's) can parse it.
 *
 * Conventions
 *   - Every entry that can fail returns int: 0 = ok; FHIP_EINVAL (-1) = bad argument (shape,
 *     null pointer, unsupported size); FHIP_ENODEV (-2) = no usable gfx950 device;
 *     FHIP_ENOMEM (-3) = allocation failed; 1000 + hipError_t = a HIP runtime error.
 *     fhip_last_error() returns a human-readable message for the last failure on the calling
 *     thread. (The CUDA ABI returned void and printed; cuda_backend.h:227-237 already used
 *     int codes for its NCCL entries, which this ABI adopts throughout.)
 *   - Pointers named d* are device pointers, h* are host pointers.
 *   - All launches and async copies go to the library's current stream (fhip_set_stream; the
 *     null/default stream until set). Calls are NOT thread-safe: the host serializes them,
 *     exactly as the CUDA tenant's single cudaMu mutex does (internal/compute/cuda.go:40-43).
 *     Work queued on different streams may run concurrently: the library keeps one scratch
 *     workspace per stream, so matmuls on two streams never share scratch.
 *   - Weights are uploaded once in a backend-private "tiled" layout (fhip_*_upload /
 *     fhip_*_repack). The layout is a lossless byte permutation of the GGUF blocks (the exact
 *     inverse is fhip_*_unpack); it costs the same 144 B per 256 Q4_K weights, 210 B per 256
 *     Q6_K weights and 34 B per 32 Q8_0 weights, padded only to a multiple of 16 output rows.
 *     The library records the format and shape of every tiled weight it lays out; the matmul,
 *     unpack and dequant entries return FHIP_EINVAL for a pointer that does not start a tiled
 *     weight of the format and [out, in] they are given (raw GGUF bytes, another shape, a freed
 *     or overwritten buffer). Writing into a tiled weight through any entry (fhip_h2d /
 *     fhip_h2d_async / fhip_memset_async / a partial fhip_d2d, the output of an unpack,
 *     dequant, quantize, matmul or MLP call), or freeing it, drops the record; an fhip_d2d of a
 *     whole tiled weight records the copy as the same weight.
 *   - Launch-shape overrides (FAK_HIP_GEMV_TW/_KW, FAK_HIP_GEMV_GLOBALX, FAK_HIP_GEMV16_FROM,
 *     FAK_HIP_GEMM32_FORM/_SK/_NWB, FAK_HIP_I8R_KW, FAK_HIP_Q8_TW/_KW) are read from the
 *     environment by fhip_init only, never per call.
 */
#ifndef FAK_HIP_BACKEND_H
#define FAK_HIP_BACKEND_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FHIP_OK 0
#define FHIP_EINVAL (-1)
#define FHIP_ENODEV (-2)
#define FHIP_ENOMEM (-3)

/* ---- runtime ----------------------------------------------------------------------------- */

/* Select device 0, verify it is gfx950, and report its name (up to namelen-1 chars), gfx
 * arch number (e.g. 950) and total memory; (re)read the launch-shape overrides. Idempotent.
 * Replaces fcuda_init (internal/compute/cuda_backend.h:25). Non-zero when no gfx950 device is
 * reachable. */
int fhip_init(char *name, int namelen, int *arch, size_t *total_mem);
/* Replaces fcuda_mem_info (cuda_backend.h:28). */
int fhip_mem_info(size_t *free_mem, size_t *total_mem);
/* Message for the last failing call on this thread ("" if none). */
const char *fhip_last_error(void);

/* Device memory from a size-bucketed pool: fhip_free returns the block to the pool, not to the
 * driver (fcuda_malloc / fcuda_free / fcuda_trim_pool_large, cuda_backend.h:31-34).
 * fhip_malloc returns NULL on failure (reason via fhip_last_error). */
void *fhip_malloc(size_t bytes);
void fhip_free(void *d);
/* Release pooled (free) blocks until at most max_keep_bytes stay cached. */
void fhip_trim_pool(size_t max_keep_bytes);
/* Synchronous copies (fcuda_h2d / fcuda_d2h / fcuda_d2d, cuda_backend.h:35-37) and a device
 * synchronize (fcuda_sync, :38). */
int fhip_h2d(void *d, const void *h, size_t bytes);
int fhip_d2h(void *h, const void *d, size_t bytes);
int fhip_d2d(void *dst, const void *src, size_t bytes);
int fhip_sync(void);
/* Asynchronous copies on the current stream (no counterpart in the CUDA ABI, which ran
 * every copy synchronously on its single g_stream). */
int fhip_h2d_async(void *d, const void *h, size_t bytes);
int fhip_d2h_async(void *h, const void *d, size_t bytes);
int fhip_memset_async(void *d, int value, size_t bytes);

/* Streams and events (the CUDA tenant has one global g_stream, cuda_kernels.cu:28-32; this
 * backend exposes the stream as a handle so a host can overlap work or capture graphs).
 * Streams are created at the default priority. Each stream gets its own scratch workspace on
 * first use. Destroying a stream (or outgrowing its workspace) frees the buffer once the stream
 * has drained; if a graph was ever captured on the stream the buffer is kept instead, since the
 * graph's kernels may still use it, and fhip_trim_pool frees such buffers once no graph is
 * alive. */
int fhip_stream_create(void **stream);
int fhip_stream_destroy(void *stream);
/* Make `stream` (NULL = the default stream) the target of every later launch and async copy. */
int fhip_set_stream(void *stream);
int fhip_stream_sync(void *stream);
/* Graph capture of a sequence of calls (e.g. one decode token), the role of the reference's
 * CUDA graph (internal/compute/cuda_kernels.cu:977-1043). Capture runs on the current stream,
 * which must come from fhip_stream_create. Between begin and end only launch-only calls may be
 * made: the *_matmul_f32 / *_group_f32 entries and fhip_q8_quantize_f32 (no fhip_malloc, no
 * synchronous copies, no fhip_memset_async: memset nodes are not allowed in these graphs). Run
 * each call once before capture so the library workspace already has its size. A graph replays
 * the captured launches with the same device pointers on the stream it was captured on, which
 * must be current (fhip_graph_launch returns FHIP_EINVAL otherwise: its kernels use that
 * stream's workspace and would race with work queued there). */
int fhip_graph_begin(void);
int fhip_graph_end(void **graph);
int fhip_graph_launch(void *graph);
int fhip_graph_destroy(void *graph);
int fhip_event_create(void **event);
int fhip_event_destroy(void *event);
/* Record on the current stream. */
int fhip_event_record(void *event);
/* Wait for `end`, then report the elapsed milliseconds between two recorded events. */
int fhip_event_elapsed_ms(void *start, void *end, float *ms);
/* Measurement hook (no counterpart in the reference): the next 1..4-token Q4_K GEMV launch
 * records `start` and `stop` at its own dispatch's start and end (hipExtLaunchKernel), so
 * fhip_event_elapsed_ms gives that kernel's duration without queue or host time. Refused
 * during graph capture; captured launches leave a pending pair for the next eager one. */
int fhip_time_next_launch(void *start, void *stop);

/* ---- Q4_K (256-weight super-blocks of 144 B: f16 d, f16 dmin, 12 B of 6-bit scales/mins,
 *      128 B of nibbles; internal/model/quant_q4k.go:22-26) ------------------------------- */

/* Bytes of the tiled layout for an [out, in] weight (in % 256 == 0). */
size_t fhip_q4k_packed_bytes(int out, int in);
/* dPacked <- tiled layout of the raw row-major GGUF bytes dRaw (out*(in/256)*144 bytes). */
int fhip_q4k_repack(void *dPacked, const uint8_t *dRaw, int out, int in);
/* dRaw <- raw GGUF bytes recovered from the tiled layout (exact inverse of fhip_q4k_repack). */
int fhip_q4k_unpack(uint8_t *dRaw, const void *dPacked, int out, int in);
/* dW[out*in] <- f32 dequantized weights, bit-identical to q4kDequantSuperBlock
 * (internal/model/quant_q4k.go:90-111) for every input, NaN payloads included. Test hook. */
int fhip_q4k_dequant_f32(float *dW, const void *dPacked, int out, int in);
/* Allocate (pool) a tiled Q4_K weight and fill it from host raw GGUF bytes: the upload path
 * of uploadQ4K (internal/compute/cuda.go:803-822). Returns NULL on failure. Free with
 * fhip_free. */
void *fhip_q4k_upload(const uint8_t *hRaw, int out, int in);
/* Y[P,out] = X[P,in] @ W[out,in]^T with W a tiled Q4_K weight, X and Y row-major f32 — the
 * replacement for fcuda_q4k_matmul_f32 (internal/compute/cuda_backend.h:120), which took the
 * raw bytes; this one takes the tiled buffer fhip_q4k_upload / fhip_q4k_repack produced and
 * returns FHIP_EINVAL for anything else (see Conventions).
 * P <= 16 runs the small-M GEMV (decode / speculative verify); 17 <= P <= 32 the same 32x32
 * kernel with one f16 activation row per token (small prefill chunks); larger P the MFMA GEMM.
 * Error bound vs the f32 reference: GEMV max|dY|/RMS(Y) <= 1e-3, GEMM <= 1e-2. */
int fhip_q4k_matmul_f32(const void *dPacked, const float *dX, float *dY, int out, int in,
                        int P);
/* count (1..8) tiled Q4_K weights [out[i]][in] that share one activation X[P,in] (a layer's
 * q/k/v or gate/up): Y_i = X @ W_i^T for each i — the group dispatch of q4kGroupDispatch /
 * metalgemm.GEMVGroup (internal/model/metal_q4k_on.go:139-190), which runs the members in one
 * command buffer. dPacked, dY and out are host arrays of device pointers / row counts. For
 * P <= 4 the members run as one grid that quantizes X once; otherwise one call per member.
 * Each Y_i meets the fhip_q4k_matmul_f32 bound (not bit-identical to it: the K split may differ). */
int fhip_q4k_matmul_group_f32(const void *const *dPacked, float *const *dY, const int *out,
                              int count, const float *dX, int in, int P);
/* The int8 Q4_K route (FAK_KQ_INT8): Y[P,out] from a tiled Q4_K weight with every activation row
 * quantized to int8 per 32 values — the replacement for q4kMatRowsInto / q4kGemmInto when
 * q4kSDOTEnabled (internal/model/quant_q4k.go:125-136,190-218 -> q4kMatRowsRangeInt8,
 * internal/model/quant_q4k_int8.go:135-142, and per token q4kGemmRangeInt8, quant_q4k.go:
 * 359-372). Every value is bit-identical to that CPU route (quantizeRowQ8scalar, the int32
 * sub-block sums, and q4kCombineRow's f32 chain in its order). dX must be 16-byte aligned. */
int fhip_q4k_matmul_int8_f32(const void *dPacked, const float *dX, float *dY, int out, int in,
                             int P);

/* The same matmul for callers that cannot allocate device memory: code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc. No counterpart in the
 * reference. It runs the kernels of fhip_q4k_matmul_f32 (same results, bit for bit) but keeps
 * their scratch (activation operands, token scales, K-range partial sums) in a static 64 MiB
 * device array per device instead of the library workspace, and calls no hipMalloc / hipFree.
 * A call whose scratch would exceed 64 MiB returns FHIP_EINVAL without launching anything.
 * The scratch is: for 1..4 tokens at most in/256 * 3.3 KB; for 5..32 tokens (3..32 when
 * in >= 24576) the K-range partial sums, 4 * P * out bytes per 1,024 values of in (about
 * in * out * P / 256 bytes); for the prefill GEMM its f16 operands (2 * P * in bytes) plus
 * partial sums when K is split. So every 7B / 27B FFN, attention and 152064 x 3584 lm_head
 * call of up to 32 tokens fits, and so does a prefill of 512 tokens at the 7B shapes; a
 * 16-token call on a 17408 x 65536 weight (71 MB) and a 1,024-token prefill through the
 * 18944 -> 3584 projection do not. The array keeps the last call's contents and is shared by
 * every call on the device: calls that overlap on one device (two streams, two threads) race on
 * it. */
int fhip_q4k_matmul_noalloc_f32(const void *dPacked, const float *dX, float *dY, int out, int in,
                                int P);

/* Measurement hooks for the decode GEMV's bandwidth floors (no counterpart in the reference;
 * for profiling this backend). Each folds what it reads into one word per wave, written to
 * dSink (a device buffer of the *_sink_words count of uint32), so no load is dropped.
 * fhip_probe_read: every byte of d read once (16-byte non-temporal loads, a contiguous 16 KB per
 * workgroup, four per thread all issued before any is used): the plain-read ceiling of one
 * launch.
 * fhip_probe_q4k_records: the one-token GEMV's own grid and record loads over a tiled Q4_K
 * weight, with no arithmetic. */
size_t fhip_probe_read_sink_words(size_t bytes);
int fhip_probe_read(const void *d, size_t bytes, uint32_t *dSink);
size_t fhip_probe_q4k_records_sink_words(int out, int in);
int fhip_probe_q4k_records(const void *dPacked, int out, int in, uint32_t *dSink);

/* ---- Q6_K (256-weight super-blocks of 210 B; internal/model/quant_kquant.go:45,139-163) ---- */

/* Bytes of a raw Q6_K weight [out][in] (in a multiple of 256); 0 for a bad shape. */
size_t fhip_q6k_bytes(int out, int in);
/* Bytes of the tiled device layout (16-row tiles of 3360-byte records; out padded to 16). */
size_t fhip_q6k_packed_bytes(int out, int in);
/* Device raw GGUF rows -> tiled layout, and back (lossless byte permutation). */
int fhip_q6k_repack(void *dPacked, const uint8_t *dRaw, int out, int in);
int fhip_q6k_unpack(uint8_t *dRaw, const void *dPacked, int out, int in);
/* Allocate a tiled Q6_K weight and fill it from host raw GGUF bytes: the resident-weight upload
 * of quantizeKQuantFromRaw(kind Q6_K) (internal/model/quant_kquant.go:236-250). Free with
 * fhip_free. */
void *fhip_q6k_upload(const uint8_t *hRaw, int out, int in);
/* dW[out][in] = the dequantized weights of a tiled Q6_K weight, bit-identical to
 * q6kDequantSuperBlock (internal/model/quant_kquant.go:139-163). Test hook. */
int fhip_q6k_dequant_f32(float *dW, const void *dPacked, int out, int in);
/* Y[P][out] = X[P][in] @ W^T for a tiled Q6_K weight: the replacement for
 * kQuantMatRowsInto(kind Q6_K) (internal/model/quant_kquant.go:188-232), whose f32 route
 * dequantizes each super-block and dots it; bound max|dY|/RMS(Y) <= 1e-3. dX and the weight
 * 16-byte aligned. */
int fhip_q6k_matmul_f32(const void *dPacked, const float *dX, float *dY, int out, int in,
                        int P);

/* ---- Fused decode MLP (dense SwiGLU FFN of one decode step) ------------------------------- */

/* Y[P][hidden] = down(silu(gate X) * (up X)) for P = 0..4 tokens, with silu(z) =
 * z / (1 + f32(exp(f64(-z)))) (internal/model/forward.go:452). gate and up are tiled Q4_K
 * [inter][hidden], down tiled Q4_K [hidden][inter]; hidden and inter multiples of 256. The
 * replacement for mg_q4k_mlp (internal/metalgemm/q4k.m:458-520; FusedMLP,
 * internal/metalgemm/q4k.go:144-161): two launches on the library stream, the intermediate stays
 * on the device, no host synchronization. Each stage meets the GEMV bound; the output is within
 * max|dY|/RMS(Y) <= 1e-3 of the CPU gate/up -> silu*up -> down chain (denseSwiGLU,
 * internal/model/moe.go:111-136). dX and the weights 16-byte aligned. */
int fhip_q4k_mlp_f32(const void *dGate, const void *dUp, const void *dDown, const float *dX,
                     float *dY, int hidden, int inter, int P);
/* The same with a raw Q6_K down projection (fhip_q6k_upload): the q4_k_m layout; the
 * replacement for mg_q4k_mlp_q6down (internal/metalgemm/q4k.m:680-740; FusedMLPQ6Down,
 * internal/metalgemm/q4k.go:180-205). */
int fhip_q4k_mlp_q6down_f32(const void *dGate, const void *dUp, const void *dDownQ6,
                            const float *dX, float *dY, int hidden, int inter, int P);

/* ---- Q8_0 (32-weight blocks of 34 B: f16 d + 32 int8; internal/ggufload/gguf.go:24) ----- */

size_t fhip_q8_0_packed_bytes(int out, int in);
int fhip_q8_0_repack(void *dPacked, const uint8_t *dRaw, int out, int in);
int fhip_q8_0_unpack(uint8_t *dRaw, const void *dPacked, int out, int in);
/* bit-identical to q8_0DequantBlock (internal/model/quant_iquant.go:14-19). Test hook. */
int fhip_q8_0_dequant_f32(float *dW, const void *dPacked, int out, int in);
void *fhip_q8_0_upload(const uint8_t *hRaw, int out, int in);
/* Y[P,out] = X[P,in] @ W^T with W a tiled Q8_0 weight and f32 activations: the device form of
 * kQuantMatRowsRange(kind Q8_0) (internal/model/quant_kquant.go:210-232). f32 accumulate,
 * max|dY|/RMS(Y) <= 1e-3. */
int fhip_q8_0_matmul_f32(const void *dPacked, const float *dX, float *dY, int out, int in,
                         int P);

/* ---- HAL Q8 lane: int8 codes [out][in] + f32 scales [out][in/block], activation quantized on
 * the device (compute.NewQ8 tensors, internal/compute/cpuref.go:53-56) ------------------- */

/* quantizeVecQ8 (internal/compute/cpuref.go:505-527) of each row of X[rows][in]:
 * scales[r][b] = amax/127, codes = q8round(x / scale) (internal/model/quant.go:89-104),
 * all-zero blocks give scale 0 and zero codes. Bit-identical to the CPU reference. The device
 * form of Upload(F32, Q8_0) narrowing (internal/compute/cuda.go:714-750) and of the activation
 * quantization k_q8_quant_act (internal/compute/cuda_kernels.cu:374-398). */
int fhip_q8_quantize_f32(const float *dX, int8_t *dCodes, float *dScales, int rows, int in,
                         int block);
/* Y[P,out] = X[P,in] @ W^T on a HAL Q8 weight: the replacement for fcuda_q8_matmul_f32
 * (internal/compute/cuda_backend.h:110-111), same arguments. X is quantized per row on the
 * device (quantizeVecQ8), then P == 1 follows qdot8scalar (cpuref.go:532-548, MatMul) and
 * P > 1 follows qgemm8cell with 16 lanes (cpuref.go:553-577, BatchedMatMul): results are
 * bit-identical to cpuBackend.MatMul / BatchedMatMul. block must divide in and be a multiple of
 * 4; P > 1 needs block >= 32 (the reference reads 16 pairs per block). dCodes 4-byte aligned. */
int fhip_q8_matmul_f32(const int8_t *dCodes, const float *dScales, const float *dX, float *dY,
                       int out, int in, int P, int block);

#ifdef __cplusplus
}
#endif
#endif
