// probe.hip — measurement hooks for the decode GEMV's bandwidth floors: the time a launch needs
// just to move the bytes, with no arithmetic, in two access patterns.
//   * fhip_probe_read: every byte of a buffer read once with 16-byte non-temporal loads, each
//     workgroup a contiguous 16 KB and each thread issuing its four loads before using any (the
//     plain-read ceiling of one launch);
//   * fhip_probe_q4k_records: the one-token GEMV's own pattern over a tiled Q4_K weight (its
//     grid, its workgroup shape, each wave's contiguous part of a tile's records, the same three
//     16-byte non-temporal loads per lane and record, a four-record ring), with the arithmetic
//     replaced by an XOR of the loaded words.
// Each wave folds what it loaded into one word, written to `sink`, so no load can be dropped.
// No counterpart in the reference: these are for profiling this backend.
#include <cstdint>

#include "kernels.hpp"

using namespace fhip;

namespace {

__device__ __forceinline__ uint32_t fold(uint4 v) { return v.x ^ v.y ^ v.z ^ v.w; }

__device__ __forceinline__ uint32_t wave_xor(uint32_t v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v ^= (uint32_t)__shfl_xor((int)v, m);
  return v;
}

// Workgroup w reads the contiguous 16 KB [w * 16 KB, (w + 1) * 16 KB): each thread kReadPer
// 16-byte values, all issued before any is used (one round trip), then folds them. Of the
// shapes swept at 38 MB (grid-stride or contiguous per workgroup, 4 to 32 values per thread,
// cached or non-temporal loads) this one read fastest: 7.3 us back to back (5.2 TB/s).
constexpr int kReadPer = 4;
__global__ __launch_bounds__(256) void probe_read_kernel(const uint4 *__restrict__ p, size_t n16,
                                                         uint32_t *__restrict__ sink) {
  const size_t base = (size_t)blockIdx.x * 256 * kReadPer + threadIdx.x;
  uint4 v[kReadPer];
#pragma unroll
  for (int j = 0; j < kReadPer; ++j) {
    const size_t i = base + (size_t)j * 256;
    v[j] = i < n16 ? ld_stream(p + i) : make_uint4(0, 0, 0, 0);
  }
  uint32_t acc = 0;
#pragma unroll
  for (int j = 0; j < kReadPer; ++j) acc ^= fold(v[j]);
  acc = wave_xor(acc);
  if ((threadIdx.x & 63) == 0) sink[(blockIdx.x * blockDim.x + threadIdx.x) >> 6] = acc;
}

// Workgroups of a plain read of n16 16-byte values (kReadPer per thread).
unsigned read_grid(size_t n16) { return (unsigned)((n16 + 256 * kReadPer - 1) / (256 * kReadPer)); }

__global__ __launch_bounds__(1024) void probe_records_kernel(const uint8_t *__restrict__ W,
                                                             int ntiles, int nblk, int TW, int KW,
                                                             uint32_t *__restrict__ sink) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15;
  const int tile = wave / KW, part = wave - tile * KW;
  const int T = blockIdx.x * TW + tile;
  uint32_t acc = 0;
  if (T < ntiles) {
    const int b0 = part * nblk / KW, b1 = (part + 1) * nblk / KW;
    const uint8_t *base = W + (size_t)T * nblk * kQ4kRecord;
    constexpr int PF = 4;
    uint4 ring[PF][3];
    auto load = [&](int b, uint4 (&o)[3]) {
      const uint8_t *rec = base + (size_t)b * kQ4kRecord;
      o[0] = ld_stream(rec + 16 * r);
      o[1] = ld_stream(rec + kQ4kHdr + 16 * lane);
      o[2] = ld_stream(rec + kQ4kHdr + 1024 + 16 * lane);
    };
#pragma unroll
    for (int u = 0; u < PF; ++u)
      if (b0 + u < b1) load(b0 + u, ring[u]);
    for (int bb = b0; bb < b1; bb += PF) {
#pragma unroll
      for (int u = 0; u < PF; ++u) {
        const int b = bb + u;
        if (b >= b1) break;
        acc ^= fold(ring[u][0]) ^ fold(ring[u][1]) ^ fold(ring[u][2]);
        if (b + PF < b1) load(b + PF, ring[u]);
      }
    }
  }
  acc = wave_xor(acc);
  if (lane == 0) sink[blockIdx.x * (TW * KW) + wave] = acc;
}

}  // namespace

extern "C" {

size_t fhip_probe_read_sink_words(size_t bytes) { return (size_t)read_grid(bytes / 16) * 4; }

int fhip_probe_read(const void *d, size_t bytes, uint32_t *dSink) {
  clear_error();
  if (!d || !dSink || bytes % 16 || ((uintptr_t)d & 15))
    return fail(FHIP_EINVAL, "fhip_probe_read: need a 16-byte aligned buffer of a multiple of 16 "
                             "bytes and a sink");
  const unsigned grid = read_grid(bytes / 16);
  if (grid == 0) return FHIP_OK;
  probe_read_kernel<<<grid, 256, 0, stream()>>>(reinterpret_cast<const uint4 *>(d), bytes / 16,
                                                dSink);
  FHIP_CHECK_LAUNCH("probe_read_kernel");
  return FHIP_OK;
}

size_t fhip_probe_q4k_records_sink_words(int out, int in) {
  if (out <= 0 || in <= 0 || in % 256) return 0;
  int TW, KW;
  q4k_gemv1_shape(q4k_tiles(out), in, TW, KW);
  return (size_t)ceil_div(q4k_tiles(out), TW) * TW * KW;
}

int fhip_probe_q4k_records(const void *dPacked, int out, int in, uint32_t *dSink) {
  clear_error();
  if (out <= 0 || in <= 0 || in % 256 || !dSink)
    return fail(FHIP_EINVAL, "fhip_probe_q4k_records: bad shape or null sink");
  if (int rc = check_weight("fhip_probe_q4k_records", dPacked, kWeightQ4K, out, in)) return rc;
  const int ntiles = q4k_tiles(out), nblk = in / 256;
  int TW, KW;
  q4k_gemv1_shape(ntiles, in, TW, KW);
  probe_records_kernel<<<ceil_div(ntiles, TW), 64 * TW * KW, 0, stream()>>>(
      (const uint8_t *)dPacked, ntiles, nblk, TW, KW, dSink);
  FHIP_CHECK_LAUNCH("probe_records_kernel");
  return FHIP_OK;
}

}  // extern "C"
