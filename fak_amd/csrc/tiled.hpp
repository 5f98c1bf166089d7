// tiled.hpp — the backend-private device layouts of GGUF Q4_K and Q8_0 weights.
//
// Q4_K tiled layout. A weight [N rows][K/256 super-blocks] of 144-byte GGUF super-blocks
// (internal/model/quant_q4k.go:22-26: d f16 | dmin f16 | 12 B packed 6-bit scales/mins | 128 B
// nibbles) is cut into tiles of 16 rows. Tile T, super-block b becomes one 2304-byte record at
// byte ((T * nblk) + b) * 2304:
//
//   [0, 256)        16 row headers: row r's bytes [0,16) (d, dmin, scales) at offset 16*r.
//   [256, 1280)     "part 0": 64 lanes x 16 B. Lane l = 16*g + r holds row r's nibble bytes
//                   qs[8g .. 8g+8) ++ qs[32+8g .. 32+8g+8)    (qs = super-block bytes [16,144)).
//   [1280, 2304)    "part 1": the same for qs[64+8g ..) ++ qs[96+8g ..).
//
// One 64-lane wave therefore reads a record with three perfectly coalesced 16-byte loads per
// lane (header, part 0, part 1), and the 16 bytes a lane gets are exactly the nibbles it feeds
// to a 16x16x32 MFMA as the weight operand for output row r and K-group g. Nibble byte
// 32c + 8g + i (chunk c = 0..3, i = 0..7) carries weight 64c + 8g + i in its low nibble and
// weight 64c + 32 + 8g + i in its high nibble — the GGUF order of q4kDequantSuperBlock
// (internal/model/quant_q4k.go:97-110). Rows past N in the last tile are zero bytes (d = 0).
// The byte count is N_pad/16 * nblk * 2304 = N_pad * nblk * 144: the GGUF size, padded to 16
// rows.
//
// Q6_K tiled layout. A weight [N][K/256] of 210-byte GGUF super-blocks (ql[128] | qh[64] |
// int8 scales[16] | f16 d; internal/model/quant_kquant.go:139-163) is cut into tiles of 16 rows.
// Tile T, super-block b becomes one 3360-byte record at byte ((T * nblk) + b) * 3360:
//
//   [0, 256)        row r's 16 scales at 16 r (dword c, byte g = scale of group 4c + g)
//   [256, 288)      row r's f16 d at 256 + 2 r
//   [288, 2336)     ql: half h, lane l = 16 g + r at 288 + 1024 h + 16 l: row r's ql bytes
//                   [64 h + 16 g, +16)
//   [2336, 3360)    qh: half h, g1 = g & 1 at 2336 + 512 h + 256 g1 + 16 r: row r's qh bytes
//                   [32 h + 16 g1, +16)
//
// Weight 128 h + 32 i + l of a super-block (l < 32) is the low (i < 2) or high (i >= 2) nibble
// of ql[64 h + 32 (i & 1) + l] with bits 2i..2i+1 of qh[32 h + l] above it, so the 16 weights
// of group j = 8 h + 4 k + g (k = i >> 1 ... i = 2k + (g >> 1), l = 16 (g & 1) + pos) are the
// nibble k of lane l's 16 ql bytes and the 2-bit field 4k + 2 (g >> 1) of its 16 qh bytes: one
// 16-byte operand per lane and 16x16x64 MFMA. Rows past N are zero bytes (d = 0).
//
// Q8_0 tiled layout. A weight [N][K/32] of 34-byte blocks (f16 d + 32 int8; gguf.go:24) is cut
// into tiles of 16 rows and pairs of blocks (64 weights). Record (T, pair) is 1088 bytes:
//   [0, 64)         16 rows x 2 f16 scales (row r at 4*r).
//   [64, 1088)      64 lanes x 16 B: lane l = 16*g + r holds row r's codes [8g, 8g+8) of the
//                   pair's first block ++ codes [8g, 8g+8) of its second block.
// Each 32-weight block is one K=32 MFMA step, exactly like a Q4_K sub-block. An odd final block
// (K/32 odd) is paired with a zero block (d = 0, codes 0).
#pragma once

#include <cstddef>
#include <cstdint>

namespace fhip {

constexpr int kTileRows = 16;
constexpr int kQ4kBlock = 144;
constexpr int kQ4kRecord = 2304;  // 16 rows x 144 B
constexpr int kQ4kHdr = 256;

constexpr int kQ8Block = 34;
constexpr int kQ8Group = 2;        // blocks per record
constexpr int kQ8Record = 1088;    // 16 rows x 2 blocks x 34 B
constexpr int kQ8Hdr = 64;

inline int ceil_div(int a, int b) { return (a + b - 1) / b; }
inline int q4k_tiles(int out) { return ceil_div(out, kTileRows); }
inline size_t q4k_packed_bytes(int out, int in) {
  return (size_t)q4k_tiles(out) * (size_t)(in / 256) * kQ4kRecord;
}
constexpr int kQ6kBlock = 210;
constexpr int kQ6kRecord = 3360;  // 16 rows x 210 B
constexpr int kQ6kD = 256, kQ6kQl = 288, kQ6kQh = 2336;
inline size_t q6k_packed_bytes(int out, int in) {
  return (size_t)q4k_tiles(out) * (size_t)(in / 256) * kQ6kRecord;
}

inline int q8_groups(int in) { return ceil_div(in / 32, kQ8Group); }
inline size_t q8_packed_bytes(int out, int in) {
  return (size_t)q4k_tiles(out) * (size_t)q8_groups(in) * kQ8Record;
}

}  // namespace fhip
