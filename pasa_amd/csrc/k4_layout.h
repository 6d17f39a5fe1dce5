// LDS images shared by the D = 128 K4 kernel (k4_sparse_attn_dma) and the pack kernel
// that writes its phase-2 operands.
#pragma once

#include "common.h"

namespace pasa {

constexpr int kGroup = 32;  // key blocks per group of the first-order correction

// V^ transposed (feature rows e of the group's 32 block sums), as the 16x16x32 MFMA reads
// it: rows of 80 bytes (64 + 16 of padding, so that the 16-byte reads of 16 consecutive
// rows hit 16 distinct chunk positions), and chunk c of a row holding blocks 4c .. 4c + 3
// and 16 + 4c .. 16 + 4c + 3: the 8 k-slots a lane of group c feeds to one MFMA, in the
// order its P-bar operand holds them.
constexpr int kVtRow = 80;
__host__ __device__ __forceinline__ constexpr int vt_block_of(int chunk, int i) {
  return ((i & 4) << 2) | (chunk << 2) | (i & 3);
}

// Phase-2 pack image for the D = 128 direct-load kernels, split between their two
// LDS tile buffers: [Hbar^T: 128 rows x 256 B, XOR layout of a K tile] -> K buffer;
// [kbar: 32 rows x 256 B, XOR layout][V^ transposed: 128 rows x kVtRow] -> V buffer.
// Both parts are whole multiples of 4 KB, so the waves of a workgroup (four, or two)
// split their 1 KB direct loads evenly.
template <int BT>
struct K4DPack {
  static constexpr int HT_BYTES = 128 * 256;
  static constexpr int KB_OFF = 0;                       // within the V-buffer part
  static constexpr int VT_OFF = 32 * 256;
  static constexpr int RAW2 = VT_OFF + 128 * kVtRow;
  static constexpr int PART2 = (RAW2 + 4095) / 4096 * 4096;
  static constexpr int BYTES = HT_BYTES + PART2;
  static_assert(HT_BYTES % 4096 == 0, "pack split");
};

// Byte offset of element (row, col) in a 256-byte-row tile whose 16-byte chunk c
// of row r is stored at c ^ (r & 15).
__host__ __device__ __forceinline__ constexpr int xor_tile_byte(int row, int col) {
  return row * 256 + ((((col >> 3) ^ row) & 15) << 4) + (col & 7) * 2;
}

}  // namespace pasa
