// LDS tile layout shared by the prefill and split-K kernels.
#pragma once

#include "fa_device.hpp"

namespace fa {

// K and V tiles are [BN rows][D] 16-bit elements with no padding; 16-byte chunks
// are XOR-swizzled per row so that every read pattern hits all 64 LDS banks once,
// and so that direct global->LDS loads (which write 64 lanes x 16 B contiguously)
// can fill a tile.  Physical chunk = logical chunk ^ swizzle(row).
//
// A chunk's bank group (16 bytes = 4 of the 64 banks) is its physical index mod 16,
// since rows are multiples of 256 bytes at D >= 128; at D = 64, 32 and 16 a 256-byte line
// holds 2, 4 and 8 rows.  At D = 256 a row is two bank
// lines; the XOR values stay below 16, so they keep a chunk's high bit and give the
// same bank pattern as at D = 128.
template <int D, int BN>
struct TileShape {
  static constexpr int CPR = D / 8;                         // 16-byte chunks per row
  static constexpr int ROWS_PER_256B = D >= 128 ? 1 : 128 / D;  // rows sharing one 256-byte bank line
  static constexpr int TILE = BN * D;                       // elements per K (or V) tile
  static constexpr int STAGE = 2 * TILE;                    // K then V
  // K rows are read 16 at a time at one logical chunk: map them to 16 distinct bank groups.
  __device__ static constexpr int swz_k(int row) { return (row / ROWS_PER_256B) % (CPR < 16 ? CPR : 16); }
  // V is read transposed: 4 consecutive rows (starting at a multiple of 4) x 4 chunks
  // (starting at a multiple of 4) per 32 lanes.  At D = 32 those are 4 whole 64-byte rows,
  // one 256-byte bank line, so no swizzle is needed.
  __device__ static constexpr int swz_v(int row) {
    return D >= 128 ? 4 * (row & 3) + ((row >> 2) & 3) : (D == 64 ? 4 * ((row >> 1) & 1) : 0);
  }
};

// LDS row r of a K tile holds key kperm(r) (bits 2 and 3 swapped): the S^T
// A-operand then reads consecutive rows yet receives the key order whose C
// fragment hands each lane 8 contiguous keys per 16-key step.
__device__ __forceinline__ constexpr int kperm(int r) { return (r & ~0xC) | ((r & 4) << 1) | ((r & 8) >> 1); }

}  // namespace fa

namespace fa {

// FP8 K/V tiles: [BN rows][D bytes], raw e4m3fn as loaded, 16-byte chunks
// XOR-swizzled per row.  64 banks x 4 bytes = 256 bytes hold 256 / D rows.
template <int D, int BN>
struct TileShape8 {
  static constexpr int CPR = D / 16;             // 16-byte chunks per row
  static constexpr int ROWS_PER_256B = 256 / D;  // rows sharing one 256-byte bank line
  static constexpr int TILE = BN * D;            // bytes per K (or V) tile
  // K is read 8 bytes per lane, 32 rows at one logical chunk: rows of one bank line
  // position get distinct chunks (two lanes share a bank pair at most).
  __device__ static constexpr int swz_k(int row) { return (row / ROWS_PER_256B) % CPR; }
  // V is read with ds_read_b64_tr_b8: 8 consecutive rows at one chunk per 16 lanes,
  // the chunk's parity differing between the two 16-lane halves of 32 lanes.  Even
  // XOR values keep the parities apart and spread the 8 rows over distinct banks.
  __device__ static constexpr int swz_v(int row) { return 2 * ((row / ROWS_PER_256B) % (CPR / 2)); }
};

}  // namespace fa
