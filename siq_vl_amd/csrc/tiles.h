// Global -> LDS staging of [rows x D] bf16 tiles for the attention kernels.
//
// A tile is taken from a token-major tensor (one row = one token of one head,
// D contiguous bf16, rows `stride` elements apart).  The unit of work is
// 4 consecutive rows x 8 consecutive columns (four 16-byte global loads held in
// registers), so the same registers can be written to LDS row-major
// ([rows][D+8], 16-byte stores) and/or transposed ([D][rows+8], 8-byte stores
// of 4 rows).  The +8 element padding keeps the MFMA operand reads (16 bytes
// from 16 different rows per quarter-wave) free of bank conflicts.
//
// Lane -> unit mapping:
//  * GFAST = false: the 16-byte column chunk varies fastest, so one load
//    instruction of a wave reads whole 256-byte rows (best coalescing);
//    used for tiles that are only stored row-major.
//  * GFAST = true: the 4-row group varies fastest, which makes the transposed
//    8-byte LDS stores conflict-free; used for tiles stored transposed.
#pragma once
#include "common.h"

namespace siq {

template <int ROWS, int D, int NT, bool GFAST>
struct Tile4x8 {
  static constexpr int CH = D / 8;     // 16-byte chunks per row
  static constexpr int G = ROWS / 4;   // 4-row groups
  static constexpr int UNITS = CH * G;
  static constexpr int PER = (UNITS + NT - 1) / NT;
  static constexpr int RS = D + 8;     // row-major LDS stride (elements)
  static constexpr int TS = ROWS + 8;  // transposed LDS stride (elements)
  static_assert(ROWS % 4 == 0 && D % 8 == 0, "tile shape");

  u32x4 v[PER][4];

  __device__ __forceinline__ static void unit(int u, int& c, int& g) {
    if (GFAST) {
      g = u % G;
      c = u / G;
    } else {
      c = u % CH;
      g = u / CH;
    }
  }
  __device__ __forceinline__ static bool live(int u) { return (UNITS % NT == 0) || u < UNITS; }

  // base: element (row 0, col 0) of the tile; rows >= nrows are filled with zeros
  // and never touched in global memory.
  __device__ __forceinline__ void load(const bf16* base, int64_t stride, int nrows, int tid) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int u = tid + i * NT;
      if (!live(u)) continue;
      int c, g;
      unit(u, c, g);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int row = 4 * g + j;
        if (row < nrows) {
          v[i][j] = *reinterpret_cast<const u32x4*>(base + (int64_t)row * stride + 8 * c);
        } else {
          v[i][j] = u32x4{0u, 0u, 0u, 0u};
        }
      }
    }
  }

  __device__ __forceinline__ void store_rows(bf16* s, int tid) const {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int u = tid + i * NT;
      if (!live(u)) continue;
      int c, g;
      unit(u, c, g);
#pragma unroll
      for (int j = 0; j < 4; ++j) *reinterpret_cast<u32x4*>(s + (4 * g + j) * RS + 8 * c) = v[i][j];
    }
  }

  __device__ __forceinline__ void store_cols(bf16* s, int tid) const {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int u = tid + i * NT;
      if (!live(u)) continue;
      int c, g;
      unit(u, c, g);
      u32x2 cols[8];
      transpose4x8(v[i], cols);
#pragma unroll
      for (int j = 0; j < 8; ++j) *reinterpret_cast<u32x2*>(s + (8 * c + j) * TS + 4 * g) = cols[j];
    }
  }
};

// Per-sequence extents, clamped on the device to [0, total): x = q start,
// y = q length, z = k start, w = k length.
struct SeqInfo {
  int q_start, q_len, k_start, k_len;
};

}  // namespace siq
