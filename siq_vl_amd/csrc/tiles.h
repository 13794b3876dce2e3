// Global -> LDS staging of [rows x D] bf16 tiles and the transposed LDS
// operand read, shared by the attention kernels.
//
// Tiles are always stored row-major in LDS and never transposed in registers:
// an MFMA operand that needs k along the tile rows (V^T, K^T, Q^T, dO^T) is
// read with ds_read_b64_tr_b16 (gfx950).
//
// Row padding (kRowPad): a quarter-wave reads 16 B from each of 16 rows for
// the row-major operand, and 32 B from each of 4 consecutive rows for the
// transposed one.  With 64 four-byte banks both are conflict-free when the row
// stride is 12 dwords mod 64 (D = 128: 64 + 12) or 52 (D = 64: 32 + 20):
// 16 rows land on 16 distinct 4-bank groups and 4 rows on 4 disjoint 8-bank
// spans.
#pragma once
#include "common.h"

namespace siq {

typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;

template <int D>
struct RowPad;
template <>
struct RowPad<128> {
  static constexpr int value = 24;  // elements: 12 dwords
};
template <>
struct RowPad<64> {
  static constexpr int value = 40;  // elements: 20 dwords
};

// Row-major staging.  One unit = one 16-byte chunk; consecutive lanes take
// consecutive chunks of a row, so a wave's load instruction reads whole rows.
// Each thread keeps the 32-bit element offset of its chunks (fixed for the
// whole kernel); full tiles load with uniform base + offset, tail tiles read
// the last valid row instead of rows past the end (always in bounds) and
// replace them by zeros with a select, so no load is predicated.
template <int ROWS, int D, int NT>
struct RowTile {
  static constexpr int CH = D / 8;
  static constexpr int UNITS = ROWS * CH;
  static constexpr int PER = (UNITS + NT - 1) / NT;
  static constexpr int RS = D + RowPad<D>::value;
  static_assert(UNITS % NT == 0, "every thread stages the same number of chunks");

  u32x4 v[PER];
  uint32_t off[PER];  // element offset of chunk i inside the tile
  int row[PER];

  __device__ __forceinline__ void init(int64_t stride, int tid) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int u = tid + i * NT;
      const int c = u % CH, r = u / CH;
      row[i] = r;
      off[i] = (uint32_t)(r * stride + 8 * c);
    }
  }

  // base: (row 0, col 0) of the tile in global memory; rows >= nrows become 0.
  __device__ __forceinline__ void load(const bf16* base, int64_t stride, int nrows) {
    if (nrows >= ROWS) {
#pragma unroll
      for (int i = 0; i < PER; ++i) v[i] = *reinterpret_cast<const u32x4*>(base + off[i]);
      return;
    }
    if (nrows <= 0) {
#pragma unroll
      for (int i = 0; i < PER; ++i) v[i] = u32x4{0u, 0u, 0u, 0u};
      return;
    }
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int r = row[i];
      const uint32_t o = r < nrows ? off[i] : off[i] - (uint32_t)((r - nrows + 1) * stride);
      const u32x4 x = *reinterpret_cast<const u32x4*>(base + o);
      v[i] = r < nrows ? x : u32x4{0u, 0u, 0u, 0u};
    }
  }

  __device__ __forceinline__ void store(bf16* s, int tid) const {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int u = tid + i * NT;
      const int c = u % CH, r = u / CH;
      *reinterpret_cast<u32x4*>(s + r * RS + 8 * c) = v[i];
    }
  }
};

// Transposed MFMA operand from a row-major LDS tile T[k][m] (row stride rs).
// ds_read_b64_tr_b16: within each 16-lane group, lane p = 4j + q supplies the
// address of row j of a 4 x 16 block (8 bytes at column group q) and lane i
// receives element i % 4 of the chunks supplied by lanes 4j + i / 4, j = 0..3,
// i.e. 4 consecutive rows of one column.  Two reads give 8 k values.
//
// TrRead precomputes the lane-dependent part once.  read(T, k0, m0) returns for
// lane l the values T[k0 + krow(i, h)][m0 + perm32(l % 32)], i = 0..7, with
//   krow(i, h) = 4h + i        (i < 4),   8 + 4h + (i - 4)   (i >= 4),
// which is exactly the row order r -> 8*(r/4) + 4h + (r%4) of an MFMA D tile:
// P or dS taken from accumulators 8j..8j+7 pairs with the tr read at k0 + 16j.
// The column permutation perm32 (chosen per supplying lane) makes the product's
// rows come out as 8 consecutive m per accumulator group.
struct TrRead {
  int base;  // element offset of this lane's first supplied address
  __device__ __forceinline__ void init(int rs, int lane) {
    const int G = lane >> 4, p = lane & 15, j = p >> 2, q = p & 3;
    const int col = 16 * (G & 1) + 8 * (q & 1) + 4 * (q >> 1);
    base = (4 * (G >> 1) + j) * rs + col;
  }
  __device__ __forceinline__ bf16x8 read(const bf16* T, int rs, int k0, int m0) const {
    const bf16* a = T + base + k0 * rs + m0;
    const bf16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)a);
    const bf16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(a + 8 * rs));
    return bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  }
};

// Natural (unpermuted) D-tile row of accumulator r in lane half h.
__device__ __forceinline__ constexpr int nrow(int r, int h) { return 8 * (r >> 2) + 4 * h + (r & 3); }

// Per-sequence extents, clamped on the device to [0, total).
struct SeqInfo {
  int q_start, q_len, k_start, k_len;
};

}  // namespace siq
