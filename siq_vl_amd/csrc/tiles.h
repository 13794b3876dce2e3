// Global -> LDS staging of [rows x D] bf16 tiles and the MFMA operand reads
// from them, shared by the attention kernels.
//
// Staging uses gfx950's direct loads (global_load_lds_dwordx4): each wave
// instruction moves 64 x 16 bytes from global memory straight into 1 KB of
// contiguous LDS (lane l's chunk at byte 16 l), with no VGPRs in between, so
// the next tile can be in flight while the current one is multiplied without
// spending registers on it.
//
// LDS layout: rows are D bf16 long with no padding; within row r the 16-byte
// chunk c is stored at chunk position c ^ swz(r).  Two read patterns must be
// bank-conflict free (64 banks of 4 bytes):
//  * row operand (ds_read_b128): a quarter-wave reads one chunk from each of
//    16 consecutive rows -> swz must be a bijection on (r mod 16) for D = 128
//    (a 256-byte row spans all banks) and on (r mod 2, chunk) for D = 64;
//  * transposed operand (ds_read_b64_tr_b16): half a wave reads the 4 chunks
//    c0 .. c0 + 3 (c0 a multiple of 4) of 4 consecutive rows (first row a
//    multiple of 4) -> the 16 chunk positions must fall in distinct bank groups.
// D = 128: swz(r) = 4 (r mod 4) + (r / 4 mod 4)   (bits 2-3 separate the rows)
// D = 64:  swz(r) = 4 (r / 2 mod 2) + (r / 4 mod 4) (rows alternate bank halves)
#pragma once
#include "common.h"

namespace siq {

typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;
typedef __attribute__((address_space(3))) void lds_void;

template <int D>
__device__ __forceinline__ int swz(int r) {
  static_assert(D == 128 || D == 64, "head dim");
  if (D == 128) return ((r & 3) << 2) | ((r >> 2) & 3);
  return (((r >> 1) & 1) << 2) | ((r >> 2) & 3);
}

__device__ __forceinline__ int wave_uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }

// Direct staging of a ROWS x D tile by the NW waves of a workgroup.  Wave w
// issues instructions w*PERW .. w*PERW + PERW - 1; instruction i covers rows
// [i*RPI, (i+1)*RPI) (1 KB, 64 chunks), lane l taking row i*RPI + l / CH and
// chunk position l % CH.  The swizzle repeats every 16 rows, so a lane only
// keeps PAT = 16 / RPI chunk offsets.  Rows >= nrows load the last valid row
// instead (always in bounds; consumers mask those rows or multiply them by
// exact zeros).
template <int ROWS, int D, int NW>
struct LdsTile {
  static constexpr int CH = D / 8;
  static constexpr int RPI = 64 / CH;          // rows per wave instruction
  static constexpr int NINSTR = ROWS / RPI;
  static constexpr int PERW = NINSTR / NW;
  static constexpr int PAT = 16 / RPI;          // distinct swizzle patterns
  static constexpr int ELEMS = ROWS * D;
  static_assert(NINSTR % NW == 0 && PERW % PAT == 0, "tile splits evenly over the waves");

  uint32_t coff[PAT];  // element offset of this lane's chunk inside its row, for instruction p (p < PAT)
  int lrow;            // row of this lane inside an instruction

  __device__ __forceinline__ void init(int64_t stride, int lane) {
    (void)stride;
    lrow = lane / CH;
    const int pc = lane % CH;
#pragma unroll
    for (int pi = 0; pi < PAT; ++pi) coff[pi] = (uint32_t)(8 * (pc ^ swz<D>(pi * RPI + lrow)));
  }

  // gbase: (row 0, col 0) of the tile in global memory; lds: the tile's LDS
  // base; wu: this wave's index among the NW staging waves (wave-uniform).
  // Offsets are 32-bit element counts from gbase (a tile spans < 2^31 elements).
  //
  // UNTRACKED = true issues the loads through inline asm, hidden from the
  // compiler's wait insertion: it cannot tell the ring slot being filled from
  // the ones being read and would wait for every prefetch before the next LDS
  // read.  The caller then orders them itself (wait_vmcnt, then a barrier).
  template <bool UNTRACKED = false>
  __device__ __forceinline__ void issue(const bf16* gbase, int64_t stride, int nrows, bf16* lds, int wu) const {
#pragma unroll
    for (int k = 0; k < PERW; ++k) issue_one<UNTRACKED>(k, gbase, stride, nrows, lds, wu);
  }

  // Element offsets (from the tile's first row) of this wave's PERW
  // instructions for a whole tile (nrows >= ROWS), computed once so that a
  // loop over whole tiles issues them without address arithmetic.
  __device__ __forceinline__ void full_offsets(int64_t stride, int wu, uint32_t (&o)[PERW]) const {
#pragma unroll
    for (int k = 0; k < PERW; ++k) o[k] = (uint32_t)((wu * PERW + k) * RPI + lrow) * (uint32_t)stride + coff[k % PAT];
  }

  // A whole tile from the offsets of full_offsets, untracked (as issue<true>).
  __device__ __forceinline__ void issue_full(const bf16* gbase, const uint32_t (&o)[PERW], bf16* lds, int wu) const {
#pragma unroll
    for (int k = 0; k < PERW; ++k) {
      const uint32_t la = (uint32_t)(uintptr_t)(lds_void*)(lds + (wu * PERW + k) * 512);
      asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %0, %1" : : "v"(o[k] << 1), "s"(gbase), "{m0}"(la)
                   : "memory");
    }
  }

  // Instruction k (< PERW) of this wave's share, so that a caller can spread
  // its loads between other work.
  template <bool UNTRACKED = false>
  __device__ __forceinline__ void issue_one(int k, const bf16* gbase, int64_t stride, int nrows, bf16* lds,
                                            int wu) const {
    const uint32_t st = (uint32_t)stride;
    const int i = wu * PERW + k;
    int r = i * RPI + lrow;
    if (nrows < ROWS) r = min(r, nrows - 1);
    const uint32_t o = (uint32_t)r * st + coff[k % PAT];
    if constexpr (UNTRACKED) {
      // lane l's 16 bytes land at LDS byte m0 + 16 l.  s_nop 4: m0 needs one wait state after its
      // write, and the base SGPRs may have been written by a VALU instruction (an SGPR written by
      // VALU and read by VMEM needs five), which the compiler's hazard checks do not see in asm.
      const uint32_t la = (uint32_t)(uintptr_t)(lds_void*)(lds + i * 512);
      asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %0, %1" : : "v"(o << 1), "s"(gbase), "{m0}"(la)
                   : "memory");
    } else {
      // uniform base + 32-bit byte offset: the saddr + voffset form
      __builtin_amdgcn_global_load_lds(reinterpret_cast<const char*>(gbase) + (o << 1), (lds_void*)(lds + i * 512),
                                       16, 0, 0);
    }
  }
};

// Row operand reads: lane l reads row (rbase + l % 32), logical chunk
// 2 ks + h (d = 16 ks + 8 h .. +7), for ks = 0 .. D/16 - 1.  The swizzle XORs
// bits below the row offset, so the element offset of chunk 2 ks + h is
// base ^ 16 ks with base = (l % 32) D + 8 (swz(l % 32) ^ h): one register per
// lane (row bases are multiples of 32 rows).
template <int D>
struct RowRead {
  uint32_t base;
  __device__ __forceinline__ void init(int lane) {
    const int l32 = lane & 31, h = lane >> 5;
    base = (uint32_t)(l32 * D + 8 * (swz<D>(l32) ^ h));
  }
  // T: tile base, rb: first row of the 32-row block (multiple of 32)
  __device__ __forceinline__ bf16x8 read(const bf16* T, int rb, int ks) const {
    return ld_bf16x8(T + rb * D + (base ^ (uint32_t)(16 * ks)));
  }
};

// Writes in the staging layout from the MFMA row layout: lane l owns tile row
// rb + l % 32 (rb a multiple of 32) and writes its 16-byte logical chunks c,
// so that whole rows can then be read out 256 bytes at a time (RowSpan).
template <int D>
struct RowWrite {
  uint32_t base;
  int s;
  __device__ __forceinline__ void init(int lane) {
    const int l32 = lane & 31;
    base = (uint32_t)(l32 * D);
    s = swz<D>(l32);
  }
  __device__ __forceinline__ void write(bf16* T, int rb, int c, const bf16x8& v) const {
    st_bf16x8(T + rb * D + base + 8 * (c ^ s), v);
  }
};

// Whole-row access to a staged tile: instruction i of a wave covers tile rows
// rb + RPI i .. rb + RPI i + RPI - 1, lane l taking row rb + RPI i + l / CH and
// logical chunk l % CH, so each instruction reads or writes RPI whole rows of
// global memory (N32 instructions cover the wave's 32 rows).
template <int D>
struct RowSpan {
  static constexpr int CH = D / 8, RPI = 64 / CH, N32 = 32 / RPI;
  int lr, c;
  __device__ __forceinline__ void init(int lane) {
    lr = lane / CH;
    c = lane % CH;
  }
  __device__ __forceinline__ int row(int rb, int i) const { return rb + RPI * i + lr; }
  // element offset of this lane's chunk of tile row r in the staging layout
  __device__ __forceinline__ uint32_t lds(int r) const { return (uint32_t)(r * D + 8 * (c ^ swz<D>(r))); }
};

// Transposed operand reads with ds_read_b64_tr_b16.  Within each 16-lane
// group, lane p = 4j + q supplies the address of row j of a 4 x 16 block
// (8 bytes at column group q) and lane i receives element i % 4 of the chunks
// supplied by lanes 4j + i / 4 (j = 0..3): 4 consecutive rows of one column.
// read(T, k0, dt) returns for lane l the values
//   T[k0 + krow(i, h)][32 dt + perm32(l % 32)],  i = 0..7,
//   krow(i, h) = 4h + i (i < 4), 8 + 4h + (i - 4) (i >= 4),
// which is the row order r -> 8 (r/4) + 4h + (r%4) of an MFMA D tile: P or dS
// taken from accumulators 8j..8j+7 pairs with the read at k0 + 16 j.  The
// column permutation perm32 (chosen per supplying lane) makes the product's
// rows come out as 8 consecutive d per accumulator group.  k0 must be a
// multiple of 16.
template <int D>
struct TrRead {
  // element offset of (row r_e, 32-column block 0) for the lane's two 4-row
  // groups e; the block dt is reached by XOR with 32 dt (the swizzle only
  // touches chunk bits below the row offset)
  uint32_t base[2];
  __device__ __forceinline__ void init(int lane) {
    const int G = lane >> 4, p = lane & 15, j = p >> 2, q = p & 3;
    const int cl = 2 * (G & 1) + (q & 1);  // logical chunk within a 32-column block
    const int wo = 4 * (q >> 1);           // element offset inside the chunk
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int r = 4 * (G >> 1) + j + 8 * e;
      base[e] = (uint32_t)(r * D + 8 * (cl ^ swz<D>(r)) + wo);
    }
  }
  __device__ __forceinline__ bf16x8 read(const bf16* T, int k0, int dt) const {
    const bf16* t = T + k0 * D;
    const bf16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(t + (base[0] ^ (uint32_t)(32 * dt))));
    const bf16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(t + (base[1] ^ (uint32_t)(32 * dt))));
    return bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  }
};

// One dword per lane from gptr straight into LDS (lane l's 4 bytes land at LDS
// byte lds + 4 l), untracked like LdsTile::issue<true>: the caller orders it
// with wait_vmem and a barrier.  s_nop 0: m0 needs one wait state after its
// write; the address is a VGPR pair.
__device__ __forceinline__ void dma4_untracked(const void* gptr, const void* lds) {
  const uint32_t la = (uint32_t)(uintptr_t)(lds_void*)lds;
  asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, off" : : "v"(gptr), "{m0}"(la) : "memory");
}

// Makes a wave-uniform value opaque, so the compiler keeps it in SGPRs rather
// than re-reading it from the kernel arguments on every trip of a loop.
template <typename T>
__device__ __forceinline__ void pin_sgpr(T& x) {
  asm volatile("" : "+s"(x));
}

// Wait for this wave's outstanding global (and direct-to-LDS) loads.
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Wait for this wave's outstanding LDS reads (lgkmcnt(0), vmcnt untouched).
__device__ __forceinline__ void wait_lds() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// Wait until at most N of this wave's global loads are outstanding (loads
// complete in issue order, so everything but the newest N has landed).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (0x7 << 4) | (0xF << 8) | ((N >> 4) << 14));
}

// Per-sequence extents, clamped on the device to [0, total).
struct SeqInfo {
  int q_start, q_len, k_start, k_len;
};

}  // namespace siq
