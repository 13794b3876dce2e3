// Tiled bf16 GEMM core for gfx950 shared by the fused CE and the projector:
// C[i][j] = sum_k A[i][k] B[j][k] over 256 x 256 tiles, 8 waves, k-steps of
// 64 staged in LDS by direct global->LDS loads (two slabs in flight), operand
// reads with ds_read_b128 / ds_read_b64_tr_b16, v_mfma_f32_32x32x16_bf16.
#pragma once
#include "common.h"

namespace siq {
namespace gemm {

constexpr int BI = 256, BJ = 256, BK = 64, NT = 512;
constexpr int NW = NT / 64;         // 8 waves: 2 along I (128 rows each) x 4 along J (64 cols each)
constexpr int SLAB = 256 * BK;      // bf16 elements of one staged operand slab (32 KB)
constexpr int kXcds = 8;

typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;

struct GOp {
  const bf16* base;
  int64_t ld, rows, cols;  // element (r, c) at base[r * ld + c]; 16-byte chunks along c
};

// Operand slabs live in LDS in one of two orientations, both XOR-swizzled at
// 16-byte granularity so the MFMA operand reads are bank-conflict free (64
// banks of 4 bytes):
//  * KC ("k contiguous"): [256 rows][64 k], 128-byte rows; the slab's rows are
//    the operand's M (or N) index.  Read as row operands (one chunk from each
//    of 16 consecutive rows per quarter-wave): swz_kc spreads 16 rows over
//    distinct (bank half, chunk) pairs.
//  * NKC: [64 k][256 cols], 512-byte rows; the slab's columns are the operand's
//    M (or N) index.  Read with ds_read_b64_tr_b16 (4 aligned chunks from each
//    of 4 consecutive rows per half-wave): swz_nkc XORs the row into bits 2-3
//    of the chunk index, so the 16 positions land in 16 distinct bank groups.
__device__ __forceinline__ int swz_kc(int r) { return (((r >> 1) & 3) << 1) | ((r >> 3) & 1); }
__device__ __forceinline__ int swz_nkc(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }

// One wave instruction of direct global->LDS loading: lane l's 16 bytes land
// at LDS byte lds + 16 l.  Written as inline asm so that the compiler's wait
// insertion does not track these loads: it cannot tell the slab being read
// from the one being loaded (both live in one LDS array) and would wait for
// the prefetch before the first transposed read of every step.  The GEMM loop
// orders them with the LDS reads itself (wait_vmem, then a barrier).  The LDS
// address goes in m0 (one wait state after its write) and the uniform base in
// SGPRs, which the compiler may have just written from a VALU instruction
// (v_readfirstlane; an SGPR written by VALU and read by VMEM needs five wait
// states): its hazard checks do not look inside the asm, so it starts with
// s_nop 4.
__device__ __forceinline__ void dma16(const bf16* gbase, uint32_t elem_off, const bf16* lds) {
  const uint32_t la = (uint32_t)(uintptr_t)(lds_void*)lds;
  const uint32_t byte_off = elem_off << 1;
  asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %0, %1" : : "v"(byte_off), "s"(gbase), "{m0}"(la)
               : "memory");
}
__device__ __forceinline__ void dma16(const bf16* gptr, const bf16* lds) {
  const uint32_t la = (uint32_t)(uintptr_t)(lds_void*)lds;
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(gptr), "{m0}"(la) : "memory");
}

// Direct global->LDS staging of one slab: 32 instructions of 1 KB, 8 per wave.
// Rows / chunks past the operand's extent re-read the last valid one (always in
// bounds); the garbage that produces is either never stored (M/N tails) or
// multiplied by rows the B-operand pass zeroes (K tails).
template <bool KC>
struct SlabLoad {
  static constexpr int PERW = 32 / NW;  // instructions per wave (32 per slab)
  int lrow, lpc;  // this lane's row inside an instruction and physical chunk
  int wrow;       // first slab row of this wave's instructions
  uint32_t off0, off1;  // KC: element offsets of instructions k = 0, 1 (k + 2 adds 16 rows)
  __device__ __forceinline__ void init(const GOp& op, int lane, int w) {
    if (KC) {
      lrow = lane / 8;
      lpc = lane % 8;
      wrow = 8 * PERW * w;   // instruction i = PERW w + k covers rows 8i .. 8i + 7
      const int r0 = wrow + lrow, r1 = wrow + 8 + lrow;
      off0 = (uint32_t)(r0 * op.ld + 8 * (lpc ^ swz_kc(r0)));
      off1 = (uint32_t)(r1 * op.ld + 8 * (lpc ^ swz_kc(r1)));
    } else {
      lrow = lane / 32;
      lpc = lane % 32;
      wrow = 2 * PERW * w;   // instruction i = PERW w + k covers rows 2i, 2i + 1
      off0 = off1 = 0;
    }
  }
  // r0: first M/N index of the tile, k0: first k of the slab
  __device__ __forceinline__ void issue(const GOp& op, int64_t r0, int64_t k0, bf16* lds, int wu) const {
    const bool full = KC ? (r0 + 256 <= op.rows && k0 + BK <= op.cols) : (k0 + BK <= op.rows && r0 + 256 <= op.cols);
    if (full) {
      // uniform slab base + 32-bit per-lane offsets (every offset < 2^31: rows < 256 x ld or k < 64 x ld)
      const bf16* base = KC ? op.base + r0 * op.ld + k0 : op.base + k0 * op.ld + r0;
#pragma unroll
      for (int k = 0; k < PERW; ++k) {
        uint32_t o;
        if (KC) {
          o = ((k & 1) ? off1 : off0) + (uint32_t)(16 * (k >> 1) * op.ld);
        } else {
          const int r = wrow + 2 * k + lrow;
          o = (uint32_t)(r * op.ld + 8 * (lpc ^ swz_nkc(r)));
        }
        dma16(base, o, lds + (wu * PERW + k) * 512);
      }
      return;
    }
    // a uniform base at the slab's first row / chunk and 32-bit offsets
    // clamped to its last valid row / chunk, as in the full case (no per-lane
    // 64-bit addresses).  A slab that starts outside the operand (a tile wholly
    // past its M / N extent; k-steps always start inside) is not loaded: its
    // products only reach outputs that are never stored.
    const int64_t fr = KC ? r0 : k0, fc = KC ? k0 : r0;
    if (fr >= op.rows || fc + 8 > op.cols) return;
    const bf16* base = op.base + fr * op.ld + fc;
    const int rmax = (int)min(op.rows - 1 - fr, (int64_t)255), cmax = (int)min(op.cols - 8 - fc, (int64_t)248);
#pragma unroll
    for (int k = 0; k < PERW; ++k) {
      const int r = KC ? wrow + 8 * k + lrow : wrow + 2 * k + lrow;
      const int c = KC ? (lpc ^ swz_kc(r)) : (lpc ^ swz_nkc(r));
      const int gr = min(r, rmax), gc = min(8 * c, cmax);
      dma16(base, (uint32_t)(gr * (int)op.ld + gc), lds + (wu * PERW + k) * 512);
    }
  }
};

// MFMA operand reads of the wave's block of NTL 32-row tiles of a slab,
// starting at slab row (KC) / column (NKC) `base`: returns for lane l the 8 k
// values (16 ks + 8 h + i, i = 0..7) of operand row base + 32 t +
// rowmap(l % 32), with rowmap = perm32 when PERM (A operands: the product's
// rows then come out as 8 consecutive indices per accumulator group) and the
// identity otherwise (B operands).
template <bool KC, bool PERM, int NTL>
struct SlabRead {
  uint32_t off[4][2];  // KC: [ks][-]; NKC: [t][e]
  int rowb;
  __device__ __forceinline__ void init(int lane, int base) {
    const int l32 = lane & 31, h = lane >> 5;
    if (KC) {
      const int r = base + (PERM ? perm32(l32) : l32);
      const int f = swz_kc(r);
      rowb = r * BK;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) off[ks][0] = (uint32_t)(rowb + (((2 * ks + h) ^ f) << 3));
    } else {
      const int G = lane >> 4, p = lane & 15, j = p >> 2, q = p & 3;
      const int cs = PERM ? 16 * (G & 1) + 8 * (q & 1) + 4 * (q >> 1) : 16 * (G & 1) + 4 * q;
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int r = 8 * (G >> 1) + j + 4 * e;  // row within a 16-row k group
        const int f = swz_nkc(r);
#pragma unroll
        for (int t = 0; t < NTL; ++t) {
          const int col = base + 32 * t + cs;
          off[t][e] = (uint32_t)(r * 256 + ((((col >> 3) & 15) ^ f) << 3) + ((col >> 7) << 7) + (col & 7));
        }
      }
    }
  }
  __device__ __forceinline__ bf16x8 read(const bf16* S, int t, int ks) const {
    if (KC) return ld_bf16x8(S + off[ks][0] + t * 32 * BK);
    const bf16* base = S + ks * 16 * 256;
    const bf16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(base + off[t][0]));
    const bf16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(base + off[t][1]));
    return bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  }
};

__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Zeroes the K tail of a B slab (k >= kval) after it lands, for the last,
// partial k-step: the slab loader fills those rows / chunks by re-reading the
// last valid one, and the product must not see them.  KC [256][64]: thread t
// owns row t / 2, logical chunks 4 (t % 2) .. +3; NKC [64][256]: row t / 8,
// chunks 4 (t % 8) .. +3.
template <bool KC>
__device__ __forceinline__ void ztail_pass(bf16* S, int kval, int tid) {
  const int r = KC ? tid >> 1 : tid >> 3;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int c = KC ? 4 * (tid & 1) + k : 4 * (tid & 7) + k;
    const int pc = KC ? (c ^ swz_kc(r)) : (c ^ swz_nkc(r));
    bf16* ptr = S + (KC ? r * BK : r * 256) + pc * 8;
    if (KC) {
      if (8 * c + 8 > kval) {
        bf16x8 x = ld_bf16x8(ptr);
#pragma unroll
        for (int i = 0; i < 8; ++i) x[i] = 8 * c + i < kval ? x[i] : (bf16)0.f;
        st_bf16x8(ptr, x);
      }
    } else if (r >= kval) {
      st_bf16x8(ptr, zero_bf16x8());
    }
  }
}

// Maps a 1-D block id onto (I tile, J tile).  Block b is dispatched to XCD
// b % 8, so each XCD gets a contiguous run of the linear tile order; inside it
// tiles go in groups of GI I-tiles (I fastest), so the 32 workgroups running
// together on an XCD cover about GI I-tiles x 32/GI J-tiles and both operands'
// slabs are shared through that XCD's L2.
__device__ __forceinline__ bool tile_of(int nI, int nJ, int GI, int& ti, int& tj) {
  const int total = nI * nJ;
  const int per = (total + kXcds - 1) / kXcds;
  const int lin = (int)(blockIdx.x % kXcds) * per + (int)(blockIdx.x / kXcds);
  if (lin >= total) return false;
  const int g = lin / (GI * nJ), within = lin - g * GI * nJ;
  const int gsize = min(GI, nI - g * GI);
  ti = g * GI + within % gsize;
  tj = within / gsize;
  return true;
}

// C[i][j] = sum_k A[i][k] B[j][k] over k in [kb, ke) (kb, ke multiples of BK
// except ke at the operand's end) with 8 waves of 128x64 (4x2 MFMA 32x32
// tiles; two waves per SIMD).  acc[ti][tj][r] holds
// i = i0 + 128*wi + 32*ti + drow(r, h), j = j0 + 64*wj + 32*tj + l32.  A
// last k-step that ends past ke has its B slab's tail zeroed (ztail_pass).
//
// LA / LB load the A / B slab of the k-step starting at k0 into an LDS slab:
// issue(k0, lds, wu), every row / chunk in bounds (OpLoad below for a
// row-major operand; gathering loaders work the same way).
//
// PF: the operand fragments of each k-step are read two 16-wide k-slices
// ahead of the products that use them (the reads of slice ks + 2 go out right
// after the products of ks), with scheduling groups pinning that order (the
// compiler otherwise pulls every read next to its first use and waits on it).
// It pays where both operands are k-contiguous (six 16-byte reads per slice);
// with a transposed operand (ten or twelve reads per slice, more than the LDS
// counter holds two slices of) the plain order is faster.
template <bool AKC, bool BKC, class LA, class LB, bool PF = false>
__device__ __forceinline__ void gemm_core_l(bf16* smem, const LA& la, const LB& lb, int64_t kb, int64_t ke,
                                            f32x16 (&acc)[4][2]) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wi = w & 1, wj = w >> 1;
  const int wu = __builtin_amdgcn_readfirstlane(w);
  SlabRead<AKC, true, 4> ra;
  SlabRead<BKC, false, 2> rb;
  ra.init(lane, 128 * wi);
  rb.init(lane, 64 * wj);
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) acc[a][b] = zero16();
  const int nk = ke > kb ? (int)((ke - kb + BK - 1) / BK) : 0;
  if (nk > 0) {
    la.issue(kb, smem, wu);
    lb.issue(kb, smem + SLAB, wu);
  }
  wait_vmem();
  __syncthreads();
  // the B slab of k-step s, once landed: zero its tail if the step ends past ke
  auto ztail = [&](int s, bf16* Bslab) {
    const int64_t k0 = kb + (int64_t)s * BK;
    if (k0 + BK > ke) {
      ztail_pass<BKC>(Bslab, (int)(ke - k0), tid);
      __syncthreads();
    }
  };
  if (nk > 0) ztail(0, smem + SLAB);
  for (int it = 0; it < nk; ++it) {
    const bf16* As = smem + (it & 1) * 2 * SLAB;
    const bf16* Bs = As + SLAB;
    const bool more = it + 1 < nk;
    bf16* nx = smem + ((it + 1) & 1) * 2 * SLAB;
    const int64_t kn = kb + (int64_t)(it + 1) * BK;
    if (more) {
      la.issue(kn, nx, wu);
      lb.issue(kn, nx + SLAB, wu);
    }
    if constexpr (PF) {
      constexpr int KS = BK / 16;
      constexpr int R = (AKC ? 4 : 8) + (BKC ? 2 : 4);  // LDS read instructions per slice
      bf16x8 af[KS][4], bfr[KS][2];
      auto fetch = [&](int ks) {
#pragma unroll
        for (int t = 0; t < 4; ++t) af[ks][t] = ra.read(As, t, ks);
#pragma unroll
        for (int t = 0; t < 2; ++t) bfr[ks][t] = rb.read(Bs, t, ks);
      };
      fetch(0);
      fetch(1);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
          for (int b = 0; b < 2; ++b) acc[a][b] = mfma32(af[ks][a], bfr[ks][b], acc[a][b]);
        if (ks + 2 < KS) fetch(ks + 2);
      }
      // groups (mask 0x100: LDS reads, 0x008: MFMA): reads of slices 0, 1; products of 0; reads of 2; ...
      __builtin_amdgcn_sched_group_barrier(0x100, 2 * R, 0);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
        if (ks + 2 < KS) __builtin_amdgcn_sched_group_barrier(0x100, R, 0);
      }
    } else {
#pragma unroll
      for (int ks = 0; ks < BK / 16; ++ks) {
        bf16x8 af[4], bfr[2];
#pragma unroll
        for (int t = 0; t < 4; ++t) af[t] = ra.read(As, t, ks);
#pragma unroll
        for (int t = 0; t < 2; ++t) bfr[t] = rb.read(Bs, t, ks);
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
          for (int b = 0; b < 2; ++b) acc[a][b] = mfma32(af[a], bfr[b], acc[a][b]);
      }
    }
    wait_vmem();
    __syncthreads();
    if (more) ztail(it + 1, nx + SLAB);
  }
}

// A row-major operand (GOp) whose slabs start at M / N index r0.
template <bool KC>
struct OpLoad {
  SlabLoad<KC> sl;
  GOp op;
  int64_t r0;
  __device__ __forceinline__ void init(const GOp& o, int64_t first, int lane, int w) {
    op = o;
    r0 = first;
    sl.init(o, lane, w);
  }
  __device__ __forceinline__ void issue(int64_t k0, bf16* lds, int wu) const { sl.issue(op, r0, k0, lds, wu); }
};

// gemm_core_l over two row-major operands, tile (i0, j0).
template <bool AKC, bool BKC, bool PF = false>
__device__ __forceinline__ void gemm_core(bf16* smem, const GOp& A, const GOp& B, int64_t i0, int64_t j0, int64_t kb,
                                          int64_t ke, f32x16 (&acc)[4][2]) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  OpLoad<AKC> la;
  OpLoad<BKC> lb;
  la.init(A, i0, lane, w);
  lb.init(B, j0, lane, w);
  gemm_core_l<AKC, BKC, OpLoad<AKC>, OpLoad<BKC>, PF>(smem, la, lb, kb, ke, acc);
}

}  // namespace gemm
}  // namespace siq
