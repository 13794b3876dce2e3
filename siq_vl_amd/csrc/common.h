// Shared device helpers for the SiQ-VL hot-path kernels (gfx950 / CDNA4).
//
// Conventions used by every kernel in this directory:
//  * wavefront = 64 lanes; MFMA = v_mfma_f32_32x32x16_bf16 (A 32x16, B 16x32,
//    D 32x32 fp32).  For that instruction lane l supplies row (l % 32) of A /
//    column (l % 32) of B and the 8 bf16 of "k-slot group" h = l / 32.  The
//    hardware pairs A and B by (h, register) slot, so the numbering of k inside
//    one instruction is a free choice as long as both operands use the same one.
//  * D layout: lane l, accumulator element r (0..15) holds
//        row = 8*(r/4) + 4*(l/32) + (r%4),  col = l % 32.
//    Loading A-operand row m from source row perm32(m) (bits 2 and 3 swapped)
//    turns that into  row' = 16*(r/8) + 8*(l/32) + (r%8): the 8 accumulators
//    r = 8j..8j+7 of a lane are 8 *consecutive* source rows.  That is what lets
//    a D tile be fed straight back as the B operand of the next MFMA (k-slot
//    (h, i) <-> row 16j + 8h + i) and lets outputs leave as 16-byte stores.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace siq {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr int kWave = 64;

__device__ __forceinline__ f32x16 mfma32(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

// Row permutation applied to A-operand rows (see header comment).
__device__ __forceinline__ int perm32(int m) {
  return (m & ~12) | ((m & 4) << 1) | ((m & 8) >> 1);
}

// Row (within a 32-row MFMA tile) that accumulator r of this lane refers to,
// when the A operand was loaded through perm32.
__device__ __forceinline__ int drow(int r, int h) { return 16 * (r >> 3) + 8 * h + (r & 7); }

__device__ __forceinline__ float exp2f_fast(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ bf16x8 zero_bf16x8() {
  u32x4 z = {0u, 0u, 0u, 0u};
  return __builtin_bit_cast(bf16x8, z);
}

// Pack 8 fp32 (accumulators base..base+7 of an f32x16) into bf16 (RNE).
__device__ __forceinline__ bf16x8 pack8(const f32x16& v, int base) {
  bf16x8 r;
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = (bf16)v[base + i];
  return r;
}

__device__ __forceinline__ bf16x8 ld_bf16x8(const bf16* p) { return *reinterpret_cast<const bf16x8*>(p); }
__device__ __forceinline__ void st_bf16x8(bf16* p, const bf16x8& v) { *reinterpret_cast<bf16x8*>(p) = v; }

// 4 rows x 8 bf16 (each row a u32x4) -> 8 columns x 4 bf16 (u32x2 each):
// out[j] = {r0[j], r1[j], r2[j], r3[j]}.
__device__ __forceinline__ void transpose4x8(const u32x4 (&rows)[4], u32x2 (&cols)[8]) {
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const uint32_t a0 = rows[0][w], a1 = rows[1][w], a2 = rows[2][w], a3 = rows[3][w];
    cols[2 * w][0] = __builtin_amdgcn_perm(a1, a0, 0x05040100u);
    cols[2 * w][1] = __builtin_amdgcn_perm(a3, a2, 0x05040100u);
    cols[2 * w + 1][0] = __builtin_amdgcn_perm(a1, a0, 0x07060302u);
    cols[2 * w + 1][1] = __builtin_amdgcn_perm(a3, a2, 0x07060302u);
  }
}

// fp32 -> nearest-even bf16 -> fp32.  Used where a result must repeat a bf16
// torch op's rounding exactly.  The empty asm makes x opaque: the compiler
// otherwise treats (float)(bf16)(a * b) of two bf16 values as a bf16 multiply
// that it may fuse, unrounded, into a following add (v_fmac_f32).  The
// conversion itself is gfx950's v_cvt_pk_bf16_f32 (round to nearest even, as
// torch rounds).
__device__ __forceinline__ float rbf(float x) {
  asm("" : "+v"(x));
  return (float)(bf16)x;
}

// Rotary embedding of one 8-element chunk pair (x1 at d, x2 at d + D/2), as
// transformers' apply_rotary_pos_emb evaluates it on bf16 tensors
// (modeling_qwen2.py:105-135: q * cos + rotate_half(q) * sin, each op rounded):
//   o1 = rb(rb(x1 c1) + rb(-x2 s1)),  o2 = rb(rb(x2 c2) + rb(x1 s2)).
__device__ __forceinline__ void rope_fwd8(const bf16x8& x1, const bf16x8& x2, const bf16x8& c1, const bf16x8& c2,
                                          const bf16x8& s1, const bf16x8& s2, bf16x8& o1, bf16x8& o2) {
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const float u = (float)x1[k], v = (float)x2[k];
    o1[k] = (bf16)(rbf(u * (float)c1[k]) + rbf(-v * (float)s1[k]));
    o2[k] = (bf16)(rbf(v * (float)c2[k]) + rbf(u * (float)s2[k]));
  }
}

// Its autograd backward on the bf16 upstream gradients g1 (at d), g2 (at d + D/2):
//   dx1 = rb(rb(g1 c1) + rb(g2 s2)),  dx2 = rb(rb(g2 c2) - rb(g1 s1)).
__device__ __forceinline__ void rope_bwd8(const bf16x8& g1, const bf16x8& g2, const bf16x8& c1, const bf16x8& c2,
                                          const bf16x8& s1, const bf16x8& s2, bf16x8& o1, bf16x8& o2) {
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const float u = (float)g1[k], v = (float)g2[k];
    o1[k] = (bf16)(rbf(u * (float)c1[k]) + rbf(v * (float)s2[k]));
    o2[k] = (bf16)(rbf(v * (float)c2[k]) - rbf(u * (float)s1[k]));
  }
}

// The same rotation with fp32 cos / sin rows (bf16 q / k under bf16 autocast
// over fp32 master weights, where transformers' rotary embedding hands over
// fp32 cos / sin): torch promotes every product and the sum to fp32, and the
// attention's cast to bf16 rounds once at the end:
//   o1 = rb(fl(fl(x1 c1) - fl(x2 s1))),  o2 = rb(fl(fl(x2 c2) + fl(x1 s2))),
// with fl = fp32 rounding (no fused multiply-add: each product is made opaque
// before the add).
__device__ __forceinline__ float opq(float x) {
  asm("" : "+v"(x));
  return x;
}
__device__ __forceinline__ void rope_fwd8_f32(const bf16x8& x1, const bf16x8& x2, const float (&c1)[8],
                                              const float (&c2)[8], const float (&s1)[8], const float (&s2)[8],
                                              bf16x8& o1, bf16x8& o2) {
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const float u = (float)x1[k], v = (float)x2[k];
    o1[k] = (bf16)(opq(u * c1[k]) - opq(v * s1[k]));
    o2[k] = (bf16)(opq(v * c2[k]) + opq(u * s2[k]));
  }
}

// Its autograd backward: each product's gradient is formed in fp32 and cast
// to the bf16 input's dtype, and the two contributions to x are added in bf16:
//   dx1 = rb(rb(fl(g1 c1)) + rb(fl(g2 s2))),  dx2 = rb(rb(fl(g2 c2)) - rb(fl(g1 s1))).
__device__ __forceinline__ void rope_bwd8_f32(const bf16x8& g1, const bf16x8& g2, const float (&c1)[8],
                                              const float (&c2)[8], const float (&s1)[8], const float (&s2)[8],
                                              bf16x8& o1, bf16x8& o2) {
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const float u = (float)g1[k], v = (float)g2[k];
    o1[k] = (bf16)(rbf(u * c1[k]) + rbf(v * s2[k]));
    o2[k] = (bf16)(rbf(v * c2[k]) - rbf(u * s1[k]));
  }
}

__device__ __forceinline__ float wave_max_xor32(float x) { return fmaxf(x, __shfl_xor(x, 32)); }
__device__ __forceinline__ float wave_sum_xor32(float x) { return x + __shfl_xor(x, 32); }

// The same two reductions with gfx950's v_permlane32_swap (a VALU exchange of
// the wave's halves, no LDS round trip).  Every lane of the wave must be
// active.  r[0] holds x of lanes 0..31 in both halves, r[1] x of lanes 32..63,
// so both halves get bitwise the same result.
__device__ __forceinline__ float half_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __builtin_amdgcn_fmed3f(__uint_as_float(r[0]), __uint_as_float(r[1]), INFINITY);
}
__device__ __forceinline__ float half_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Sum of the 8 bf16 of v plus acc, two per v_dot2c_f32_bf16 (products with 1
// are exact; fp32 accumulation).
__device__ __forceinline__ float sum8_bf16(const bf16x8& v, float acc) {
  const bf16x2 one = {(bf16)1.f, (bf16)1.f};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const bf16x2 pr = {v[2 * i], v[2 * i + 1]};
    acc = __builtin_amdgcn_fdot2_f32_bf16(pr, one, acc, false);
  }
  return acc;
}

}  // namespace siq
