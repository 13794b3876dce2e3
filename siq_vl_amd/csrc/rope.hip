// Fused rotary position embedding of q and k (forward and backward) for gfx950.
//
// Semantics: transformers models/qwen2/modeling_qwen2.py:105-135
// (rotate_half, apply_rotary_pos_emb; called at :206-211), evaluated as the
// reference evaluates it on bf16 tensors -- every torch op rounds its result
// to bf16:
//   out = (x * cos) + (rotate_half(x) * sin),  rotate_half(x) = cat(-x2, x1),
//   out[d]        = rb(rb(x[d] cos[d])               + rb(-x[d + D/2] sin[d])),
//   out[d + D/2]  = rb(rb(x[d + D/2] cos[d + D/2])   + rb(x[d] sin[d + D/2])),
// with rb = round to nearest even bf16 and d < D/2.  Each product of two bf16
// values is exact in fp32, so fp32 arithmetic followed by the same roundings
// reproduces the reference bit for bit.  The backward is the reference's
// autograd graph of those ops (MulBackward, the narrow / cat / neg backwards
// and the bf16 accumulation of the two contributions to x):
//   dx[d]        = rb(rb(g[d] cos[d])             + rb(g[d + D/2] sin[d + D/2])),
//   dx[d + D/2]  = rb(rb(g[d + D/2] cos[d + D/2]) - rb(g[d] sin[d])).
//
// The reference runs that as about eight elementwise passes per tensor
// (mul, two narrows, neg, cat, mul, add, and their backwards); here q and k
// go through one launch that reads each element once and writes it once:
// HBM-bound, 2 * (Hq + Hkv) * D * 2 bytes per token plus the cos / sin rows
// (L2 hits after the first head of a token).
//
// Work split: one thread per (row, 8-element chunk of the first half), row =
// (batch b, position s, head h) of q or k; the thread loads its chunk and the
// matching chunk of the second half (two 16-byte loads), and the cos / sin
// chunks of both halves, and writes both output chunks.  Consecutive threads
// take consecutive chunks of one row, so a wave covers whole rows.
#include "rope.h"

namespace siq {

namespace {

// fp32 -> nearest-even bf16 -> fp32, in integer arithmetic.  Written out
// because the compiler treats (float)(bf16)(a * b) of two bf16 values as a
// bf16 multiply it may then fuse, unrounded, into the following add
// (v_fmac_f32), which would break the reference's rounding.
__device__ __forceinline__ float rbf(float x) {
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  const uint32_t r = (u + 0x7FFFu + ((u >> 16) & 1u)) & 0xFFFF0000u;
  return x != x ? x : __builtin_bit_cast(float, r);
}

template <bool BWD>
__global__ __launch_bounds__(256) void rope_kernel(const RopeArgs a) {
  const int cph = a.d / 16;  // chunks per half row
  const int64_t qrows = a.batch * a.seqlen * a.hq;
  const int64_t rows = qrows + a.batch * a.seqlen * a.hkv;
  const int64_t total = rows * cph;
  const int half = a.d / 2;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = i / cph;
    const int c = (int)(i - row * cph);
    const bool isq = row < qrows;
    const int64_t r = isq ? row : row - qrows;
    const int H = isq ? a.hq : a.hkv;
    const int64_t bs = r / H;
    const int h = (int)(r - bs * H);
    const int64_t b = bs / a.seqlen, s = bs - b * a.seqlen;
    const RopeTensor& xin = isq ? a.x[0] : a.x[1];
    const RopeTensor& xout = isq ? a.y[0] : a.y[1];
    const bf16* src = xin.p + b * xin.sb + s * xin.ss + h * xin.sh + 8 * c;
    bf16* dst = xout.p + b * xout.sb + s * xout.ss + h * xout.sh + 8 * c;
    const bf16* cp = a.cos.p + b * a.cos.sb + s * a.cos.ss + 8 * c;
    const bf16* sp = a.sin.p + b * a.sin.sb + s * a.sin.ss + 8 * c;
    const bf16x8 x1 = ld_bf16x8(src), x2 = ld_bf16x8(src + half);
    const bf16x8 c1 = ld_bf16x8(cp), c2 = ld_bf16x8(cp + half);
    const bf16x8 s1 = ld_bf16x8(sp), s2 = ld_bf16x8(sp + half);
    bf16x8 o1, o2;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float u = (float)x1[k], v = (float)x2[k];
      if (!BWD) {
        o1[k] = (bf16)(rbf(u * (float)c1[k]) + rbf(-v * (float)s1[k]));
        o2[k] = (bf16)(rbf(v * (float)c2[k]) + rbf(u * (float)s2[k]));
      } else {
        o1[k] = (bf16)(rbf(u * (float)c1[k]) + rbf(v * (float)s2[k]));
        o2[k] = (bf16)(rbf(v * (float)c2[k]) - rbf(u * (float)s1[k]));
      }
    }
    st_bf16x8(dst, o1);
    st_bf16x8(dst + half, o2);
  }
}

}  // namespace

hipError_t launch_rope(const RopeArgs& a, bool backward, int blocks, hipStream_t stream) {
  if (backward)
    hipLaunchKernelGGL(rope_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL(rope_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, stream, a);
  return hipGetLastError();
}

}  // namespace siq
