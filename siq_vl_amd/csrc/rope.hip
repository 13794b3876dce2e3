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
// hq may be 0 (a k-only pass, for the attention kernels that rotate q
// themselves).
//
// Work split: a thread owns one 8-element chunk c of the first half (and the
// matching chunk of the second) of one token at a time: D / 16 threads per
// token, 256 / (D / 16) tokens per block step, blocks striding over tokens
// (batch b, position s).  The thread loads its token's cos / sin chunks once
// and applies them to every q and k head of the token (two 16-byte loads and
// two 16-byte stores per head); a wave covers the same head of several
// tokens, whole 2 D-byte rows each.  Index arithmetic is one 32-bit division
// per token.
#include "rope.h"

namespace siq {

namespace {

template <bool BWD>
__device__ __forceinline__ void rope_row(const bf16* src, bf16* dst, int half, const bf16x8& c1, const bf16x8& c2,
                                         const bf16x8& s1, const bf16x8& s2) {
  const bf16x8 x1 = ld_bf16x8(src), x2 = ld_bf16x8(src + half);
  bf16x8 o1, o2;
  if (!BWD)
    rope_fwd8(x1, x2, c1, c2, s1, s2, o1, o2);
  else
    rope_bwd8(x1, x2, c1, c2, s1, s2, o1, o2);
  st_bf16x8(dst, o1);
  st_bf16x8(dst + half, o2);
}

template <bool BWD>
__global__ __launch_bounds__(256) void rope_kernel(const RopeArgs a) {
  const int cph = a.d / 16;          // chunks per half row (threads per token)
  const int tpb = 256 / cph;         // tokens per block step
  const int t = threadIdx.x;
  if (t >= tpb * cph) return;  // 256 not a multiple of D / 16
  const int c = t % cph;
  const int half = a.d / 2;
  const uint32_t S = (uint32_t)a.seqlen;
  const uint32_t ntok = (uint32_t)(a.batch * a.seqlen);
  for (uint32_t tok = blockIdx.x * tpb + t / cph; tok < ntok; tok += gridDim.x * tpb) {
    const uint32_t b = tok / S, s = tok - b * S;
    const bf16* cp = a.cos.p + b * a.cos.sb + s * a.cos.ss + 8 * c;
    const bf16* sp = a.sin.p + b * a.sin.sb + s * a.sin.ss + 8 * c;
    const bf16x8 c1 = ld_bf16x8(cp), c2 = ld_bf16x8(cp + half);
    const bf16x8 s1 = ld_bf16x8(sp), s2 = ld_bf16x8(sp + half);
#pragma unroll 2
    for (int h = 0; h < a.hq; ++h)
      rope_row<BWD>(a.x[0].p + b * a.x[0].sb + s * a.x[0].ss + h * a.x[0].sh + 8 * c,
                    a.y[0].p + b * a.y[0].sb + s * a.y[0].ss + h * a.y[0].sh + 8 * c, half, c1, c2, s1, s2);
#pragma unroll 2
    for (int h = 0; h < a.hkv; ++h)
      rope_row<BWD>(a.x[1].p + b * a.x[1].sb + s * a.x[1].ss + h * a.x[1].sh + 8 * c,
                    a.y[1].p + b * a.y[1].sb + s * a.y[1].ss + h * a.y[1].sh + 8 * c, half, c1, c2, s1, s2);
  }
}

}  // namespace

hipError_t launch_rope(const RopeArgs& a, bool backward, hipStream_t stream) {
  const int64_t tpb = 256 / (a.d / 16);  // tokens per block step
  const int64_t ntok = a.batch * a.seqlen;
  int64_t blocks = (ntok + tpb - 1) / tpb;
  if (blocks > 2048) blocks = 2048;
  if (backward)
    hipLaunchKernelGGL(rope_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL(rope_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, stream, a);
  return hipGetLastError();
}

}  // namespace siq
