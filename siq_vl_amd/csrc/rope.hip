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
// With fp32 cos / sin (bf16 q / k under bf16 autocast over fp32 master
// weights) the products and the sum are fp32, as torch's type promotion makes
// them, and the result is rounded to bf16 once -- the rounding the attention's
// cast to its compute dtype applies to the reference's fp32 q_embed / k_embed
// (rope_fwd8_f32 / rope_bwd8_f32 in common.h).
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

// cos / sin chunks of one token: 8 bf16 or 8 fp32 values each, as fp32 or bf16 registers
template <bool CSF32>
struct CsChunk;
template <>
struct CsChunk<false> {
  bf16x8 c1, c2, s1, s2;
  __device__ void load(const RopeArgs& a, uint32_t b, uint32_t s, int c, int half) {
    const bf16* cp = a.cos.p + b * a.cos.sb + s * a.cos.ss + 8 * c;
    const bf16* sp = a.sin.p + b * a.sin.sb + s * a.sin.ss + 8 * c;
    c1 = ld_bf16x8(cp);
    c2 = ld_bf16x8(cp + half);
    s1 = ld_bf16x8(sp);
    s2 = ld_bf16x8(sp + half);
  }
  template <bool BWD>
  __device__ void apply(const bf16x8& x1, const bf16x8& x2, bf16x8& o1, bf16x8& o2) const {
    if (!BWD)
      rope_fwd8(x1, x2, c1, c2, s1, s2, o1, o2);
    else
      rope_bwd8(x1, x2, c1, c2, s1, s2, o1, o2);
  }
};
template <>
struct CsChunk<true> {
  float c1[8], c2[8], s1[8], s2[8];
  __device__ static void ld8(const float* p, float (&v)[8]) {
    const f32x4 lo = *reinterpret_cast<const f32x4*>(p), hi = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[i] = lo[i];
      v[i + 4] = hi[i];
    }
  }
  __device__ void load(const RopeArgs& a, uint32_t b, uint32_t s, int c, int half) {
    const float* cp = reinterpret_cast<const float*>(a.cos.p) + b * a.cos.sb + s * a.cos.ss + 8 * c;
    const float* sp = reinterpret_cast<const float*>(a.sin.p) + b * a.sin.sb + s * a.sin.ss + 8 * c;
    ld8(cp, c1);
    ld8(cp + half, c2);
    ld8(sp, s1);
    ld8(sp + half, s2);
  }
  template <bool BWD>
  __device__ void apply(const bf16x8& x1, const bf16x8& x2, bf16x8& o1, bf16x8& o2) const {
    if (!BWD)
      rope_fwd8_f32(x1, x2, c1, c2, s1, s2, o1, o2);
    else
      rope_bwd8_f32(x1, x2, c1, c2, s1, s2, o1, o2);
  }
};

template <bool BWD, bool CSF32>
__device__ __forceinline__ void rope_row(const bf16* src, bf16* dst, int half, const CsChunk<CSF32>& cs) {
  const bf16x8 x1 = ld_bf16x8(src), x2 = ld_bf16x8(src + half);
  bf16x8 o1, o2;
  cs.template apply<BWD>(x1, x2, o1, o2);
  st_bf16x8(dst, o1);
  st_bf16x8(dst + half, o2);
}

template <bool BWD, bool CSF32>
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
    CsChunk<CSF32> cs;
    cs.load(a, b, s, c, half);
#pragma unroll 2
    for (int h = 0; h < a.hq; ++h)
      rope_row<BWD>(a.x[0].p + b * a.x[0].sb + s * a.x[0].ss + h * a.x[0].sh + 8 * c,
                    a.y[0].p + b * a.y[0].sb + s * a.y[0].ss + h * a.y[0].sh + 8 * c, half, cs);
#pragma unroll 2
    for (int h = 0; h < a.hkv; ++h)
      rope_row<BWD>(a.x[1].p + b * a.x[1].sb + s * a.x[1].ss + h * a.x[1].sh + 8 * c,
                    a.y[1].p + b * a.y[1].sb + s * a.y[1].ss + h * a.y[1].sh + 8 * c, half, cs);
  }
}

}  // namespace

hipError_t launch_rope(const RopeArgs& a, bool backward, hipStream_t stream) {
  const int64_t tpb = 256 / (a.d / 16);  // tokens per block step
  const int64_t ntok = a.batch * a.seqlen;
  int64_t blocks = (ntok + tpb - 1) / tpb;
  if (blocks > 2048) blocks = 2048;
  if (a.cs_f32) {
    if (backward)
      hipLaunchKernelGGL((rope_kernel<true, true>), dim3((unsigned)blocks), dim3(256), 0, stream, a);
    else
      hipLaunchKernelGGL((rope_kernel<false, true>), dim3((unsigned)blocks), dim3(256), 0, stream, a);
  } else {
    if (backward)
      hipLaunchKernelGGL((rope_kernel<true, false>), dim3((unsigned)blocks), dim3(256), 0, stream, a);
    else
      hipLaunchKernelGGL((rope_kernel<false, false>), dim3((unsigned)blocks), dim3(256), 0, stream, a);
  }
  return hipGetLastError();
}

}  // namespace siq
