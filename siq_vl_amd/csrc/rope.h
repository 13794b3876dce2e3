// Internal interface of the fused rotary-embedding kernel.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.h"

namespace siq {

// A [batch, seqlen, heads, D] bf16 tensor (cos / sin: [batch, seqlen, D], sh
// unused) with element strides; d is contiguous.
struct RopeTensor {
  bf16* p;
  int64_t sb, ss, sh;
};

struct RopeArgs {
  RopeTensor x[2];  // inputs: q, k (forward) or dq_embed, dk_embed (backward)
  RopeTensor y[2];  // outputs: q_embed, k_embed (forward) or dq, dk (backward)
  RopeTensor cos, sin;  // bf16, or fp32 when cs_f32 (p then points at floats; strides in floats)
  int64_t batch, seqlen;
  int hq, hkv, d;
  int cs_f32;
};

// Needs d a multiple of 16 in [16, 512] and batch * seqlen < 2^32.
hipError_t launch_rope(const RopeArgs& a, bool backward, hipStream_t stream);

}  // namespace siq
