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
  RopeTensor cos, sin;
  int64_t batch, seqlen;
  int hq, hkv, d;
};

// Needs d a multiple of 16 in [16, 512] and batch * seqlen < 2^32.
hipError_t launch_rope(const RopeArgs& a, bool backward, hipStream_t stream);

}  // namespace siq
