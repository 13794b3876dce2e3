// Internal interface of the pixel-shuffle projector kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.h"

namespace siq {

// x [batch, side * side, dv] bf16 (the vision tower's patch grid, row-major);
// shuffled tokens m = (b, ho, wo) of side / r squared per image, features
// k = (i * r + j) * dv + c; weight [n, r * r * dv]; y [batch * t, n].
struct ProjArgs {
  const bf16* x;
  const bf16* weight;
  const bf16* dy;   // backward: upstream gradient [batch * t, n]
  bf16* y;          // forward output
  bf16* dx;         // backward: gradient of x (nullptr: not wanted)
  bf16* dweight;    // backward: gradient of weight (nullptr: not wanted)
  float* part;      // split-K partial sums (workspace)
  int64_t batch, side, dv, n;
  int r;
};

// Workspace of one call (split-K partial sums of the forward or of dweight).
size_t proj_workspace_bytes(int64_t batch, int64_t side, int64_t dv, int r, int64_t n);
hipError_t proj_fwd(const ProjArgs& a, hipStream_t stream);
hipError_t proj_bwd(const ProjArgs& a, hipStream_t stream);

}  // namespace siq
