// Internal interface of the vision-token splice kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.h"

namespace siq {

struct SpliceArgs {
  const int64_t* ids;   // [n] token ids
  const bf16* weight;   // [vocab, hidden] embedding table
  const bf16* vision;   // [n_vision, hidden] projected vision rows
  bf16* out;            // [n, hidden]
  int32_t* rank;        // [n] workspace: image tokens before each token
  int64_t n, vocab, hidden, n_vision, image_id;
};

// image_pos [n_vision]: token index of each vision row; counts [2] (device):
// image tokens found, ids outside [0, vocab).
hipError_t splice_fwd(const SpliceArgs& a, int32_t* image_pos, int64_t* counts, hipStream_t stream);
hipError_t gather_rows(const bf16* src, const int32_t* rows, int64_t n, int64_t hidden, bf16* dst, hipStream_t stream);

}  // namespace siq
