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

// Embedding-table gradient: dw [vocab, hidden] (bf16, or fp32 when fp32) from
// grad [n, hidden] of the same dtype and ids [n]; ids equal to skip0 / skip1
// or outside [0, vocab) send nothing.  ws: embedding_bwd_workspace_bytes.
size_t embedding_bwd_workspace_bytes(int64_t n, int64_t vocab);
hipError_t embedding_bwd(const void* grad, const int64_t* ids, int64_t n, int64_t vocab, int64_t hidden, bool fp32,
                         int64_t skip0, int64_t skip1, void* dw, void* ws, hipStream_t stream);

}  // namespace siq
