// Internal interface of the fused linear cross-entropy kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.h"

namespace siq {

struct FlceArgs {
  const bf16* hidden;   // [n, hdim]
  const bf16* weight;   // [vocab, hdim]
  const int64_t* labels;
  int64_t n, hdim, vocab, ignore_index;
  int reduction;        // 0 mean over valid rows, 1 sum / *divisor
  const float* divisor;
  float* loss;
  int64_t* count;
  int64_t* bad_labels;
  bool grads;           // false: loss only (dhidden and dweight unused)
  bf16* dhidden;        // [n, hdim]
  bf16* dweight;        // [vocab, hdim] or nullptr
  int64_t chunk;        // tokens per logits chunk
  void* ws;
};

size_t flce_workspace_bytes(int64_t n, int64_t hdim, int64_t vocab, int64_t chunk, bool need_dh, bool need_dw);
hipError_t flce_run(const FlceArgs& a, hipStream_t stream);
hipError_t launch_scale_bf16(const bf16* src, bf16* dst, int64_t numel, const float* scalar, hipStream_t stream);

}  // namespace siq
