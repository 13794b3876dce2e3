// Internal (C++) interface between the C-ABI layer and the attention kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tiles.h"

namespace siq {

// Tile sizes shared by the scheduler and the kernels.
constexpr int kFwdBM = 128;    // q rows per forward / dQ workgroup (4 waves x 32)
constexpr int kFwdBN = 64;     // kv rows per inner step of the forward / dQ loop
constexpr int kBwdBN = 32;     // kv rows per dK/dV workgroup (shared by its 4 waves)
constexpr int kBwdBM = 128;    // q rows per inner step of the dK/dV loop (4 waves x 32)
constexpr int kSchedKeys = 2048;

struct AttnParams {
  const bf16* q;
  const bf16* k;
  const bf16* v;
  const bf16* o;     // forward output (backward input)
  const bf16* dout;  // dO
  bf16* out;         // forward output
  float* lse;        // [hq, lse_head] natural-log LSE (forward output, backward input)
  bf16* dq;
  bf16* dk;
  bf16* dv;
  float* delta;      // [hq, lse_head] rowsum(dO * O) (backward workspace)
  const SeqInfo* seq;
  const int2* qtiles;   // (sequence, q-tile) ordered by decreasing work; x < 0 = idle
  const int2* kvtiles;  // (sequence, kv-tile) for the dK/dV kernel
  int batch, hq, hkv, n_rep;
  int64_t q_tok, q_head, k_tok, k_head, v_tok, v_head, o_tok, o_head;
  int64_t do_tok, do_head, dq_tok, dq_head, dk_tok, dk_head, dv_tok, dv_head;
  int64_t lse_head;
  int64_t total_q, total_k;
  float scale;       // softmax scale
  float scale_log2;  // scale * log2(e)
};

// Upper bound on the number of tiles of `rows` rows over `batch` sequences
// holding `total` tokens: sum ceil(L_b / rows) <= total / rows + batch.
inline int64_t tile_cap(int64_t total, int batch, int rows) { return total / rows + batch + 1; }

hipError_t launch_schedule(const int* cu_q, const int* cu_k, int batch, int64_t total_q, int64_t total_k,
                           int causal, SeqInfo* seq, int2* qtiles, int qcap, int2* kvtiles, int kvcap,
                           hipStream_t stream);
hipError_t launch_attn_fwd(const AttnParams& p, int d, int causal, int qcap, hipStream_t stream);
hipError_t launch_attn_bwd(const AttnParams& p, int d, int causal, int qcap, int kvcap, hipStream_t stream);

}  // namespace siq
