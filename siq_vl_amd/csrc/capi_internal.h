// Helpers of the C-ABI layer shared by its source files (capi.cpp and the
// allocation-free entry point): validation, error recording, attention plan
// layout / build and the forward launch over a plan.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace siq_capi {

int fail(int code, const char* fmt, ...);
int ok();
bool aligned16(const void* p);

// An attention plan: header, per-sequence extents, the q-tile list (forward,
// dQ) and the dK/dV work items with their split tiles, and the scheduler's
// per-sequence prefix buffers (used for batches too long for its LDS).  It
// depends on the sequences, the head counts and causality, not on the
// tensors.
struct PlanLayout {
  size_t header, seq, qtiles, kvitems, seqbuf, splits, nsplit, qfirst, total;
  int qcap, kvcap;
};

PlanLayout plan_layout(int batch, int64_t total_q, int64_t total_k, bool kv);
hipError_t build_plan(char* base, const PlanLayout& L, const int32_t* cu_q, const int32_t* cu_k, int batch,
                      int64_t total_q, int64_t total_k, int hq, int hkv, bool causal, bool kv, hipStream_t s);
int check_attn_common(int batch, int max_q, int max_k, int64_t total_q, int64_t total_k, int hq, int hkv, int d,
                      float scale);
int check_cu(int batch, const void* cu_q, const void* cu_k);
int check_fwd_tensors(const void* q, const void* k, const void* v, void* o, float* lse, int64_t total_q,
                      int64_t total_k, const int64_t* strides);
// The rotary embedding fused into the attention kernels: cos / sin rows per
// token, and (forward) where the rotated q rows go.
struct RopeIn {
  const void* cos;
  const void* sin;
  int64_t cos_tok, sin_tok;
  void* qe;
  int64_t qe_tok, qe_head;
};

int run_fwd(const void* q, const void* k, const void* v, void* o, float* lse, int batch, int64_t total_q,
            int64_t total_k, int hq, int hkv, int d, const int64_t* strides, float scale, int causal,
            char* plan_base, const PlanLayout& L, hipStream_t s, const RopeIn* rope);

}  // namespace siq_capi
