// siq_attn_varlen_fwd_noalloc: the varlen attention forward without a
// caller workspace, for callers that cannot allocate device memory (code
// under HIP graph capture, tight serving loops, harnesses that forbid it).
//
// The forward's only scratch is the batch's plan (header, per-sequence
// extents and the q-tile list, written by the scheduler and read by the
// forward kernel).  Here it lives in `scratch`, a file-scope device array of
// kScratchBytes: every GPU the library runs on holds its own copy until the
// process ends.  Its device address is looked up once per device with
// hipGetSymbolAddress (the array's name is only a host-side stand-in) and
// kept; the kernels receive that address like any workspace pointer.  The
// scheduler writes every plan field the forward reads, so nothing needs
// clearing between calls.  All calls on one GPU share the array: calls that
// overlap on one GPU (on different streams) race.
#include <hip/hip_runtime.h>

#include <mutex>

#include "../../include/siq_kernels.h"
#include "attn.h"
#include "capi_internal.h"

namespace {

using namespace siq_capi;

constexpr size_t kScratchBytes = size_t(1) << 20;
__device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
char* g_scratch[kMaxDevices];  // device address of each device's copy, resolved on first use

// Address of the current device's copy of `scratch`.
int current_scratch(char** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(SIQ_ERR_LAUNCH, "no usable current HIP device (device %d)", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fail(SIQ_ERR_LAUNCH, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                  hipGetErrorString(e));
    g_scratch[dev] = static_cast<char*>(p);
  }
  *out = g_scratch[dev];
  return SIQ_OK;
}

}  // namespace

extern "C" int siq_attn_varlen_fwd_noalloc(const void* q, const void* k, const void* v, void* o, float* lse,
                                           const int32_t* cu_q, const int32_t* cu_k, int batch, int max_q, int max_k,
                                           int64_t total_q, int64_t total_k, int hq, int hkv, int d,
                                           const int64_t* strides, float scale, int causal, void* stream) {
  int rc = check_attn_common(batch, max_q, max_k, total_q, total_k, hq, hkv, d, scale);
  if (rc || (rc = check_cu(batch, cu_q, cu_k))) return rc;
  if ((rc = check_fwd_tensors(q, k, v, o, lse, total_q, total_k, strides))) return rc;
  if (batch == 0 || total_q == 0) return ok();
  const PlanLayout L = plan_layout(batch, total_q, total_k, false);
  if (L.total > kScratchBytes)
    return fail(SIQ_ERR_WORKSPACE,
                "batch %d with %lld query tokens needs a %zu-byte plan, beyond the %zu-byte static scratch of the "
                "allocation-free forward (use siq_attn_varlen_fwd with a workspace)",
                batch, (long long)total_q, L.total, kScratchBytes);
  char* base = nullptr;
  if ((rc = current_scratch(&base))) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const hipError_t e = build_plan(base, L, cu_q, cu_k, batch, total_q, total_k, hq, hkv, causal != 0, false, s);
  if (e != hipSuccess) return fail(SIQ_ERR_LAUNCH, "schedule launch failed: %s", hipGetErrorString(e));
  return run_fwd(q, k, v, o, lse, batch, total_q, total_k, hq, hkv, d, strides, scale, causal, base, L, s, nullptr);
}
