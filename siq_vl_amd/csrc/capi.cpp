// extern "C" boundary: host-side validation, workspace carving, launches.
// Every check here happens before anything is enqueued, so a rejected call
// leaves the stream untouched.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <string>

#include "../../include/siq_kernels.h"
#include "attn.h"
#include "capi_internal.h"
#include "flce.h"
#include "probe.h"
#include "proj.h"
#include "rope.h"
#include "splice.h"

namespace siq_capi {

namespace {
thread_local std::string g_last_error;
}  // namespace

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int ok() {
  g_last_error.clear();
  return SIQ_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

PlanLayout plan_layout(int batch, int64_t total_q, int64_t total_k, bool kv) {
  PlanLayout L{};
  L.qcap = (int)siq::tile_cap(total_q, batch, siq::kFwdBM);
  L.kvcap = kv ? (int)siq::kv_item_cap(total_k, batch) : 0;
  size_t off = 0;
  L.header = off;
  off += align256(sizeof(siq::PlanHeader));
  L.seq = off;
  off += align256(sizeof(siq::SeqInfo) * (size_t)(batch > 0 ? batch : 1));
  L.qtiles = off;
  off += align256(sizeof(siq::QTile) * (size_t)L.qcap);
  L.kvitems = off;
  off += align256(sizeof(siq::KvItem) * (size_t)L.kvcap);
  L.seqbuf = off;
  if (kv) off += align256(sizeof(int) * ((size_t)(batch > 0 ? batch : 1) + 1));
  L.splits = off;
  if (kv) off += align256(sizeof(siq::SplitTile) * (size_t)siq::kMaxSplitTiles);
  L.nsplit = off;
  if (kv) off += 256;
  L.qfirst = off;
  off += align256(sizeof(int) * ((size_t)(batch > 0 ? batch : 1) + 1));
  L.total = off;
  return L;
}

// The backward's own scratch beyond the plan: split-tile partial sums,
// Delta = rowsum(dO o O), LSE * log2(e) and, for the atomic backward, the
// fp32 dQ sums [total_q][hq][d].
struct BwdLayout {
  size_t part, delta, lse2, dq_acc, total;
};

BwdLayout bwd_layout(int64_t total_q, int hq, int d, bool deterministic) {
  BwdLayout L{};
  size_t off = 0;
  L.part = off;
  off += align256(sizeof(float) * (size_t)siq::kSplitSlots * 2 * siq::kBwdBN * (size_t)d);
  L.delta = off;
  off += align256(sizeof(float) * (size_t)hq * (size_t)total_q);
  L.lse2 = off;
  off += align256(sizeof(float) * (size_t)hq * (size_t)total_q);
  L.dq_acc = off;
  if (!deterministic) off += align256(sizeof(float) * (size_t)total_q * (size_t)hq * (size_t)d);
  L.total = off;
  return L;
}

// Builds the plan at `base` (laid out by L) on `stream`.
hipError_t build_plan(char* base, const PlanLayout& L, const int32_t* cu_q, const int32_t* cu_k, int batch,
                      int64_t total_q, int64_t total_k, int hq, int hkv, bool causal, bool kv, hipStream_t s) {
  return siq::launch_schedule(cu_q, cu_k, batch, total_q, total_k, causal ? 1 : 0, hq / hkv, hkv,
                              reinterpret_cast<siq::PlanHeader*>(base + L.header),
                              reinterpret_cast<siq::SeqInfo*>(base + L.seq),
                              reinterpret_cast<siq::QTile*>(base + L.qtiles), siq::kFwdBM, L.qcap,
                              kv ? reinterpret_cast<siq::KvItem*>(base + L.kvitems) : nullptr, L.kvcap,
                              kv ? reinterpret_cast<int*>(base + L.seqbuf) : nullptr,
                              kv ? reinterpret_cast<siq::SplitTile*>(base + L.splits) : nullptr,
                              kv ? reinterpret_cast<int*>(base + L.nsplit) : nullptr,
                              reinterpret_cast<int*>(base + L.qfirst), s);
}

int check_attn_common(int batch, int max_q, int max_k, int64_t total_q, int64_t total_k, int hq, int hkv, int d,
                      float scale) {
  if (batch < 0) return fail(SIQ_ERR_INVALID_ARGUMENT, "batch must be >= 0 (got %d)", batch);
  if (total_q < 0 || total_k < 0 || total_q >= (int64_t(1) << 31) || total_k >= (int64_t(1) << 31))
    return fail(SIQ_ERR_INVALID_ARGUMENT, "total_q/total_k must be in [0, 2^31) (got %lld, %lld)",
                (long long)total_q, (long long)total_k);
  if (max_q < 0 || max_k < 0) return fail(SIQ_ERR_INVALID_ARGUMENT, "max_seqlen must be >= 0");
  if (hq <= 0 || hkv <= 0) return fail(SIQ_ERR_INVALID_ARGUMENT, "head counts must be positive (hq=%d, hkv=%d)", hq, hkv);
  if (hq % hkv != 0)
    return fail(SIQ_ERR_INVALID_ARGUMENT, "hq (%d) must be a multiple of hkv (%d) for GQA", hq, hkv);
  if (d != 64 && d != 128) return fail(SIQ_ERR_UNSUPPORTED, "head_dim %d unsupported (64 or 128)", d);
  if (!std::isfinite(scale)) return fail(SIQ_ERR_INVALID_ARGUMENT, "softmax_scale must be finite");
  return SIQ_OK;
}

int check_cu(int batch, const void* cu_q, const void* cu_k) {
  if (batch > 0 && (cu_q == nullptr || cu_k == nullptr))
    return fail(SIQ_ERR_INVALID_ARGUMENT, "cu_seqlens_q / cu_seqlens_k must not be NULL");
  return SIQ_OK;
}

int check_tensor(const char* name, const void* p, const int64_t* st, bool need) {
  if (!need) return SIQ_OK;
  if (p == nullptr) return fail(SIQ_ERR_INVALID_ARGUMENT, "%s must not be NULL", name);
  if (!aligned16(p)) return fail(SIQ_ERR_ALIGNMENT, "%s is not 16-byte aligned", name);
  if (st[0] < 0 || st[1] < 0 || (st[0] & 7) || (st[1] & 7))
    return fail(SIQ_ERR_ALIGNMENT, "%s strides (%lld, %lld) must be non-negative multiples of 8 elements", name,
                (long long)st[0], (long long)st[1]);
  return SIQ_OK;
}

}  // namespace siq_capi

using namespace siq_capi;

extern "C" {

int siq_abi_version(void) { return SIQ_ABI_VERSION; }

const char* siq_last_error(void) { return g_last_error.c_str(); }

size_t siq_attn_fwd_workspace_bytes(int batch, int64_t total_q, int64_t total_k, int hq, int hkv, int d) {
  (void)hkv;
  if (batch < 0 || total_q < 0 || total_k < 0 || hq <= 0 || d <= 0) return 0;
  return plan_layout(batch, total_q, total_k, false).total;
}

size_t siq_attn_bwd_workspace_bytes(int batch, int64_t total_q, int64_t total_k, int hq, int hkv, int d,
                                    int deterministic) {
  (void)hkv;
  if (batch < 0 || total_q < 0 || total_k < 0 || hq <= 0 || d <= 0) return 0;
  return plan_layout(batch, total_q, total_k, true).total + bwd_layout(total_q, hq, d, deterministic != 0).total;
}

size_t siq_attn_plan_bytes(int batch, int64_t total_q, int64_t total_k) {
  if (batch < 0 || total_q < 0 || total_k < 0) return 0;
  return plan_layout(batch, total_q, total_k, true).total;
}

size_t siq_attn_bwd_plan_workspace_bytes(int batch, int64_t total_q, int64_t total_k, int hq, int hkv, int d,
                                         int deterministic) {
  (void)batch;
  (void)total_k;
  (void)hkv;
  if (total_q < 0 || hq <= 0 || d <= 0) return 0;
  return bwd_layout(total_q, hq, d, deterministic != 0).total;
}

int siq_attn_build_plan(const int32_t* cu_q, const int32_t* cu_k, int batch, int64_t total_q, int64_t total_k,
                        int hq, int hkv, int causal, void* plan, size_t plan_bytes, void* stream) {
  int rc = check_attn_common(batch, 0, 0, total_q, total_k, hq, hkv, 128, 1.f);
  if (rc || (rc = check_cu(batch, cu_q, cu_k))) return rc;
  const PlanLayout L = plan_layout(batch, total_q, total_k, true);
  if (plan == nullptr || plan_bytes < L.total || !aligned16(plan))
    return fail(SIQ_ERR_WORKSPACE, "plan needs %zu bytes (16-byte aligned), got %zu", L.total, plan_bytes);
  const hipError_t e = build_plan(static_cast<char*>(plan), L, cu_q, cu_k, batch, total_q, total_k, hq, hkv,
                                  causal != 0, true, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(SIQ_ERR_LAUNCH, "schedule launch failed: %s", hipGetErrorString(e));
  return ok();
}

}  // extern "C"

namespace siq_capi {

// Fills the plan pointers of p from a plan laid out by L at base.
void set_plan(siq::AttnParams& p, char* base, const PlanLayout& L) {
  p.plan = reinterpret_cast<siq::PlanHeader*>(base + L.header);
  p.seq = reinterpret_cast<const siq::SeqInfo*>(base + L.seq);
  p.qtiles = reinterpret_cast<const siq::QTile*>(base + L.qtiles);
  p.kvitems = reinterpret_cast<const siq::KvItem*>(base + L.kvitems);
  p.splits = reinterpret_cast<const siq::SplitTile*>(base + L.splits);
  p.nsplit = reinterpret_cast<const int*>(base + L.nsplit);
}

void set_common(siq::AttnParams& p, int batch, int64_t total_q, int64_t total_k, int hq, int hkv,
                const int64_t* strides, int nstrides, float scale) {
  p.batch = batch;
  p.hq = hq;
  p.hkv = hkv;
  p.n_rep = hq / hkv;
  int64_t* dst[16] = {&p.q_tok, &p.q_head, &p.k_tok, &p.k_head, &p.v_tok, &p.v_head, &p.o_tok, &p.o_head,
                      &p.do_tok, &p.do_head, &p.dq_tok, &p.dq_head, &p.dk_tok, &p.dk_head, &p.dv_tok, &p.dv_head};
  for (int i = 0; i < nstrides; ++i) *dst[i] = strides[i];
  p.lse_head = total_q;
  p.total_q = total_q;
  p.total_k = total_k;
  p.scale = scale;
  p.scale_log2 = scale * siq::kLog2e;
}

int check_fwd_tensors(const void* q, const void* k, const void* v, void* o, float* lse, int64_t total_q,
                      int64_t total_k, const int64_t* strides) {
  if (strides == nullptr) return fail(SIQ_ERR_INVALID_ARGUMENT, "strides must not be NULL");
  const bool nq = total_q > 0, nk = total_k > 0;
  int rc;
  if ((rc = check_tensor("q", q, strides + 0, nq)) || (rc = check_tensor("k", k, strides + 2, nk)) ||
      (rc = check_tensor("v", v, strides + 4, nk)) || (rc = check_tensor("o", o, strides + 6, nq)))
    return rc;
  if (nq && (lse == nullptr || (reinterpret_cast<uintptr_t>(lse) & 3u)))
    return fail(SIQ_ERR_ALIGNMENT, "lse must be a non-NULL 4-byte aligned fp32 pointer");
  return SIQ_OK;
}

int check_bwd_tensors(const void* q, const void* k, const void* v, const void* o, const float* lse,
                      const void* dout, void* dq, void* dk, void* dv, int64_t total_q, int64_t total_k,
                      const int64_t* strides) {
  if (strides == nullptr) return fail(SIQ_ERR_INVALID_ARGUMENT, "strides must not be NULL");
  const bool nq = total_q > 0, nk = total_k > 0;
  int rc;
  if ((rc = check_tensor("q", q, strides + 0, nq)) || (rc = check_tensor("k", k, strides + 2, nk)) ||
      (rc = check_tensor("v", v, strides + 4, nk)) || (rc = check_tensor("o", o, strides + 6, nq)) ||
      (rc = check_tensor("dout", dout, strides + 8, nq)) || (rc = check_tensor("dq", dq, strides + 10, nq)) ||
      (rc = check_tensor("dk", dk, strides + 12, nk)) || (rc = check_tensor("dv", dv, strides + 14, nk)))
    return rc;
  if (nq && (lse == nullptr || (reinterpret_cast<uintptr_t>(lse) & 3u)))
    return fail(SIQ_ERR_ALIGNMENT, "lse must be a non-NULL 4-byte aligned fp32 pointer");
  return SIQ_OK;
}

// Forward over a built plan (at plan_base, laid out by L); rope non-null:
// q is rotated inside the kernel and the rotated rows go to rope->qe.
int run_fwd(const void* q, const void* k, const void* v, void* o, float* lse, int batch, int64_t total_q,
            int64_t total_k, int hq, int hkv, int d, const int64_t* strides, float scale, int causal,
            char* plan_base, const PlanLayout& L, hipStream_t s, const RopeIn* rope) {
  siq::AttnParams p{};
  if (rope != nullptr) {
    p.rcos = static_cast<const siq::bf16*>(rope->cos);
    p.rsin = static_cast<const siq::bf16*>(rope->sin);
    p.rc_tok = rope->cos_tok;
    p.rs_tok = rope->sin_tok;
    p.qe = static_cast<siq::bf16*>(rope->qe);
    p.qe_tok = rope->qe_tok;
    p.qe_head = rope->qe_head;
  }
  p.q = static_cast<const siq::bf16*>(q);
  p.k = static_cast<const siq::bf16*>(k);
  p.v = static_cast<const siq::bf16*>(v);
  p.out = static_cast<siq::bf16*>(o);
  p.lse = lse;
  set_plan(p, plan_base, L);
  set_common(p, batch, total_q, total_k, hq, hkv, strides, 8, scale);
  const hipError_t e = siq::launch_attn_fwd(p, d, causal != 0, L.qcap, s);
  if (e != hipSuccess) return fail(SIQ_ERR_LAUNCH, "attention forward launch failed: %s", hipGetErrorString(e));
  return ok();
}

// Backward over a built plan and the backward's own scratch at ws.
int run_bwd(const void* q, const void* k, const void* v, const void* o, const float* lse, const void* dout, void* dq,
            void* dk, void* dv, int batch, int64_t total_q, int64_t total_k, int hq, int hkv, int d,
            const int64_t* strides, float scale, int causal, bool deterministic, char* plan_base,
            const PlanLayout& L, char* ws, hipStream_t s, const RopeIn* rope = nullptr) {
  const BwdLayout B = bwd_layout(total_q, hq, d, deterministic);
  siq::AttnParams p{};
  if (rope != nullptr) {
    p.rcos = static_cast<const siq::bf16*>(rope->cos);
    p.rsin = static_cast<const siq::bf16*>(rope->sin);
    p.rc_tok = rope->cos_tok;
    p.rs_tok = rope->sin_tok;
  }
  p.q = static_cast<const siq::bf16*>(q);
  p.k = static_cast<const siq::bf16*>(k);
  p.v = static_cast<const siq::bf16*>(v);
  p.o = static_cast<const siq::bf16*>(o);
  p.dout = static_cast<const siq::bf16*>(dout);
  p.lse = const_cast<float*>(lse);
  p.dq = static_cast<siq::bf16*>(dq);
  p.dk = static_cast<siq::bf16*>(dk);
  p.dv = static_cast<siq::bf16*>(dv);
  p.delta = reinterpret_cast<float*>(ws + B.delta);
  p.lse2 = reinterpret_cast<float*>(ws + B.lse2);
  p.dkv_part = reinterpret_cast<float*>(ws + B.part);
  p.dq_acc = deterministic ? nullptr : reinterpret_cast<float*>(ws + B.dq_acc);
  set_plan(p, plan_base, L);
  set_common(p, batch, total_q, total_k, hq, hkv, strides, 16, scale);
  const hipError_t e = siq::launch_attn_bwd(p, d, causal != 0, L.qcap, L.kvcap, s);
  if (e != hipSuccess) return fail(SIQ_ERR_LAUNCH, "attention backward launch failed: %s", hipGetErrorString(e));
  return ok();
}

}  // namespace siq_capi

using namespace siq_capi;

extern "C" {

int siq_attn_varlen_fwd(const void* q, const void* k, const void* v, void* o, float* lse, const int32_t* cu_q,
                        const int32_t* cu_k, int batch, int max_q, int max_k, int64_t total_q, int64_t total_k,
                        int hq, int hkv, int d, const int64_t* strides, float scale, int causal, void* ws,
                        size_t ws_bytes, void* stream) {
  int rc = check_attn_common(batch, max_q, max_k, total_q, total_k, hq, hkv, d, scale);
  if (rc || (rc = check_cu(batch, cu_q, cu_k))) return rc;
  if ((rc = check_fwd_tensors(q, k, v, o, lse, total_q, total_k, strides))) return rc;
  if (batch == 0 || total_q == 0) return ok();
  const PlanLayout L = plan_layout(batch, total_q, total_k, false);
  if (ws == nullptr || ws_bytes < L.total || !aligned16(ws))
    return fail(SIQ_ERR_WORKSPACE, "workspace needs %zu bytes (16-byte aligned), got %zu", L.total, ws_bytes);
  hipStream_t s = static_cast<hipStream_t>(stream);
  char* base = static_cast<char*>(ws);
  const hipError_t e = build_plan(base, L, cu_q, cu_k, batch, total_q, total_k, hq, hkv, causal != 0, false, s);
  if (e != hipSuccess) return fail(SIQ_ERR_LAUNCH, "schedule launch failed: %s", hipGetErrorString(e));
  return run_fwd(q, k, v, o, lse, batch, total_q, total_k, hq, hkv, d, strides, scale, causal, base, L, s, nullptr);
}

int siq_attn_varlen_fwd_plan(const void* q, const void* k, const void* v, void* o, float* lse, int batch,
                             int64_t total_q, int64_t total_k, int hq, int hkv, int d, const int64_t* strides,
                             float scale, int causal, const void* plan, size_t plan_bytes, void* stream) {
  int rc = check_attn_common(batch, 0, 0, total_q, total_k, hq, hkv, d, scale);
  if (rc) return rc;
  if ((rc = check_fwd_tensors(q, k, v, o, lse, total_q, total_k, strides))) return rc;
  if (batch == 0 || total_q == 0) return ok();
  const PlanLayout L = plan_layout(batch, total_q, total_k, true);
  if (plan == nullptr || plan_bytes < L.total || !aligned16(plan))
    return fail(SIQ_ERR_WORKSPACE, "plan needs %zu bytes (16-byte aligned), got %zu", L.total, plan_bytes);
  return run_fwd(q, k, v, o, lse, batch, total_q, total_k, hq, hkv, d, strides, scale, causal,
                 static_cast<char*>(const_cast<void*>(plan)), L, static_cast<hipStream_t>(stream), nullptr);
}

int siq_attn_varlen_bwd(const void* q, const void* k, const void* v, const void* o, const float* lse,
                        const void* dout, void* dq, void* dk, void* dv, const int32_t* cu_q, const int32_t* cu_k,
                        int batch, int max_q, int max_k, int64_t total_q, int64_t total_k, int hq, int hkv, int d,
                        const int64_t* strides, float scale, int causal, int deterministic, void* ws,
                        size_t ws_bytes, void* stream) {
  int rc = check_attn_common(batch, max_q, max_k, total_q, total_k, hq, hkv, d, scale);
  if (rc || (rc = check_cu(batch, cu_q, cu_k))) return rc;
  if ((rc = check_bwd_tensors(q, k, v, o, lse, dout, dq, dk, dv, total_q, total_k, strides))) return rc;
  if (batch == 0 || (total_q == 0 && total_k == 0)) return ok();
  const PlanLayout L = plan_layout(batch, total_q, total_k, true);
  const size_t need = L.total + bwd_layout(total_q, hq, d, deterministic != 0).total;
  if (ws == nullptr || ws_bytes < need || !aligned16(ws))
    return fail(SIQ_ERR_WORKSPACE, "workspace needs %zu bytes (16-byte aligned), got %zu", need, ws_bytes);
  hipStream_t s = static_cast<hipStream_t>(stream);
  char* base = static_cast<char*>(ws);
  const hipError_t e = build_plan(base, L, cu_q, cu_k, batch, total_q, total_k, hq, hkv, causal != 0, true, s);
  if (e != hipSuccess) return fail(SIQ_ERR_LAUNCH, "schedule launch failed: %s", hipGetErrorString(e));
  return run_bwd(q, k, v, o, lse, dout, dq, dk, dv, batch, total_q, total_k, hq, hkv, d, strides, scale, causal,
                 deterministic != 0, base, L, base + L.total, s);
}

int siq_attn_varlen_bwd_plan(const void* q, const void* k, const void* v, const void* o, const float* lse,
                             const void* dout, void* dq, void* dk, void* dv, int batch, int64_t total_q,
                             int64_t total_k, int hq, int hkv, int d, const int64_t* strides, float scale, int causal,
                             int deterministic, const void* plan, size_t plan_bytes, void* ws, size_t ws_bytes,
                             void* stream) {
  int rc = check_attn_common(batch, 0, 0, total_q, total_k, hq, hkv, d, scale);
  if (rc) return rc;
  if ((rc = check_bwd_tensors(q, k, v, o, lse, dout, dq, dk, dv, total_q, total_k, strides))) return rc;
  if (batch == 0 || (total_q == 0 && total_k == 0)) return ok();
  const PlanLayout L = plan_layout(batch, total_q, total_k, true);
  if (plan == nullptr || plan_bytes < L.total || !aligned16(plan))
    return fail(SIQ_ERR_WORKSPACE, "plan needs %zu bytes (16-byte aligned), got %zu", L.total, plan_bytes);
  const size_t need = bwd_layout(total_q, hq, d, deterministic != 0).total;
  if (ws == nullptr || ws_bytes < need || !aligned16(ws))
    return fail(SIQ_ERR_WORKSPACE, "workspace needs %zu bytes (16-byte aligned), got %zu", need, ws_bytes);
  return run_bwd(q, k, v, o, lse, dout, dq, dk, dv, batch, total_q, total_k, hq, hkv, d, strides, scale, causal,
                 deterministic != 0, static_cast<char*>(const_cast<void*>(plan)), L, static_cast<char*>(ws),
                 static_cast<hipStream_t>(stream));
}

}  // extern "C"

namespace {

// cos / sin rows per token: 16-byte aligned, token strides multiples of 8
// elements (rows are D contiguous bf16).
int check_rope_rows(const void* cos, const void* sin, int64_t cos_tok, int64_t sin_tok, int64_t total_q) {
  if (total_q == 0) return SIQ_OK;
  if (cos == nullptr || sin == nullptr) return fail(SIQ_ERR_INVALID_ARGUMENT, "cos and sin must not be NULL");
  if (!aligned16(cos) || !aligned16(sin)) return fail(SIQ_ERR_ALIGNMENT, "cos / sin not 16-byte aligned");
  if (cos_tok < 0 || sin_tok < 0 || (cos_tok & 7) || (sin_tok & 7))
    return fail(SIQ_ERR_ALIGNMENT, "cos / sin token strides (%lld, %lld) must be non-negative multiples of 8",
                (long long)cos_tok, (long long)sin_tok);
  return SIQ_OK;
}

}  // namespace

extern "C" {

int siq_attn_rope_fwd_plan(const void* q, const void* k, const void* v, void* o, float* lse, void* q_embed,
                           const void* cos, const void* sin, int batch, int64_t total_q, int64_t total_k, int hq,
                           int hkv, int d, const int64_t* strides, float scale, int causal, const void* plan,
                           size_t plan_bytes, void* stream) {
  int rc = check_attn_common(batch, 0, 0, total_q, total_k, hq, hkv, d, scale);
  if (rc) return rc;
  if ((rc = check_fwd_tensors(q, k, v, o, lse, total_q, total_k, strides))) return rc;
  if ((rc = check_tensor("q_embed", q_embed, strides + 8, total_q > 0))) return rc;
  if ((rc = check_rope_rows(cos, sin, strides[10], strides[11], total_q))) return rc;
  if (batch == 0 || total_q == 0) return ok();
  const PlanLayout L = plan_layout(batch, total_q, total_k, true);
  if (plan == nullptr || plan_bytes < L.total || !aligned16(plan))
    return fail(SIQ_ERR_WORKSPACE, "plan needs %zu bytes (16-byte aligned), got %zu", L.total, plan_bytes);
  const RopeIn rope{cos, sin, strides[10], strides[11], q_embed, strides[8], strides[9]};
  return run_fwd(q, k, v, o, lse, batch, total_q, total_k, hq, hkv, d, strides, scale, causal,
                 static_cast<char*>(const_cast<void*>(plan)), L, static_cast<hipStream_t>(stream), &rope);
}

int siq_attn_rope_bwd_plan(const void* q_embed, const void* k, const void* v, const void* o, const float* lse,
                           const void* dout, void* dq, void* dk, void* dv, const void* cos, const void* sin, int batch,
                           int64_t total_q, int64_t total_k, int hq, int hkv, int d, const int64_t* strides,
                           float scale, int causal, const void* plan, size_t plan_bytes, void* ws, size_t ws_bytes,
                           void* stream) {
  int rc = check_attn_common(batch, 0, 0, total_q, total_k, hq, hkv, d, scale);
  if (rc) return rc;
  if ((rc = check_bwd_tensors(q_embed, k, v, o, lse, dout, dq, dk, dv, total_q, total_k, strides))) return rc;
  if ((rc = check_rope_rows(cos, sin, strides[16], strides[17], total_q))) return rc;
  if (batch == 0 || (total_q == 0 && total_k == 0)) return ok();
  const PlanLayout L = plan_layout(batch, total_q, total_k, true);
  if (plan == nullptr || plan_bytes < L.total || !aligned16(plan))
    return fail(SIQ_ERR_WORKSPACE, "plan needs %zu bytes (16-byte aligned), got %zu", L.total, plan_bytes);
  const size_t need = bwd_layout(total_q, hq, d, true).total;
  if (ws == nullptr || ws_bytes < need || !aligned16(ws))
    return fail(SIQ_ERR_WORKSPACE, "workspace needs %zu bytes (16-byte aligned), got %zu", need, ws_bytes);
  const RopeIn rope{cos, sin, strides[16], strides[17], nullptr, 0, 0};
  return run_bwd(q_embed, k, v, o, lse, dout, dq, dk, dv, batch, total_q, total_k, hq, hkv, d, strides, scale,
                 causal, true, static_cast<char*>(const_cast<void*>(plan)), L, static_cast<char*>(ws),
                 static_cast<hipStream_t>(stream), &rope);
}

size_t siq_flce_workspace_bytes(int64_t n, int64_t hdim, int64_t vocab, int64_t chunk_tokens, int need_dweight) {
  if (n < 0 || hdim <= 0 || vocab <= 0) return 0;
  return siq::flce_workspace_bytes(n, hdim, vocab, chunk_tokens, true, need_dweight != 0);
}

size_t siq_flce_loss_workspace_bytes(int64_t n, int64_t hdim, int64_t vocab) {
  if (n < 0 || hdim <= 0 || vocab <= 0) return 0;
  return siq::flce_workspace_bytes(n, hdim, vocab, 1, false, false);
}

}  // extern "C"

namespace {

// Shared by siq_flce_fwd_bwd (grads) and siq_flce_loss (loss only: no
// dhidden / dweight).
int flce_call(bool grads, const void* hidden, const void* weight, const int64_t* labels, int64_t n, int64_t hdim,
              int64_t vocab, int64_t ignore_index, int reduction, const float* divisor, float* loss, int64_t* count,
              int64_t* bad_labels, void* dhidden, void* dweight, int64_t chunk_tokens, void* ws, size_t ws_bytes,
              void* stream) {
  if (n < 0) return fail(SIQ_ERR_INVALID_ARGUMENT, "n must be >= 0");
  if (hdim <= 0 || vocab <= 0) return fail(SIQ_ERR_INVALID_ARGUMENT, "hdim and vocab must be positive");
  if (hdim % 64 != 0) return fail(SIQ_ERR_UNSUPPORTED, "hdim (%lld) must be a multiple of 64", (long long)hdim);
  if (vocab % 8 != 0) return fail(SIQ_ERR_UNSUPPORTED, "vocab (%lld) must be a multiple of 8", (long long)vocab);
  if (vocab >= (int64_t(1) << 31) || n >= (int64_t(1) << 31))
    return fail(SIQ_ERR_INVALID_ARGUMENT, "n and vocab must be < 2^31");
  if (reduction != 0 && reduction != 1) return fail(SIQ_ERR_INVALID_ARGUMENT, "reduction must be 0 (mean) or 1 (sum/divisor)");
  if (reduction == 1 && divisor == nullptr) return fail(SIQ_ERR_INVALID_ARGUMENT, "reduction 1 needs a divisor pointer");
  if (loss == nullptr || count == nullptr || bad_labels == nullptr)
    return fail(SIQ_ERR_INVALID_ARGUMENT, "loss, count and bad_labels must not be NULL");
  if (n > 0) {
    if (hidden == nullptr || labels == nullptr || (grads && dhidden == nullptr))
      return fail(SIQ_ERR_INVALID_ARGUMENT, grads ? "hidden, labels and dhidden must not be NULL"
                                                  : "hidden and labels must not be NULL");
    if (!aligned16(hidden) || (grads && !aligned16(dhidden)))
      return fail(SIQ_ERR_ALIGNMENT, "hidden/dhidden not 16-byte aligned");
  }
  if (weight == nullptr || !aligned16(weight)) return fail(SIQ_ERR_ALIGNMENT, "weight must be non-NULL and 16-byte aligned");
  if (dweight != nullptr && !aligned16(dweight)) return fail(SIQ_ERR_ALIGNMENT, "dweight not 16-byte aligned");
  if (chunk_tokens <= 0) return fail(SIQ_ERR_INVALID_ARGUMENT, "chunk_tokens must be positive");
  const size_t need = siq::flce_workspace_bytes(n, hdim, vocab, chunk_tokens, grads, dweight != nullptr);
  if (ws == nullptr || ws_bytes < need || !aligned16(ws))
    return fail(SIQ_ERR_WORKSPACE, "workspace needs %zu bytes (16-byte aligned), got %zu", need, ws_bytes);
  siq::FlceArgs a{};
  a.hidden = static_cast<const siq::bf16*>(hidden);
  a.weight = static_cast<const siq::bf16*>(weight);
  a.labels = labels;
  a.n = n;
  a.hdim = hdim;
  a.vocab = vocab;
  a.ignore_index = ignore_index;
  a.reduction = reduction;
  a.divisor = divisor;
  a.loss = loss;
  a.count = count;
  a.bad_labels = bad_labels;
  a.grads = grads;
  a.dhidden = static_cast<siq::bf16*>(dhidden);
  a.dweight = static_cast<siq::bf16*>(dweight);
  a.chunk = chunk_tokens;
  a.ws = ws;
  const hipError_t e = siq::flce_run(a, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(SIQ_ERR_LAUNCH, "fused CE launch failed: %s", hipGetErrorString(e));
  return ok();
}

}  // namespace

extern "C" {

int siq_flce_fwd_bwd(const void* hidden, const void* weight, const int64_t* labels, int64_t n, int64_t hdim,
                     int64_t vocab, int64_t ignore_index, int reduction, const float* divisor, float* loss,
                     int64_t* count, int64_t* bad_labels, void* dhidden, void* dweight, int64_t chunk_tokens,
                     void* ws, size_t ws_bytes, void* stream) {
  return flce_call(true, hidden, weight, labels, n, hdim, vocab, ignore_index, reduction, divisor, loss, count,
                   bad_labels, dhidden, dweight, chunk_tokens, ws, ws_bytes, stream);
}

int siq_flce_loss(const void* hidden, const void* weight, const int64_t* labels, int64_t n, int64_t hdim,
                  int64_t vocab, int64_t ignore_index, int reduction, const float* divisor, float* loss,
                  int64_t* count, int64_t* bad_labels, void* ws, size_t ws_bytes, void* stream) {
  return flce_call(false, hidden, weight, labels, n, hdim, vocab, ignore_index, reduction, divisor, loss, count,
                   bad_labels, nullptr, nullptr, 1, ws, ws_bytes, stream);
}

}  // extern "C"

namespace {

// Shared by siq_rope_fwd / siq_rope_bwd: validation, then one launch over the
// q rows and k rows.  strides: x0 (b, s, h), x1 (b, s, h), cos (b, s),
// sin (b, s), y0 (b, s, h), y1 (b, s, h).
int rope_call(bool backward, const void* x0, const void* x1, const void* cosp, const void* sinp, void* y0, void* y1,
              int64_t batch, int64_t seqlen, int hq, int hkv, int d, const int64_t* st, void* stream,
              int cs_dtype = SIQ_DTYPE_BF16) {
  const char* nm[6] = {backward ? "dq_embed" : "q", backward ? "dk_embed" : "k", "cos", "sin",
                       backward ? "dq" : "q_embed", backward ? "dk" : "k_embed"};
  if (batch < 0 || seqlen < 0) return fail(SIQ_ERR_INVALID_ARGUMENT, "batch and seqlen must be >= 0");
  if (hq < 0 || hkv <= 0 || hq > 4096 || hkv > 4096)
    return fail(SIQ_ERR_INVALID_ARGUMENT, "head counts must be hq in [0, 4096], hkv in [1, 4096] (hq=%d, hkv=%d)",
                hq, hkv);
  if (d < 16 || d > 512 || d % 16 != 0)
    return fail(SIQ_ERR_UNSUPPORTED, "head_dim %d unsupported (a multiple of 16 in [16, 512])", d);
  if (st == nullptr) return fail(SIQ_ERR_INVALID_ARGUMENT, "strides must not be NULL");
  if (cs_dtype != SIQ_DTYPE_BF16 && cs_dtype != SIQ_DTYPE_FP32)
    return fail(SIQ_ERR_INVALID_ARGUMENT, "cos / sin dtype must be SIQ_DTYPE_BF16 or SIQ_DTYPE_FP32");
  if (batch * seqlen == 0) return ok();
  if (batch * seqlen >= (int64_t(1) << 32) || batch >= (int64_t(1) << 31) || seqlen >= (int64_t(1) << 31))
    return fail(SIQ_ERR_INVALID_ARGUMENT, "batch * seqlen must be < 2^32");
  const void* ptr[6] = {x0, x1, cosp, sinp, y0, y1};
  const int first[6] = {0, 3, 6, 8, 10, 13}, count[6] = {3, 3, 2, 2, 3, 3};
  for (int t = 0; t < 6; ++t) {
    if (hq == 0 && (t == 0 || t == 4)) continue;  // k-only pass: q and its output are not touched
    if (ptr[t] == nullptr) return fail(SIQ_ERR_INVALID_ARGUMENT, "%s must not be NULL", nm[t]);
    if (!aligned16(ptr[t])) return fail(SIQ_ERR_ALIGNMENT, "%s is not 16-byte aligned", nm[t]);
    // 16-byte steps: 8 bf16 elements, or 4 fp32 elements for fp32 cos / sin
    const int64_t step = (cs_dtype == SIQ_DTYPE_FP32 && (t == 2 || t == 3)) ? 4 : 8;
    for (int j = 0; j < count[t]; ++j) {
      const int64_t v = st[first[t] + j];
      if (v < 0 || v % step)
        return fail(SIQ_ERR_ALIGNMENT, "%s stride %d (%lld) must be a non-negative multiple of %lld elements", nm[t],
                    j, (long long)v, (long long)step);
    }
  }
  auto ten = [&](int t) {
    siq::RopeTensor r;
    r.p = static_cast<siq::bf16*>(const_cast<void*>(ptr[t]));
    r.sb = st[first[t]];
    r.ss = st[first[t] + 1];
    r.sh = count[t] == 3 ? st[first[t] + 2] : 0;
    return r;
  };
  siq::RopeArgs a{};
  a.x[0] = ten(0);
  a.x[1] = ten(1);
  a.cos = ten(2);
  a.sin = ten(3);
  a.y[0] = ten(4);
  a.y[1] = ten(5);
  a.batch = batch;
  a.seqlen = seqlen;
  a.hq = hq;
  a.hkv = hkv;
  a.d = d;
  a.cs_f32 = cs_dtype == SIQ_DTYPE_FP32 ? 1 : 0;
  const hipError_t e = siq::launch_rope(a, backward, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(SIQ_ERR_LAUNCH, "rope launch failed: %s", hipGetErrorString(e));
  return ok();
}

}  // namespace

extern "C" {

int siq_rope_fwd(const void* q, const void* k, const void* cos, const void* sin, void* q_embed, void* k_embed,
                 int64_t batch, int64_t seqlen, int hq, int hkv, int head_dim, const int64_t* strides, void* stream) {
  return rope_call(false, q, k, cos, sin, q_embed, k_embed, batch, seqlen, hq, hkv, head_dim, strides, stream);
}

int siq_rope_bwd(const void* dq_embed, const void* dk_embed, const void* cos, const void* sin, void* dq, void* dk,
                 int64_t batch, int64_t seqlen, int hq, int hkv, int head_dim, const int64_t* strides, void* stream) {
  return rope_call(true, dq_embed, dk_embed, cos, sin, dq, dk, batch, seqlen, hq, hkv, head_dim, strides, stream);
}

int siq_rope_fwd_ex(const void* q, const void* k, const void* cos, const void* sin, void* q_embed, void* k_embed,
                    int64_t batch, int64_t seqlen, int hq, int hkv, int head_dim, const int64_t* strides,
                    int cs_dtype, void* stream) {
  return rope_call(false, q, k, cos, sin, q_embed, k_embed, batch, seqlen, hq, hkv, head_dim, strides, stream,
                   cs_dtype);
}

int siq_rope_bwd_ex(const void* dq_embed, const void* dk_embed, const void* cos, const void* sin, void* dq, void* dk,
                    int64_t batch, int64_t seqlen, int hq, int hkv, int head_dim, const int64_t* strides,
                    int cs_dtype, void* stream) {
  return rope_call(true, dq_embed, dk_embed, cos, sin, dq, dk, batch, seqlen, hq, hkv, head_dim, strides, stream,
                   cs_dtype);
}

}  // extern "C"

namespace {

// Geometry checks shared by the projector entry points.
int check_proj(int64_t batch, int64_t side, int64_t dv, int r, int64_t n) {
  if (batch < 0) return fail(SIQ_ERR_INVALID_ARGUMENT, "batch must be >= 0");
  if (side <= 0 || r <= 0) return fail(SIQ_ERR_INVALID_ARGUMENT, "side and factor must be positive");
  if (side % r != 0)
    return fail(SIQ_ERR_INVALID_ARGUMENT, "side %lld is not divisible by the pixel-shuffle factor %d", (long long)side, r);
  if (dv <= 0 || dv % 64 != 0) return fail(SIQ_ERR_UNSUPPORTED, "vision_dim %lld must be a positive multiple of 64", (long long)dv);
  if (n <= 0 || n % 8 != 0) return fail(SIQ_ERR_UNSUPPORTED, "out_features %lld must be a positive multiple of 8", (long long)n);
  const int64_t k = (int64_t)r * r * dv, m = batch * (side / r) * (side / r);
  if (batch * side * side * dv >= (int64_t(1) << 31) || m >= (int64_t(1) << 24) || k * n >= (int64_t(1) << 31) ||
      m * n >= (int64_t(1) << 31))
    return fail(SIQ_ERR_INVALID_ARGUMENT, "projector sizes too large (x, y and weight must each hold < 2^31 elements, "
                "tokens < 2^24)");
  return SIQ_OK;
}

}  // namespace

extern "C" {

size_t siq_proj_workspace_bytes(int64_t batch, int64_t side, int64_t vision_dim, int factor, int64_t out_features) {
  if (check_proj(batch, side, vision_dim, factor, out_features) != SIQ_OK) return 0;
  return siq::proj_workspace_bytes(batch, side, vision_dim, factor, out_features);
}

int siq_proj_fwd(const void* x, const void* weight, void* y, int64_t batch, int64_t side, int64_t vision_dim,
                 int factor, int64_t out_features, void* ws, size_t ws_bytes, void* stream) {
  int rc = check_proj(batch, side, vision_dim, factor, out_features);
  if (rc) return rc;
  if (weight == nullptr || !aligned16(weight)) return fail(SIQ_ERR_ALIGNMENT, "weight must be non-NULL and 16-byte aligned");
  if (batch == 0) return ok();
  if (x == nullptr || y == nullptr) return fail(SIQ_ERR_INVALID_ARGUMENT, "x and y must not be NULL");
  if (!aligned16(x) || !aligned16(y)) return fail(SIQ_ERR_ALIGNMENT, "x / y not 16-byte aligned");
  const size_t need = siq::proj_workspace_bytes(batch, side, vision_dim, factor, out_features);
  if (need > 0 && (ws == nullptr || ws_bytes < need || !aligned16(ws)))
    return fail(SIQ_ERR_WORKSPACE, "workspace needs %zu bytes (16-byte aligned), got %zu", need, ws_bytes);
  siq::ProjArgs a{};
  a.x = static_cast<const siq::bf16*>(x);
  a.weight = static_cast<const siq::bf16*>(weight);
  a.y = static_cast<siq::bf16*>(y);
  a.part = static_cast<float*>(ws);
  a.batch = batch;
  a.side = side;
  a.dv = vision_dim;
  a.n = out_features;
  a.r = factor;
  const hipError_t e = siq::proj_fwd(a, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(SIQ_ERR_LAUNCH, "projector forward launch failed: %s", hipGetErrorString(e));
  return ok();
}

int siq_proj_bwd(const void* x, const void* weight, const void* dy, void* dx, void* dweight, int64_t batch,
                 int64_t side, int64_t vision_dim, int factor, int64_t out_features, void* ws, size_t ws_bytes,
                 void* stream) {
  int rc = check_proj(batch, side, vision_dim, factor, out_features);
  if (rc) return rc;
  if (weight == nullptr || !aligned16(weight)) return fail(SIQ_ERR_ALIGNMENT, "weight must be non-NULL and 16-byte aligned");
  if (dweight != nullptr && !aligned16(dweight)) return fail(SIQ_ERR_ALIGNMENT, "dweight not 16-byte aligned");
  if (batch > 0) {
    if (x == nullptr || dy == nullptr) return fail(SIQ_ERR_INVALID_ARGUMENT, "x and dy must not be NULL");
    if (!aligned16(x) || !aligned16(dy) || (dx != nullptr && !aligned16(dx)))
      return fail(SIQ_ERR_ALIGNMENT, "x / dy / dx not 16-byte aligned");
    const size_t need = siq::proj_workspace_bytes(batch, side, vision_dim, factor, out_features);
    if (dweight != nullptr && need > 0 && (ws == nullptr || ws_bytes < need || !aligned16(ws)))
      return fail(SIQ_ERR_WORKSPACE, "workspace needs %zu bytes (16-byte aligned), got %zu", need, ws_bytes);
  }
  siq::ProjArgs a{};
  a.x = static_cast<const siq::bf16*>(x);
  a.weight = static_cast<const siq::bf16*>(weight);
  a.dy = static_cast<const siq::bf16*>(dy);
  a.dx = batch > 0 ? static_cast<siq::bf16*>(dx) : nullptr;
  a.dweight = static_cast<siq::bf16*>(dweight);
  a.part = static_cast<float*>(ws);
  a.batch = batch;
  a.side = side;
  a.dv = vision_dim;
  a.n = out_features;
  a.r = factor;
  const hipError_t e = siq::proj_bwd(a, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(SIQ_ERR_LAUNCH, "projector backward launch failed: %s", hipGetErrorString(e));
  return ok();
}

size_t siq_splice_workspace_bytes(int64_t n_tokens) {
  if (n_tokens < 0) return 0;
  return align256(sizeof(int32_t) * (size_t)(n_tokens > 0 ? n_tokens : 1));
}

int siq_splice_fwd(const int64_t* input_ids, int64_t n_tokens, const void* weight, int64_t vocab, int64_t hidden,
                   const void* vision, int64_t n_vision, int64_t image_token_id, void* out, int32_t* image_pos,
                   int64_t* counts, void* ws, size_t ws_bytes, void* stream) {
  if (n_tokens < 0 || n_vision < 0) return fail(SIQ_ERR_INVALID_ARGUMENT, "n_tokens and n_vision must be >= 0");
  if (n_tokens >= (int64_t(1) << 31) || n_vision >= (int64_t(1) << 31))
    return fail(SIQ_ERR_INVALID_ARGUMENT, "n_tokens and n_vision must be < 2^31");
  if (vocab <= 0 || hidden <= 0) return fail(SIQ_ERR_INVALID_ARGUMENT, "vocab and hidden must be positive");
  if (hidden % 8 != 0) return fail(SIQ_ERR_UNSUPPORTED, "hidden (%lld) must be a multiple of 8", (long long)hidden);
  if (counts == nullptr || (reinterpret_cast<uintptr_t>(counts) & 7u))
    return fail(SIQ_ERR_ALIGNMENT, "counts must be a non-NULL 8-byte aligned int64[2]");
  if (weight == nullptr || !aligned16(weight)) return fail(SIQ_ERR_ALIGNMENT, "weight must be non-NULL and 16-byte aligned");
  if (n_vision > 0 && (vision == nullptr || !aligned16(vision) || image_pos == nullptr))
    return fail(SIQ_ERR_INVALID_ARGUMENT, "vision (16-byte aligned) and image_pos must not be NULL");
  if (n_tokens > 0 && (input_ids == nullptr || out == nullptr || !aligned16(out)))
    return fail(SIQ_ERR_INVALID_ARGUMENT, "input_ids and out (16-byte aligned) must not be NULL");
  const size_t need = siq_splice_workspace_bytes(n_tokens);
  if (ws == nullptr || ws_bytes < need || !aligned16(ws))
    return fail(SIQ_ERR_WORKSPACE, "workspace needs %zu bytes (16-byte aligned), got %zu", need, ws_bytes);
  siq::SpliceArgs a{};
  a.ids = input_ids;
  a.weight = static_cast<const siq::bf16*>(weight);
  a.vision = static_cast<const siq::bf16*>(vision);
  a.out = static_cast<siq::bf16*>(out);
  a.rank = static_cast<int32_t*>(ws);
  a.n = n_tokens;
  a.vocab = vocab;
  a.hidden = hidden;
  a.n_vision = n_vision;
  a.image_id = image_token_id;
  const hipError_t e = siq::splice_fwd(a, image_pos, counts, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(SIQ_ERR_LAUNCH, "splice launch failed: %s", hipGetErrorString(e));
  return ok();
}

int siq_gather_rows(const void* src, const int32_t* rows, int64_t n, int64_t hidden, void* dst, void* stream) {
  if (n < 0 || n >= (int64_t(1) << 31)) return fail(SIQ_ERR_INVALID_ARGUMENT, "n must be in [0, 2^31)");
  if (hidden <= 0 || hidden % 8 != 0) return fail(SIQ_ERR_UNSUPPORTED, "hidden (%lld) must be a positive multiple of 8", (long long)hidden);
  if (n == 0) return ok();
  if (src == nullptr || rows == nullptr || dst == nullptr) return fail(SIQ_ERR_INVALID_ARGUMENT, "src, rows and dst must not be NULL");
  if (!aligned16(src) || !aligned16(dst)) return fail(SIQ_ERR_ALIGNMENT, "src / dst not 16-byte aligned");
  const hipError_t e = siq::gather_rows(static_cast<const siq::bf16*>(src), rows, n, hidden, static_cast<siq::bf16*>(dst),
                                        static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(SIQ_ERR_LAUNCH, "gather launch failed: %s", hipGetErrorString(e));
  return ok();
}

size_t siq_embedding_bwd_workspace_bytes(int64_t n_tokens, int64_t vocab) {
  if (n_tokens < 0 || vocab <= 0) return 0;
  return siq::embedding_bwd_workspace_bytes(n_tokens, vocab);
}

int siq_embedding_bwd(const void* grad, const int64_t* input_ids, int64_t n_tokens, int64_t vocab, int64_t hidden,
                      int dtype, int64_t skip_id0, int64_t skip_id1, void* dweight, void* ws, size_t ws_bytes,
                      void* stream) {
  if (n_tokens < 0 || n_tokens >= (int64_t(1) << 31)) return fail(SIQ_ERR_INVALID_ARGUMENT, "n_tokens must be in [0, 2^31)");
  if (vocab <= 0 || vocab >= (int64_t(1) << 31)) return fail(SIQ_ERR_INVALID_ARGUMENT, "vocab must be in [1, 2^31)");
  if (hidden <= 0 || hidden % 8 != 0)
    return fail(SIQ_ERR_UNSUPPORTED, "hidden (%lld) must be a positive multiple of 8", (long long)hidden);
  if (dtype != SIQ_DTYPE_BF16 && dtype != SIQ_DTYPE_FP32)
    return fail(SIQ_ERR_INVALID_ARGUMENT, "dtype must be SIQ_DTYPE_BF16 or SIQ_DTYPE_FP32");
  if (dweight == nullptr || !aligned16(dweight)) return fail(SIQ_ERR_ALIGNMENT, "dweight must be non-NULL and 16-byte aligned");
  if (n_tokens > 0 && (grad == nullptr || input_ids == nullptr || !aligned16(grad)))
    return fail(SIQ_ERR_INVALID_ARGUMENT, "grad (16-byte aligned) and input_ids must not be NULL");
  const size_t need = siq_embedding_bwd_workspace_bytes(n_tokens, vocab);
  if (ws == nullptr || ws_bytes < need || !aligned16(ws))
    return fail(SIQ_ERR_WORKSPACE, "workspace needs %zu bytes (16-byte aligned), got %zu", need, ws_bytes);
  const hipError_t e = siq::embedding_bwd(grad, input_ids, n_tokens, vocab, hidden, dtype == SIQ_DTYPE_FP32, skip_id0,
                                          skip_id1, dweight, ws, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(SIQ_ERR_LAUNCH, "embedding backward launch failed: %s", hipGetErrorString(e));
  return ok();
}

int siq_scale_bf16_inplace(void* data, int64_t numel, const float* scalar, void* stream) {
  return siq_scale_bf16(data, data, numel, scalar, stream);
}

int siq_scale_bf16(const void* src, void* dst, int64_t numel, const float* scalar, void* stream) {
  if (numel < 0) return fail(SIQ_ERR_INVALID_ARGUMENT, "numel must be >= 0");
  if (numel == 0) return ok();
  if (src == nullptr || dst == nullptr || scalar == nullptr)
    return fail(SIQ_ERR_INVALID_ARGUMENT, "src, dst and scalar must not be NULL");
  if (!aligned16(src) || !aligned16(dst)) return fail(SIQ_ERR_ALIGNMENT, "src / dst not 16-byte aligned");
  const hipError_t e = siq::launch_scale_bf16(static_cast<const siq::bf16*>(src), static_cast<siq::bf16*>(dst), numel,
                                              scalar, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(SIQ_ERR_LAUNCH, "scale launch failed: %s", hipGetErrorString(e));
  return ok();
}

int siq_probe_clock(uint64_t* out, int64_t spin_ticks, void* stream) {
  if (out == nullptr || (reinterpret_cast<uintptr_t>(out) & 7u))
    return fail(SIQ_ERR_ALIGNMENT, "out must be a non-NULL 8-byte aligned uint64[2]");
  if (spin_ticks <= 0 || spin_ticks > 100000000)
    return fail(SIQ_ERR_INVALID_ARGUMENT, "spin_ticks must be in [1, 1e8] (ticks of 10 ns)");
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) !=
                                              hipSuccess)
    return fail(SIQ_ERR_LAUNCH, "cannot query the device");
  const hipError_t e = siq::launch_clock_probe(out, spin_ticks, cus > 0 ? cus : 1, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(SIQ_ERR_LAUNCH, "clock probe launch failed: %s", hipGetErrorString(e));
  return ok();
}

}  // extern "C"
