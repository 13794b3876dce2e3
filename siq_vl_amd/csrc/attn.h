// Internal (C++) interface between the C-ABI layer and the attention kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tiles.h"

namespace siq {

// Tile sizes shared by the scheduler and the kernels.
constexpr int kFwdBM = 128;    // q rows per forward unit (4 waves x 32) and per dQ workgroup
constexpr int kFwdBN = 64;     // kv rows per inner step of the forward / dQ loop
constexpr int kBwdBN = 128;    // kv rows per dK/dV work item (4 quarters of 32)
constexpr int kBwdBM = 64;     // q rows per step of the dK/dV loop (2 groups of 32)
constexpr int kSchedKeys = 2048;
// dK/dV load balance: a kv tile's steps (q block x q-head of the GQA group) run
// in one workgroup unless the tile is heavier than total / kSplitTarget steps;
// heavier tiles are cut into pieces whose fp32 partial sums are added, in
// piece order, by a small kernel after the dK/dV kernel.
constexpr int kSplitTarget = 256;
constexpr int kMinSplitSteps = 4;
// Pieces longer than this many steps amortise their fp32 partial sums, so they
// are cut twice as fine (piece length >= hkv total / (2 kSplitTarget)).
constexpr int kLongPiece = 256;
constexpr int kSplitSlots = 4 * kSplitTarget + 2;  // bound on sum(pieces x hkv) over split tiles
constexpr int kMaxSplitTiles = kSplitSlots / 2;    // a split tile has >= 2 pieces
constexpr int kXcds = 8;                           // MI355X: workgroup b runs on XCD b % 8

// One forward / dQ work unit: q tile t of sequence b (b < 0: idle), with the
// sequence's extents copied in, so a workgroup starts from one load of its
// entry rather than two dependent ones.
struct QTile {
  SeqInfo s;
  int b, t, pad0, pad1;
};
// One dK/dV work item: steps [s0, s1) of kv tile t of sequence b (extents in
// s; b < 0: idle); piece `piece` of np (np == 1: the whole tile, written
// directly as bf16).  Steps walk the q blocks downwards from the last one,
// each over the n_rep q-heads.  A piece of a split tile writes fp32 sums to
// slot (slot0 + piece) * hkv + hk.
struct KvItem {
  SeqInfo s;
  int b, t, s0, s1, piece, np, slot0, pad;
};
// A split tile, for the kernel that adds its pieces' partial sums.
struct SplitTile {
  int b, t, np, slot0;
};

// Block b of a launch runs on XCD b % 8.  Hands each XCD runs of G consecutive
// entries of a work list (a bijection on [0, n)), so that the workgroups
// resident on one XCD at the same time work on neighbouring entries and share
// their operands through that XCD's L2.  Entries past the last whole run of
// 8 G keep their index.
__device__ __forceinline__ int xcd_order(int b, int n, int G) {
  const int full = (n / (kXcds * G)) * (kXcds * G);
  if (b >= full) return b;
  const int x = b % kXcds, k = b / kXcds;  // k-th block dispatched to XCD x
  return ((k / G) * kXcds + x) * G + (k % G);
}

// Header of an attention plan (the schedule of one packed batch, reusable
// by every layer's forward and backward).  The scheduler writes it; each
// attention kernel compares it with its own arguments before using the plan
// and, on a mismatch, leaves its outputs alone and flags kStatusMismatch
// (a plan built for other sequences or heads could otherwise send a kernel
// outside its tensors).  status_q / status_kv: bits set by the scheduler's two
// blocks (kStatusOverflow: a work list or the split slots would not hold the
// schedule -- impossible by the bounds below, kept as a tripwire).
constexpr int kPlanMagic = 0x51504c4e;  // "QPLN"
constexpr int kStatusOverflow = 1;
constexpr int kStatusMismatch = 2;
struct PlanHeader {
  int64_t total_q, total_k;
  int magic, batch, n_rep, hkv, causal, has_kv;
  int status_q, status_kv, status_use, pad;
};

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
  float* lse2;       // [hq, lse_head] LSE * log2(e) (backward workspace)
  float* dq_acc;     // [total_q, hq, D] fp32 dQ sums of the atomic backward; nullptr: deterministic
  const SeqInfo* seq;
  const QTile* qtiles;       // q tiles ordered by decreasing work; b < 0 = idle
  const KvItem* kvitems;     // dK/dV work items (longest sequences first); b < 0 = idle
  float* dkv_part;           // [kSplitSlots][2][kBwdBN][D] fp32 partial dK / dV of split tiles
  const SplitTile* splits;   // [kMaxSplitTiles] split tiles
  const int* nsplit;         // number of split tiles
  PlanHeader* plan;          // the plan these lists belong to
  // Rotary embedding of q inside the kernels (rcos != nullptr): cos / sin rows
  // per token ([total_q, D] bf16, D contiguous, token strides rc_tok /
  // rs_tok).  The forward reads q before rotation, rotates it in registers and
  // writes the rotated rows to qe (for the backward); the dQ kernel reads the
  // rotated q and writes dq through the rotation's backward.
  const bf16* rcos;
  const bf16* rsin;
  int64_t rc_tok, rs_tok;
  bf16* qe;
  int64_t qe_tok, qe_head;
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
// Upper bound on the number of dK/dV work items (tiles plus extra pieces).
inline int64_t kv_item_cap(int64_t total_k, int batch) {
  return tile_cap(total_k, batch, kBwdBN) + 2 * kSplitTarget + 1;
}

// The plan header, read whole.  A kernel issues this load before the load of
// its work-list entry and waits for both together (one memory round trip at
// the start of every workgroup instead of three dependent ones).
__device__ __forceinline__ PlanHeader plan_header(const AttnParams& p) { return *p.plan; }

// True when the plan was built for these arguments; the caller returns on
// false.  Every field is compared (no short-circuit, so no field waits on
// another's test).  A mismatch is recorded in the plan's status_use.
__device__ __forceinline__ bool plan_header_ok(const PlanHeader& h, const AttnParams& p, bool causal, bool need_kv) {
  const bool ok = (h.magic == kPlanMagic) & (h.total_q == p.total_q) & (h.total_k == p.total_k) &
                  (h.batch == p.batch) & (h.n_rep == p.n_rep) & (h.hkv == p.hkv) & (h.causal == (causal ? 1 : 0)) &
                  (!need_kv | (h.has_kv != 0));
  if (!ok && threadIdx.x == 0) atomicOr(&p.plan->status_use, kStatusMismatch);
  return ok;
}

__device__ __forceinline__ bool plan_matches(const AttnParams& p, bool causal, bool need_kv) {
  return plan_header_ok(plan_header(p), p, causal, need_kv);
}

hipError_t launch_schedule(const int* cu_q, const int* cu_k, int batch, int64_t total_q, int64_t total_k,
                           int causal, int n_rep, int hkv, PlanHeader* plan, SeqInfo* seq, QTile* qtiles, int qrows,
                           int qcap, KvItem* kvitems, int kvcap, int* seqbuf, SplitTile* splits, int* nsplit,
                           int* qfirst, hipStream_t stream);
hipError_t launch_attn_fwd(const AttnParams& p, int d, int causal, int qcap, hipStream_t stream);
hipError_t launch_attn_bwd(const AttnParams& p, int d, int causal, int qcap, int kvcap, hipStream_t stream);

}  // namespace siq
