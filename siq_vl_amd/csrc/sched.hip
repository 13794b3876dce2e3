// Device-side work scheduler for varlen attention.
//
// Packing puts sequences of very different lengths in one batch (a 16k-token
// sequence next to 81-token image blocks).  Launching one workgroup per
// (sequence, tile) in cu_seqlens order would leave the heaviest causal tiles
// for last.  This kernel reads cu_seqlens on the device (no host sync), clamps
// every extent to [0, total) so a malformed cu_seqlens can never drive a kernel
// out of bounds, and writes the work lists ordered by decreasing work with a
// counting sort.  The attention kernels then map blockIdx.x -> work.
//
// Both blocks read cu_seqlens once, into LDS.  Each sorts a flattened list of
// tiles (a prefix over the sequences' tile counts maps tile i back to its
// sequence), one tile per thread, so a long sequence is no serial loop.
// Block 0 builds the q-tile list of the forward and dQ kernels (tiles of
// `qrows` rows), heaviest first (work key: kv rows seen, in units of 64).  Block 1 builds the dK/dV
// work items: a kv tile has n_rep x (q blocks that can see it) steps; tiles
// with more than S steps are cut into pieces of at most S steps, so that the
// longest item stays near the average load of a CU: S = hkv steps /
// kSplitTarget (steps counted per kv-head), halved -- but not below
// kLongPiece -- when that exceeds kLongPiece, and at least kMinSplitSteps.
// The pieces are placed heaviest first, and split tiles are listed for the
// kernel that adds their partial sums.
//
// Bounds (why the work lists and split slots always hold the schedule):
//  * q tiles: sum_b ceil(L_b / qrows) <= total / qrows + batch < qcap;
//  * S >= hkv * steps / (2 kSplitTarget), so a split tile (w > S steps) has
//    np = ceil(w / S) < 2 w / S pieces: the extra items sum_split (np - 1) <
//    steps / S <= 2 kSplitTarget / hkv, and the slots sum_split np * hkv <
//    2 hkv steps / S <= 4 kSplitTarget;
// both fit kv_item_cap and kSplitSlots.  The scheduler still checks every
// placement and records an overflow in the plan header (status_q /
// status_kv) instead of writing past a list.
#include "attn.h"

namespace siq {

namespace {

constexpr int kSchedThreads = 1024;

__device__ __forceinline__ int clampi(int x, int lo, int hi) { return x < lo ? lo : (x > hi ? hi : x); }

__device__ __forceinline__ SeqInfo seq_extent(const int* cu_q, const int* cu_k, int b, int64_t total_q,
                                             int64_t total_k) {
  const int tq = (int)total_q, tk = (int)total_k;
  SeqInfo s;
  s.q_start = clampi(cu_q[b], 0, tq);
  s.q_len = clampi(cu_q[b + 1], s.q_start, tq) - s.q_start;
  s.k_start = clampi(cu_k[b], 0, tk);
  s.k_len = clampi(cu_k[b + 1], s.k_start, tk) - s.k_start;
  return s;
}

// kv rows that q tile t of `rows` rows sees (causal alignment is
// bottom-right: q row i sees k rows <= i + (Lk - Lq)), in units of 64.
__device__ __forceinline__ int q_tile_key(const SeqInfo& s, int t, int rows, int causal) {
  const int off = s.k_len - s.q_len;
  int n = s.k_len;
  if (causal) n = max(0, min(s.k_len, (t + 1) * rows + off));
  const int key = (n + 63) >> 6;
  return key < kSchedKeys - 1 ? key : kSchedKeys - 1;
}

// dK/dV steps of kv tile t: n_rep x the q blocks of kBwdBM rows that can see
// any of its rows (the dK/dV kernel walks exactly these, in this order).
__device__ __forceinline__ int kv_tile_steps(const SeqInfo& s, int t, int causal, int n_rep) {
  const int off = s.k_len - s.q_len;
  const int qb0 = causal ? max(0, t * kBwdBN - off) / kBwdBM : 0;
  const int nqb = s.q_len > qb0 * kBwdBM ? (s.q_len - qb0 * kBwdBM + kBwdBM - 1) / kBwdBM : 0;
  return nqb * n_rep;
}

__device__ __forceinline__ int clamp_key(int w) { return w < kSchedKeys - 1 ? w : kSchedKeys - 1; }

__device__ int block_exclusive_scan(int* buf, int n, int* wsum) {
  // buf[0..n) -> exclusive prefix sums; returns the total.  n <= 2 * kSchedThreads.
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int a = (2 * tid < n) ? buf[2 * tid] : 0;
  const int b = (2 * tid + 1 < n) ? buf[2 * tid + 1] : 0;
  int x = a + b;
  int incl = x;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(incl, o);
    if (lane >= o) incl += y;
  }
  if (lane == 63) wsum[wv] = incl;
  __syncthreads();
  if (tid == 0) {
    int run = 0;
    for (int i = 0; i < kSchedThreads / 64; ++i) {
      const int t = wsum[i];
      wsum[i] = run;
      run += t;
    }
    wsum[kSchedThreads / 64] = run;
  }
  __syncthreads();
  const int excl = wsum[wv] + incl - x;
  if (2 * tid < n) buf[2 * tid] = excl;
  if (2 * tid + 1 < n) buf[2 * tid + 1] = excl + a;
  const int total = wsum[kSchedThreads / 64];
  __syncthreads();
  return total;
}

// In-place exclusive scan of a global array of any length, 2 kSchedThreads
// entries at a time through `buf` (LDS); returns the total.
__device__ int scan_global(int* a, int n, int* buf, int* wsum) {
  const int tid = threadIdx.x;
  int carry = 0;
  for (int c0 = 0; c0 < n; c0 += 2 * kSchedThreads) {
    const int m = min(2 * kSchedThreads, n - c0);
    for (int i = tid; i < m; i += kSchedThreads) buf[i] = a[c0 + i];
    __syncthreads();
    const int tot = block_exclusive_scan(buf, m, wsum);
    for (int i = tid; i < m; i += kSchedThreads) a[c0 + i] = buf[i] + carry;
    carry += tot;
    __threadfence_block();
    __syncthreads();
  }
  return carry;
}

// Sequence extents of the batch, read from cu_seqlens once into LDS (batches
// of up to kSeqLds sequences; longer ones read them from global memory at each
// use).
constexpr int kSeqLds = 1024;

__global__ __launch_bounds__(kSchedThreads) void schedule_kernel(const int* __restrict__ cu_q,
                                                                 const int* __restrict__ cu_k, int batch,
                                                                 int64_t total_q, int64_t total_k, int causal,
                                                                 int n_rep, int hkv, PlanHeader* __restrict__ plan,
                                                                 SeqInfo* __restrict__ seq,
                                                                 QTile* __restrict__ qtiles, int qrows, int qcap,
                                                                 KvItem* __restrict__ kvitems, int kvcap,
                                                                 int* __restrict__ seqbuf,
                                                                 SplitTile* __restrict__ splits,
                                                                 int* __restrict__ nsplit, int* __restrict__ qfirst) {
  __shared__ int hist[kSchedKeys];
  __shared__ int wsum[kSchedThreads / 64 + 1];
  __shared__ long long wsteps[kSchedThreads / 64];
  __shared__ int nslot, nsplit_sh, status_sh;
  __shared__ SeqInfo seq_sh[kSeqLds];
  // [batch + 1] first flattened tile (q tiles in block 0, kv tiles in block 1)
  // of each sequence: in LDS when it fits, else in qfirst / seqbuf
  __shared__ int tfirst_sh[kSchedKeys];
  const int tid = threadIdx.x;
  const bool seq_lds = batch <= kSeqLds;

  for (int i = tid; i < kSchedKeys; i += kSchedThreads) hist[i] = 0;
  if (tid == 0) {
    nslot = 0;
    nsplit_sh = 0;
    status_sh = 0;
  }
  if (seq_lds) {
    for (int b = tid; b < batch; b += kSchedThreads) {
      const SeqInfo s = seq_extent(cu_q, cu_k, b, total_q, total_k);
      seq_sh[b] = s;
      if (blockIdx.x == 0) seq[b] = s;
    }
  } else if (blockIdx.x == 0) {
    for (int b = tid; b < batch; b += kSchedThreads) seq[b] = seq_extent(cu_q, cu_k, b, total_q, total_k);
  }
  __syncthreads();
  auto seq_of = [&](int b) { return seq_lds ? seq_sh[b] : seq_extent(cu_q, cu_k, b, total_q, total_k); };
  int* tfirst = batch + 1 <= kSchedKeys ? tfirst_sh : (blockIdx.x == 0 ? qfirst : seqbuf);
  // flattened tile i -> (sequence, tile): last b with tfirst[b] <= i
  auto locate = [&](int i, int& b, int& t) {
    int lo = 0, hi = batch - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (tfirst[mid] <= i) lo = mid; else hi = mid - 1;
    }
    b = lo;
    t = i - tfirst[lo];
  };

  if (blockIdx.x == 0) {
    // q tiles of the forward / dQ kernels, heaviest first: a counting sort over
    // the flattened tiles (one tile per thread and pass)
    for (int b = tid; b < batch; b += kSchedThreads) tfirst[b] = (seq_of(b).q_len + qrows - 1) / qrows;
    __threadfence_block();
    __syncthreads();
    const int ntiles = scan_global(tfirst, batch, hist, wsum);
    if (tid == 0) tfirst[batch] = ntiles;
    for (int i = tid; i < kSchedKeys; i += kSchedThreads) hist[i] = 0;
    __threadfence_block();
    __syncthreads();
    for (int i = tid; i < ntiles; i += kSchedThreads) {
      int b, t;
      locate(i, b, t);
      atomicAdd(&hist[kSchedKeys - 1 - q_tile_key(seq_of(b), t, qrows, causal)], 1);
    }
    __syncthreads();
    const int total = block_exclusive_scan(hist, kSchedKeys, wsum);
    for (int i = tid; i < ntiles; i += kSchedThreads) {
      int b, t;
      locate(i, b, t);
      const SeqInfo s = seq_of(b);
      const int pos = atomicAdd(&hist[kSchedKeys - 1 - q_tile_key(s, t, qrows, causal)], 1);
      if (pos < qcap) qtiles[pos] = QTile{s, b, t, 0, 0};
      else atomicOr(&status_sh, kStatusOverflow);
    }
    for (int i = total + tid; i < qcap; i += kSchedThreads) qtiles[i] = QTile{SeqInfo{0, 0, 0, 0}, -1, -1, 0, 0};
    __syncthreads();
    if (tid == 0) {
      PlanHeader h;
      h.total_q = total_q;
      h.total_k = total_k;
      h.magic = kPlanMagic;
      h.batch = batch;
      h.n_rep = n_rep;
      h.hkv = hkv;
      h.causal = causal ? 1 : 0;
      h.has_kv = kvitems != nullptr ? 1 : 0;
      h.status_q = status_sh;
      h.status_kv = 0;
      h.status_use = 0;
      h.pad = 0;
      if (kvitems != nullptr) {
        // block 1 owns status_kv: write every other field
        plan->total_q = h.total_q;
        plan->total_k = h.total_k;
        plan->magic = h.magic;
        plan->batch = h.batch;
        plan->n_rep = h.n_rep;
        plan->hkv = h.hkv;
        plan->causal = h.causal;
        plan->has_kv = h.has_kv;
        plan->status_q = h.status_q;
        plan->status_use = 0;
      } else {
        *plan = h;
      }
    }
    return;
  }

  // dK/dV work items.  1: kv tiles per sequence (prefix sums) and the total
  // number of steps (per kv-head).
  long long mine = 0;
  for (int b = tid; b < batch; b += kSchedThreads) {
    const SeqInfo s = seq_of(b);
    const int nt = (s.k_len + kBwdBN - 1) / kBwdBN;
    tfirst[b] = nt;
    for (int t = 0; t < nt; ++t) mine += kv_tile_steps(s, t, causal, n_rep);
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) mine += __shfl_xor(mine, o);
  if ((tid & 63) == 0) wsteps[tid >> 6] = mine;
  __threadfence_block();
  __syncthreads();
  long long steps = 0;
  for (int i = 0; i < kSchedThreads / 64; ++i) steps += wsteps[i];
  const int ntiles = scan_global(tfirst, batch, hist, wsum);
  if (tid == 0) tfirst[batch] = ntiles;
  for (int i = tid; i < kSchedKeys; i += kSchedThreads) hist[i] = 0;
  __threadfence_block();
  __syncthreads();
  // 2: piece length S >= hkv * steps / (2 kSplitTarget), so that the split
  // pieces (each kv-head counted) number at most 4 kSplitTarget and the items
  // at most 2 kSplitTarget more than the tiles: S = hkv * steps / kSplitTarget
  // (about a CU's share of the steps), halved when that is longer than
  // kLongPiece steps (long pieces amortise their partial sums, and finer ones
  // balance the CUs better).
  long long sl = (steps * hkv + kSplitTarget - 1) / kSplitTarget;
  if (sl > kLongPiece) {
    const long long half = (steps * hkv + 2 * kSplitTarget - 1) / (2 * kSplitTarget);
    sl = half > kLongPiece ? half : kLongPiece;
  }
  if (sl < kMinSplitSteps) sl = kMinSplitSteps;
  if (sl > (1 << 30)) sl = 1 << 30;
  const int S = (int)sl;
  // 3: counting sort of the pieces by steps, heaviest first
  for (int i = tid; i < ntiles; i += kSchedThreads) {
    int b, t;
    locate(i, b, t);
    const int w = kv_tile_steps(seq_of(b), t, causal, n_rep);
    const int np = w > S ? (w + S - 1) / S : 1;
    for (int pc = 0; pc < np; ++pc) atomicAdd(&hist[kSchedKeys - 1 - clamp_key(min(S, w - pc * S))], 1);
  }
  __syncthreads();
  const int total = block_exclusive_scan(hist, kSchedKeys, wsum);
  // 4: placement; split tiles get consecutive partial slots and a SplitTile entry
  for (int i = tid; i < ntiles; i += kSchedThreads) {
    int b, t;
    locate(i, b, t);
    const SeqInfo s = seq_of(b);
    const int w = kv_tile_steps(s, t, causal, n_rep);
    const int np = w > S ? (w + S - 1) / S : 1;
    int slot0 = -1;
    if (np > 1) {
      slot0 = atomicAdd(&nslot, np);
      const int k = atomicAdd(&nsplit_sh, 1);
      if (k < kMaxSplitTiles) splits[k] = SplitTile{b, t, np, slot0};
      if (k >= kMaxSplitTiles || (slot0 + np) * hkv > kSplitSlots) atomicOr(&status_sh, kStatusOverflow);
    }
    for (int pc = 0; pc < np; ++pc) {
      const int pos = atomicAdd(&hist[kSchedKeys - 1 - clamp_key(min(S, w - pc * S))], 1);
      KvItem it;
      it.s = s;
      it.b = b;
      it.t = t;
      it.s0 = pc * S;
      it.s1 = min(w, (pc + 1) * S);
      it.piece = pc;
      it.np = np;
      it.slot0 = slot0;
      it.pad = 0;
      if (pos < kvcap) kvitems[pos] = it;
      else atomicOr(&status_sh, kStatusOverflow);
    }
  }
  for (int i = total + tid; i < kvcap; i += kSchedThreads) {
    KvItem it{};
    it.b = -1;
    kvitems[i] = it;
  }
  __syncthreads();
  if (tid == 0) {
    *nsplit = min(nsplit_sh, kMaxSplitTiles);
    plan->status_kv = status_sh;
  }
}

}  // namespace

hipError_t launch_schedule(const int* cu_q, const int* cu_k, int batch, int64_t total_q, int64_t total_k,
                           int causal, int n_rep, int hkv, PlanHeader* plan, SeqInfo* seq, QTile* qtiles, int qrows,
                           int qcap, KvItem* kvitems, int kvcap, int* seqbuf, SplitTile* splits, int* nsplit,
                           int* qfirst, hipStream_t stream) {
  const int blocks = kvitems != nullptr ? 2 : 1;
  hipLaunchKernelGGL(schedule_kernel, dim3(blocks), dim3(kSchedThreads), 0, stream, cu_q, cu_k, batch, total_q,
                     total_k, causal, n_rep, hkv, plan, seq, qtiles, qrows, qcap, kvitems, kvcap, seqbuf, splits,
                     nsplit, qfirst);
  return hipGetLastError();
}

}  // namespace siq
