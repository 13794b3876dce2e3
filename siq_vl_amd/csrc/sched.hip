// Device-side tile scheduler for varlen attention.
//
// Packing puts sequences of very different lengths in one batch (a 16k-token
// sequence next to 81-token image blocks).  Launching one workgroup per
// (sequence, tile) in cu_seqlens order would leave the heaviest causal tiles
// for last.  This kernel reads cu_seqlens on the device (no host sync), clamps
// every extent to [0, total) so a malformed cu_seqlens can never drive a kernel
// out of bounds, and writes the tile list ordered by decreasing work with a
// counting sort.  The attention kernels then map blockIdx.x -> tile.
//
// Block 0 builds the q-tile list (forward and dQ kernels), block 1 the kv-tile
// list (dK/dV kernel).  Work keys are in units of 64 rows of the other side.
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

// Rows of the other side that tile t touches (causal alignment is bottom-right:
// q row i sees k rows <= i + (Lk - Lq)).
__device__ __forceinline__ int tile_key(const SeqInfo& s, int t, int mode, int causal) {
  const int off = s.k_len - s.q_len;
  int n;
  if (mode == 0) {
    n = s.k_len;
    if (causal) n = max(0, min(s.k_len, (t + 1) * kFwdBM + off));
  } else {
    n = s.q_len;
    if (causal) n = max(0, s.q_len - max(0, t * kBwdBN - off));
  }
  const int key = (n + 63) >> 6;
  return key < kSchedKeys - 1 ? key : kSchedKeys - 1;
}

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

__global__ __launch_bounds__(kSchedThreads) void schedule_kernel(const int* __restrict__ cu_q,
                                                                 const int* __restrict__ cu_k, int batch,
                                                                 int64_t total_q, int64_t total_k, int causal,
                                                                 SeqInfo* __restrict__ seq,
                                                                 int2* __restrict__ qtiles, int qcap,
                                                                 int2* __restrict__ kvtiles, int kvcap) {
  __shared__ int hist[kSchedKeys];
  __shared__ int wsum[kSchedThreads / 64 + 1];
  const int mode = blockIdx.x;
  int2* tiles = mode == 0 ? qtiles : kvtiles;
  const int cap = mode == 0 ? qcap : kvcap;
  const int rows = mode == 0 ? kFwdBM : kBwdBN;
  if (tiles == nullptr) return;
  const int tid = threadIdx.x;

  for (int i = tid; i < kSchedKeys; i += kSchedThreads) hist[i] = 0;
  __syncthreads();
  for (int b = tid; b < batch; b += kSchedThreads) {
    const SeqInfo s = seq_extent(cu_q, cu_k, b, total_q, total_k);
    if (mode == 0) seq[b] = s;
    const int len = mode == 0 ? s.q_len : s.k_len;
    const int nt = (len + rows - 1) / rows;
    for (int t = 0; t < nt; ++t) atomicAdd(&hist[kSchedKeys - 1 - tile_key(s, t, mode, causal)], 1);
  }
  __syncthreads();
  const int total = block_exclusive_scan(hist, kSchedKeys, wsum);
  for (int b = tid; b < batch; b += kSchedThreads) {
    const SeqInfo s = seq_extent(cu_q, cu_k, b, total_q, total_k);
    const int len = mode == 0 ? s.q_len : s.k_len;
    const int nt = (len + rows - 1) / rows;
    for (int t = 0; t < nt; ++t) {
      const int pos = atomicAdd(&hist[kSchedKeys - 1 - tile_key(s, t, mode, causal)], 1);
      if (pos < cap) tiles[pos] = make_int2(b, t);
    }
  }
  for (int i = total + tid; i < cap; i += kSchedThreads) tiles[i] = make_int2(-1, -1);
}

}  // namespace

hipError_t launch_schedule(const int* cu_q, const int* cu_k, int batch, int64_t total_q, int64_t total_k,
                           int causal, SeqInfo* seq, int2* qtiles, int qcap, int2* kvtiles, int kvcap,
                           hipStream_t stream) {
  const int blocks = kvtiles != nullptr ? 2 : 1;
  hipLaunchKernelGGL(schedule_kernel, dim3(blocks), dim3(kSchedThreads), 0, stream, cu_q, cu_k, batch, total_q,
                     total_k, causal, seq, qtiles, qcap, kvtiles, kvcap);
  return hipGetLastError();
}

}  // namespace siq
