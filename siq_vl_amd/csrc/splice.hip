// Vision-token splice fused with the embedding gather, for gfx950.
//
// Semantics: SiQ_VLForCausalLM.forward (siq_vl/model/modeling.py:252-270):
//   token_embeddings = embed_tokens(input_ids)                      (:253)
//   positions = (input_ids == image_token_index).nonzero()         (:257)
//   check #positions == #vision rows (ValueError otherwise)         (:259-267)
//   token_embeddings[positions] = vision_flat (row-major order)    (:269-270)
// Here each output row is written once, from the vision rows for image
// tokens (in row-major order of their positions) or from the embedding table
// otherwise: no embedding row is gathered only to be overwritten, and the
// count needs no nonzero() on the host.
//
// Kernels:
//  * splice_scan_kernel (one workgroup; per round 16 chunks of 1024 tokens
//    loaded at once, wave ballots, one prefix over the 256 (chunk, wave)
//    counts): exclusive prefix count of image
//    tokens in token order -> rank[p] for every token, image_pos[r] = p for
//    image slot r < n_vision, counts[0] = image tokens found, counts[1] = ids
//    outside [0, vocab) (their rows are written as zeros; the reference's
//    embedding would raise a device-side assert);
//  * splice_gather_kernel: one wave per token row, 16 bytes per lane per
//    step (HBM-bound: read and write hidden * 2 bytes per token);
//  * gather_rows_kernel: dst[i] = src[rows[i]] (the backward's vision rows).
#include "splice.h"

namespace siq {

namespace {

constexpr int kScanThreads = 1024;
constexpr int kPer = 16;  // chunks of kScanThreads tokens per round of the scan

__global__ __launch_bounds__(kScanThreads) void splice_scan_kernel(const int64_t* __restrict__ ids, int64_t n,
                                                                   int64_t vocab, int64_t image_id,
                                                                   int64_t n_vision, int32_t* __restrict__ rank,
                                                                   int32_t* __restrict__ image_pos,
                                                                   int64_t* __restrict__ counts) {
  constexpr int NWV = kScanThreads / 64;
  static_assert(kPer * NWV == 256, "one (chunk, wave) count per lane quarter");
  __shared__ int cnt_sh[kPer * NWV];  // image tokens of (chunk i, wave w) at i * NWV + w, in token order
  __shared__ long long carry_sh;
  __shared__ unsigned long long bad_sh;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const uint64_t below = lane ? (~0ull >> (64 - lane)) : 0ull;  // lanes before this one
  if (tid == 0) {
    carry_sh = 0;
    bad_sh = 0;
  }
  __syncthreads();
  unsigned long long bad = 0;
  // rounds of kPer chunks of kScanThreads tokens; token c0 + i kScanThreads + tid goes to this thread, so
  // every load and store of a chunk is one contiguous run per wave
  for (int64_t c0 = 0; c0 < n; c0 += (int64_t)kScanThreads * kPer) {
    int64_t v[kPer];
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int64_t pp = c0 + (int64_t)i * kScanThreads + tid;
      v[i] = pp < n ? ids[pp] : image_id - 1;
    }
    uint64_t m[kPer];
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const bool inb = c0 + (int64_t)i * kScanThreads + tid < n;
      const bool img = inb && v[i] == image_id;
      bad += (inb && !img && (v[i] < 0 || v[i] >= vocab)) ? 1 : 0;
      m[i] = __ballot(img);
      if (lane == 0) cnt_sh[i * NWV + wv] = __popcll(m[i]);
    }
    __syncthreads();
    // every wave forms the exclusive prefix of the 256 counts in token order: lane l holds entries 4l .. 4l + 3
    const int a0 = cnt_sh[4 * lane], a1 = cnt_sh[4 * lane + 1], a2 = cnt_sh[4 * lane + 2], a3 = cnt_sh[4 * lane + 3];
    const int lsum = a0 + a1 + a2 + a3;
    int incl = lsum;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(incl, o);
      if (lane >= o) incl += y;
    }
    const int total = __shfl(incl, 63);
    // entry i * NWV + wv sits in lane 4 i + wv / 4 at position wv % 4 (the same position for every i)
    const int k = wv & 3;
    const int mine = incl - lsum + (k > 0 ? a0 : 0) + (k > 1 ? a1 : 0) + (k > 2 ? a2 : 0);
    const long long carry = carry_sh;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int64_t pp = c0 + (int64_t)i * kScanThreads + tid;
      const long long r = carry + __shfl(mine, 4 * i + (wv >> 2)) + __popcll(m[i] & below);
      if (pp < n) {
        rank[pp] = (int32_t)r;
        if (v[i] == image_id && r < n_vision) image_pos[r] = (int32_t)pp;
      }
    }
    __syncthreads();
    if (tid == 0) carry_sh += total;
    __syncthreads();
  }
  atomicAdd(&bad_sh, bad);
  __syncthreads();
  if (tid == 0) {
    counts[0] = carry_sh;
    counts[1] = (int64_t)bad_sh;
  }
}

__global__ __launch_bounds__(256) void splice_gather_kernel(const SpliceArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t nvec = a.hidden / 8;
  for (int64_t p = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); p < a.n; p += (int64_t)gridDim.x * 4) {
    const int64_t v = a.ids[p];
    const bf16* src = nullptr;
    if (v == a.image_id) {
      const int64_t r = a.rank[p];
      if (r < a.n_vision) src = a.vision + r * a.hidden;
    } else if (v >= 0 && v < a.vocab) {
      src = a.weight + v * a.hidden;
    }
    bf16* dst = a.out + p * a.hidden;
    for (int64_t c = lane; c < nvec; c += 64) st_bf16x8(dst + 8 * c, src ? ld_bf16x8(src + 8 * c) : zero_bf16x8());
  }
}

__global__ __launch_bounds__(256) void gather_rows_kernel(const bf16* __restrict__ src, const int32_t* __restrict__ rows,
                                                          int64_t n, int64_t hidden, bf16* __restrict__ dst) {
  const int lane = threadIdx.x & 63;
  const int64_t nvec = hidden / 8;
  for (int64_t i = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); i < n; i += (int64_t)gridDim.x * 4) {
    const bf16* s = src + (int64_t)rows[i] * hidden;
    bf16* d = dst + i * hidden;
    for (int64_t c = lane; c < nvec; c += 64) st_bf16x8(d + 8 * c, ld_bf16x8(s + 8 * c));
  }
}

unsigned row_blocks(int64_t n) {
  int64_t b = (n + 3) / 4;
  if (b > 8192) b = 8192;
  return (unsigned)(b > 0 ? b : 1);
}

}  // namespace

hipError_t splice_fwd(const SpliceArgs& a, int32_t* image_pos, int64_t* counts, hipStream_t stream) {
  hipLaunchKernelGGL(splice_scan_kernel, dim3(1), dim3(kScanThreads), 0, stream, a.ids, a.n, a.vocab, a.image_id,
                     a.n_vision, a.rank, image_pos, counts);
  if (a.n > 0) hipLaunchKernelGGL(splice_gather_kernel, dim3(row_blocks(a.n)), dim3(256), 0, stream, a);
  return hipGetLastError();
}

hipError_t gather_rows(const bf16* src, const int32_t* rows, int64_t n, int64_t hidden, bf16* dst,
                       hipStream_t stream) {
  if (n > 0) hipLaunchKernelGGL(gather_rows_kernel, dim3(row_blocks(n)), dim3(256), 0, stream, src, rows, n, hidden, dst);
  return hipGetLastError();
}

}  // namespace siq
