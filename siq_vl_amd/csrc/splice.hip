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
//  * splice_fused_kernel (up to kFusedMaxTokens tokens): the whole forward
//    in one launch, each workgroup counting the image tokens before its own
//    (below); longer batches run the next two kernels;
//  * splice_scan_kernel (one workgroup; per round 16 chunks of 1024 tokens
//    loaded at once, wave ballots, one prefix over the 256 (chunk, wave)
//    counts): exclusive prefix count of image
//    tokens in token order -> rank[p] for every token, image_pos[r] = p for
//    image slot r < n_vision, counts[0] = image tokens found, counts[1] = ids
//    outside [0, vocab) (their rows are written as zeros; the reference's
//    embedding would raise a device-side assert);
//  * splice_gather_kernel: one wave per token row, 16 bytes per lane per
//    step (HBM-bound: read and write hidden * 2 bytes per token);
//  * gather_rows_kernel: dst[i] = src[rows[i]] (the backward's vision rows;
//    rows[i] < 0 gives a zero row);
//  * emb_prep_kernel, emb_sum_kernel: the embedding table's gradient
//    (below).
#include <algorithm>

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
  // fewer image tokens than vision rows (the count check fails, maybe only
  // later on the host): the slots no token filled hold -1, which the row
  // gather of the backward turns into zero rows instead of reading garbage
  for (long long r = carry_sh + tid; r < n_vision; r += kScanThreads) image_pos[r] = -1;
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

// One-kernel splice for batches of up to kFusedMaxTokens tokens (the scan
// kernel above is a single workgroup, and waiting for it costs more than
// counting again).  Workgroup w owns tokens [w R, w R + R), R = rpw (a
// multiple of 64): it counts the image tokens before its first token itself
// (every thread reads kFusedUnroll ids of the earlier tokens at a time; at
// most kFusedMaxTokens * 8 bytes, served by L2), ranks its own image tokens
// with wave ballots, records each row's source in LDS, then its eight waves
// copy the rows, kFusedUnroll 16-byte chunks per lane in flight.  The last
// workgroup reads every id, so it writes counts and fills the vision slots
// no token took with -1.  Outputs are those of splice_scan_kernel +
// splice_gather_kernel, bit for bit (the rank workspace is not used).
constexpr int kFusedThreads = 512;
constexpr int kFusedBlocks = 256;
constexpr int64_t kFusedMaxTokens = 32768;
constexpr int kFusedMaxRows = (int)(kFusedMaxTokens / kFusedBlocks);
constexpr int kFusedUnroll = 8;
static_assert(kFusedMaxRows % 64 == 0, "rows per workgroup come in waves of 64");

__global__ __launch_bounds__(kFusedThreads) void splice_fused_kernel(const SpliceArgs a, int32_t* __restrict__ image_pos,
                                                                     int64_t* __restrict__ counts, int rpw) {
  constexpr int NWV = kFusedThreads / 64;
  __shared__ const bf16* src_sh[kFusedMaxRows];
  __shared__ long long red_sh[2][NWV];
  __shared__ long long found_sh;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int64_t r0 = (int64_t)blockIdx.x * rpw;
  const bool last = blockIdx.x == gridDim.x - 1;
  const int64_t image_id = a.image_id, vocab = a.vocab;

  // image tokens (and, in the last workgroup, ids outside [0, vocab)) before r0
  long long img = 0, bad = 0;
  for (int64_t base = tid; base < r0; base += (int64_t)kFusedThreads * kFusedUnroll) {
    int64_t v[kFusedUnroll];
#pragma unroll
    for (int u = 0; u < kFusedUnroll; ++u) {
      const int64_t p = base + (int64_t)u * kFusedThreads;
      v[u] = p < r0 ? a.ids[p] : image_id - 1;
    }
#pragma unroll
    for (int u = 0; u < kFusedUnroll; ++u) {
      const bool inb = base + (int64_t)u * kFusedThreads < r0;
      img += (inb && v[u] == image_id) ? 1 : 0;
      bad += (inb && v[u] != image_id && (v[u] < 0 || v[u] >= vocab)) ? 1 : 0;
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    img += __shfl_xor(img, o);
    bad += __shfl_xor(bad, o);
  }
  if (lane == 0) {
    red_sh[0][wv] = img;
    red_sh[1][wv] = bad;
  }
  __syncthreads();
  if (wv == 0) {
    long long carry = 0, badt = 0;
#pragma unroll
    for (int w = 0; w < NWV; ++w) {
      carry += red_sh[0][w];
      badt += red_sh[1][w];
    }
    // this workgroup's tokens, 64 at a time in token order
    const uint64_t below = lane ? (~0ull >> (64 - lane)) : 0ull;
    for (int j = 0; j < rpw; j += 64) {
      const int64_t p = r0 + j + lane;
      const bool inb = p < a.n;
      const int64_t v = inb ? a.ids[p] : image_id - 1;
      const bool isimg = inb && v == image_id;
      const uint64_t m = __ballot(isimg);
      const long long r = carry + __popcll(m & below);
      const bf16* src = nullptr;
      if (isimg) {
        if (r < a.n_vision) {
          src = a.vision + r * a.hidden;
          image_pos[r] = (int32_t)p;
        }
      } else if (v >= 0 && v < vocab) {
        src = a.weight + v * a.hidden;
      }
      src_sh[j + lane] = src;
      carry += __popcll(m);
      badt += __popcll(__ballot(inb && !isimg && (v < 0 || v >= vocab)));
    }
    if (last && lane == 0) {
      counts[0] = carry;
      counts[1] = badt;
      found_sh = carry;
    }
  }
  __syncthreads();
  if (last) {
    for (long long r = found_sh + tid; r < a.n_vision; r += kFusedThreads) image_pos[r] = -1;
  }

  // rows: wave wv copies rows wv, wv + NWV, ... of the workgroup's rows that exist, as one list of
  // (row, 16-byte chunk) pairs
  const int nvec = (int)(a.hidden / 8);
  const int nrows = (int)min<int64_t>(rpw, a.n - r0);
  const int my_rows = nrows > wv ? (nrows - wv + NWV - 1) / NWV : 0;
  const int total = my_rows * nvec;
  for (int base = lane; base < total; base += 64 * kFusedUnroll) {
    bf16x8 x[kFusedUnroll];
#pragma unroll
    for (int u = 0; u < kFusedUnroll; ++u) {
      const int idx = base + 64 * u;
      if (idx < total) {
        const int k = idx / nvec, c = idx - k * nvec;
        const bf16* src = src_sh[wv + NWV * k];
        x[u] = src ? ld_bf16x8(src + 8 * c) : zero_bf16x8();
      }
    }
#pragma unroll
    for (int u = 0; u < kFusedUnroll; ++u) {
      const int idx = base + 64 * u;
      if (idx < total) {
        const int k = idx / nvec, c = idx - k * nvec;
        st_bf16x8(a.out + (r0 + wv + NWV * k) * a.hidden + 8 * c, x[u]);
      }
    }
  }
}

__global__ __launch_bounds__(256) void gather_rows_kernel(const bf16* __restrict__ src, const int32_t* __restrict__ rows,
                                                          int64_t n, int64_t hidden, bf16* __restrict__ dst) {
  const int lane = threadIdx.x & 63;
  const int64_t nvec = hidden / 8;
  for (int64_t i = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); i < n; i += (int64_t)gridDim.x * 4) {
    const int32_t r = rows[i];
    const bf16* s = src + (int64_t)r * hidden;
    bf16* d = dst + i * hidden;
    for (int64_t c = lane; c < nvec; c += 64) st_bf16x8(d + 8 * c, r >= 0 ? ld_bf16x8(s + 8 * c) : zero_bf16x8());
  }
}

// ---------------------------------------------------------------- embedding-table gradient
// dW[v] = sum of grad[p] over the tokens p with ids[p] == v, for ids in
// [0, vocab) other than the skipped ones (the image token, whose rows the
// splice overwrote, and the table's padding index); rows that no token
// reaches are zero.  The sum runs in fp32 in the order of torch's sorted
// embedding backward (aten/src/ATen/native/cuda/EmbeddingBackwardKernel.cu:
// the ids sorted stably, so each id's tokens in position order, summed in
// partial sums of at most kRowsPerPartial rows that are then added in order)
// and is rounded to the table's dtype once.
//
//  * emb_prep_kernel: one workgroup per chunk of kEmbChunk tokens clears the
//    chunk's run table, sorts the 64-bit keys (id << 32 | position in the
//    chunk; skipped and invalid ids get all-ones keys, which sort last) with
//    a bitonic network in LDS, then records each id's run [begin, end) in the
//    run table (begin = end = 0: no run); the launch's other workgroups zero
//    the table gradient meanwhile (the HBM-bound bulk of the work: one
//    streaming pass of 16-byte stores);
//  * emb_sum_kernel: one wave per sorted key; the wave of the first key of an
//    id in the first chunk that holds the id sums the id's runs over that
//    chunk and the later ones (chunks are in position order, so the
//    concatenation is the stable order) and writes the row; every other wave
//    returns at once.
constexpr int kEmbChunk = 2048;  // two keys per thread of a 1024-thread workgroup
constexpr int kRowsPerPartial = 10;

// Blocks [0, nch) sort one chunk each (after clearing that chunk's run
// table); the other blocks zero the table gradient meanwhile, so that the
// sort, which keeps only nch CUs busy, hides under the HBM-bound clear.
static_assert(kEmbChunk == 2 * 1024, "one compare-exchange pair per thread and stage");
__global__ __launch_bounds__(1024) void emb_prep_kernel(const int64_t* __restrict__ ids, int64_t n, int64_t vocab,
                                                        int64_t skip0, int64_t skip1, uint64_t* __restrict__ keys,
                                                        int2* __restrict__ seg, int nch, u32x4* __restrict__ dw,
                                                        int64_t dw16) {
  __shared__ uint64_t sk[kEmbChunk];
  const u32x4 z = {0u, 0u, 0u, 0u};
  if ((int)blockIdx.x >= nch) {
    const int64_t stride = (int64_t)(gridDim.x - nch) * 1024;
    for (int64_t i = (int64_t)(blockIdx.x - nch) * 1024 + threadIdx.x; i < dw16; i += stride) dw[i] = z;
    return;
  }
  int2* sg = seg + (int64_t)blockIdx.x * vocab;
  for (int64_t i = threadIdx.x; i < vocab; i += blockDim.x) sg[i] = make_int2(0, 0);
  const int64_t base = (int64_t)blockIdx.x * kEmbChunk;
  const int len = (int)min<int64_t>(kEmbChunk, n - base);
  int np2 = 64;
  while (np2 < len) np2 <<= 1;
  for (int i = threadIdx.x; i < np2; i += blockDim.x) {
    uint64_t k = ~0ull;
    if (i < len) {
      const int64_t v = ids[base + i];
      if (v >= 0 && v < vocab && v != skip0 && v != skip1) k = ((uint64_t)v << 32) | (uint32_t)i;
    }
    sk[i] = k;
  }
  __syncthreads();  // also orders the run table's clearing before its writes below
  // bitonic network: in each stage thread t owns the pair (i, i + j), i = t with a zero bit inserted at j
  const int t = threadIdx.x;
  for (int k = 2; k <= np2; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      const int i = 2 * t - (t & (j - 1));
      if (i + j < np2) {
        const uint64_t a = sk[i], b = sk[i + j];
        if ((a > b) == ((i & k) == 0)) {
          sk[i] = b;
          sk[i + j] = a;
        }
      }
      __syncthreads();
    }
  }
  // every key slot of the chunk is written (all-ones past the tokens), so the sum kernel reads no stale key
  uint64_t* kout = keys + base;
  for (int i = threadIdx.x; i < kEmbChunk; i += blockDim.x) {
    const uint64_t key = i < np2 ? sk[i] : ~0ull;
    kout[i] = key;
    if (key == ~0ull) continue;
    const uint32_t v = (uint32_t)(key >> 32);
    if (i == 0 || (uint32_t)(sk[i - 1] >> 32) != v) sg[v].x = i;
    if (i == len - 1 || (uint32_t)(sk[i + 1] >> 32) != v) sg[v].y = i + 1;
  }
}

template <typename T>
struct Vec16;
template <>
struct Vec16<bf16> {
  static constexpr int E = 8;
  __device__ static void load(const bf16* p, float (&x)[8]) {
    const bf16x8 v = ld_bf16x8(p);
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = (float)v[i];
  }
  __device__ static void store(bf16* p, const float (&x)[8]) {
    bf16x8 v;
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = (bf16)x[i];
    st_bf16x8(p, v);
  }
};
template <>
struct Vec16<float> {
  static constexpr int E = 4;
  __device__ static void load(const float* p, float (&x)[4]) {
    const f32x4 v = *reinterpret_cast<const f32x4*>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = v[i];
  }
  __device__ static void store(float* p, const float (&x)[4]) {
    *reinterpret_cast<f32x4*>(p) = f32x4{x[0], x[1], x[2], x[3]};
  }
};

// U 16-byte chunks of the row per lane and pass: every token's row is read
// once per pass, its U loads in flight together.
template <typename T>
__global__ __launch_bounds__(256) void emb_sum_kernel(const T* __restrict__ grad, const uint64_t* __restrict__ keys,
                                                      const int2* __restrict__ seg, int nchunks, int64_t vocab,
                                                      int64_t hidden, T* __restrict__ dw) {
  using V = Vec16<T>;
  constexpr int E = V::E, U = 4;
  const int lane = threadIdx.x & 63;
  const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (item >= (int64_t)nchunks * kEmbChunk) return;
  const int c = (int)(item / kEmbChunk), i = (int)(item % kEmbChunk);
  const uint64_t key = keys[item];
  if (key == ~0ull) return;
  const uint32_t v = (uint32_t)(key >> 32);
  if (i > 0 && (uint32_t)(keys[item - 1] >> 32) == v) return;  // not the first key of its id in this chunk
  // the id's runs in chunks c .. c + 63 (lane l: chunk c + l), one load per lane; an earlier chunk holding the
  // id means its wave writes the row
  for (int c0 = 0; c0 < c; c0 += 64) {
    const int cc = c0 + lane;
    int2 r = make_int2(0, 0);
    if (cc < c) r = seg[(int64_t)cc * vocab + v];
    if (__ballot(r.y > r.x)) return;
  }
  const int64_t nvec = hidden / E;
  for (int64_t p0 = 0; p0 < nvec; p0 += 64 * U) {
    float tot[U][E], part[U][E];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int e = 0; e < E; ++e) tot[u][e] = part[u][e] = 0.f;
    int cnt = 0;
    for (int g0 = c; g0 < nchunks; g0 += 64) {
      int2 mine = make_int2(0, 0);
      if (g0 + lane < nchunks) mine = seg[(int64_t)(g0 + lane) * vocab + v];
      const int ng = min(64, nchunks - g0);
      for (int q = 0; q < ng; ++q) {
        const int cc = g0 + q;
        const int rb = __shfl(mine.x, q), re = __shfl(mine.y, q);
        const uint64_t* kc = keys + (int64_t)cc * kEmbChunk;
        for (int t = rb; t < re; ++t) {
          const T* src = grad + ((int64_t)cc * kEmbChunk + (uint32_t)kc[t]) * hidden;
          float x[U][E];
#pragma unroll
          for (int u = 0; u < U; ++u) {
            const int64_t ch = p0 + 64 * u + lane;
            if (ch < nvec) {
              V::load(src + ch * E, x[u]);
            } else {
#pragma unroll
              for (int e = 0; e < E; ++e) x[u][e] = 0.f;
            }
          }
#pragma unroll
          for (int u = 0; u < U; ++u)
#pragma unroll
            for (int e = 0; e < E; ++e) part[u][e] += x[u][e];
          if (++cnt == kRowsPerPartial) {
#pragma unroll
            for (int u = 0; u < U; ++u)
#pragma unroll
              for (int e = 0; e < E; ++e) {
                tot[u][e] += part[u][e];
                part[u][e] = 0.f;
              }
            cnt = 0;
          }
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t ch = p0 + 64 * u + lane;
      if (ch >= nvec) continue;
      if (cnt > 0) {
#pragma unroll
        for (int e = 0; e < E; ++e) tot[u][e] += part[u][e];
      }
      V::store(dw + (int64_t)v * hidden + ch * E, tot[u]);
    }
  }
}

unsigned row_blocks(int64_t n) {
  int64_t b = (n + 3) / 4;
  if (b > 8192) b = 8192;
  return (unsigned)(b > 0 ? b : 1);
}

}  // namespace

hipError_t splice_fwd(const SpliceArgs& a, int32_t* image_pos, int64_t* counts, hipStream_t stream) {
  if (a.n > 0 && a.n <= kFusedMaxTokens) {
    // rows per workgroup: a multiple of 64 with at most kFusedBlocks workgroups
    const int64_t per = (a.n + kFusedBlocks - 1) / kFusedBlocks;
    const int rpw = (int)((per + 63) / 64 * 64);
    const unsigned blocks = (unsigned)((a.n + rpw - 1) / rpw);
    hipLaunchKernelGGL(splice_fused_kernel, dim3(blocks), dim3(kFusedThreads), 0, stream, a, image_pos, counts, rpw);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(splice_scan_kernel, dim3(1), dim3(kScanThreads), 0, stream, a.ids, a.n, a.vocab, a.image_id,
                     a.n_vision, a.rank, image_pos, counts);
  if (a.n > 0) hipLaunchKernelGGL(splice_gather_kernel, dim3(row_blocks(a.n)), dim3(256), 0, stream, a);
  return hipGetLastError();
}

size_t embedding_bwd_workspace_bytes(int64_t n, int64_t vocab) {
  const int64_t nch = n > 0 ? (n + kEmbChunk - 1) / kEmbChunk : 0;
  const size_t keys = (size_t)nch * kEmbChunk * sizeof(uint64_t);
  const size_t runs = ((size_t)nch * (size_t)vocab * sizeof(int2) + 15) & ~size_t(15);
  return ((keys + 255) & ~size_t(255)) + runs + 256;
}

hipError_t embedding_bwd(const void* grad, const int64_t* ids, int64_t n, int64_t vocab, int64_t hidden, bool fp32,
                         int64_t skip0, int64_t skip1, void* dw, void* ws, hipStream_t stream) {
  const int nch = n > 0 ? (int)((n + kEmbChunk - 1) / kEmbChunk) : 0;
  const size_t keys_bytes = ((size_t)nch * kEmbChunk * sizeof(uint64_t) + 255) & ~size_t(255);
  uint64_t* keys = static_cast<uint64_t*>(ws);
  int2* seg = reinterpret_cast<int2*>(static_cast<char*>(ws) + keys_bytes);
  const int64_t dw16 = vocab * hidden * (fp32 ? 4 : 2) / 16;  // hidden % 8 == 0
  const int clear_blocks = (int)std::min<int64_t>((dw16 + 1023) / 1024, 512);
  hipLaunchKernelGGL(emb_prep_kernel, dim3((unsigned)(nch + std::max(clear_blocks, 1))), dim3(1024), 0, stream, ids, n,
                     vocab, skip0, skip1, keys, seg, nch, static_cast<u32x4*>(dw), dw16);
  if (nch > 0) {
    const unsigned blocks = (unsigned)(((int64_t)nch * kEmbChunk + 3) / 4);
    if (fp32)
      hipLaunchKernelGGL(emb_sum_kernel<float>, dim3(blocks), dim3(256), 0, stream, static_cast<const float*>(grad),
                         keys, seg, nch, vocab, hidden, static_cast<float*>(dw));
    else
      hipLaunchKernelGGL(emb_sum_kernel<bf16>, dim3(blocks), dim3(256), 0, stream, static_cast<const bf16*>(grad), keys,
                         seg, nch, vocab, hidden, static_cast<bf16*>(dw));
  }
  return hipGetLastError();
}

hipError_t gather_rows(const bf16* src, const int32_t* rows, int64_t n, int64_t hidden, bf16* dst,
                       hipStream_t stream) {
  if (n > 0) hipLaunchKernelGGL(gather_rows_kernel, dim3(row_blocks(n)), dim3(256), 0, stream, src, rows, n, hidden, dst);
  return hipGetLastError();
}

}  // namespace siq
