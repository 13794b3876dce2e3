// Fused lm_head linear + cross-entropy (forward and backward) for gfx950.
//
// Semantics: the reference computes logits = h W^T (transformers
// models/qwen2/modeling_qwen2.py:465), upcasts them to fp32 and calls
// F.cross_entropy(ignore_index=-100) with "mean" over non-ignored rows, or
// "sum" divided by num_items_in_batch (loss/loss_utils.py:32-71).  Here:
//   loss = sum_valid (lse_n - z_{n,y_n}) * inv_den,
//   dZ   = (softmax(z_n) - onehot(y_n)) * inv_den  (0 for ignored rows),
//   dH = dZ W,  dW = dZ^T H.
//
// Rows whose label is ignore_index (or out of range) contribute nothing: their
// dH row is zero and they add nothing to the loss or dW.  So the valid rows
// are first compacted, in order, into a contiguous buffer (padded with zero
// rows to the next 256-row tile), every stage below runs on the compacted rows
// only (each workgroup reads the valid count on the device and returns early
// past it), and dH rows are scattered back to their positions.
//
// Pipeline per chunk of C compacted rows (the only logits-sized buffer is one
// chunk's softmax numerators):
//  1. logits GEMM  Z^T = W H_c^T (MFMA, 256x256 tiles, K = hdim).  The epilogue
//     never writes z: per (token, 256-column vocab tile) it keeps the tile
//     max m and the sum s of exp(z - m) (the chunked-vocab logsumexp), the
//     label logit z_y, and E = exp(z - m) in bf16 (a value in (0, 1], so bf16
//     keeps full relative precision however large the logits are).
//  2. row pass: lse = M + log(sum_t s_t exp(m_t - M)), the row's loss, and E
//     rewritten in place as dZ = E * f_t - g * [v == y] with f_t = exp(m_t -
//     lse) * g (g = inv_den, or 0 for an ignored row): one multiply per element,
//     once for both gradient GEMMs.
//  3. dH GEMM  dH_c^T = W^T dZ_c^T (split over the vocab) and
//  4. dW GEMM  dW^T = H_c^T dZ_c.
// With several chunks dW accumulates over them: in dW itself (bf16) when the
// valid rows span two chunks, in an fp32 workspace when they span more;
// whether a chunk starts, continues or finishes that sum is decided on the
// device from the valid-row count, so chunks past the valid rows cost nothing.  Every
// reduction has a fixed order, so results are bitwise reproducible.
//
// Loss only (no gradient wanted, e.g. evaluation under torch.no_grad): the
// logits epilogue keeps its tile max / sum and z_y but stores no E, the row
// pass stops at the loss, and neither gradient GEMM runs.
#include "flce.h"
#include "gemm.h"

namespace siq {

namespace {

using namespace gemm;

constexpr int kVT = BI;  // vocab columns per logits tile

// ---------------------------------------------------------------- logits
struct LogitsArgs {
  GOp W, H;               // W [V, hdim], H = hidden rows of the chunk [nc, hdim]
  const int64_t* y;       // chunk labels
  bf16* E;                // [nc, V]
  float* mpart;           // [nc, nvt] tile max (log2 units)
  float* spart;           // [nc, nvt] tile sum of exp2(z2 - m)
  float* zy;              // [nc] label logit (natural units)
  const int64_t* nvalid;  // valid (compacted) rows in all chunks
  int64_t V, nc, nvt, c0;
  int nI, nJ;
  int store_e;            // 0: loss only, E is not needed
};

__global__ __launch_bounds__(NT) void flce_logits_kernel(const LogitsArgs p) {
  __shared__ __align__(16) bf16 smem[4 * SLAB];
  int ti, tj;
  if (!tile_of(p.nI, p.nJ, 4, ti, tj)) return;
  const int64_t i0 = (int64_t)ti * BI, j0 = (int64_t)tj * BJ;
  if (j0 >= *p.nvalid - p.c0) return;  // token tile holds no valid row
  f32x16 acc[4][2];
  gemm_core<true, true, true>(smem, p.W, p.H, i0, j0, 0, p.W.cols, acc);

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, h = lane >> 5, l32 = lane & 31;
  const int wi = w & 1, wj = w >> 1;
  float* red = reinterpret_cast<float*>(smem);  // [2][256]
  // accumulator (a, b, r) holds z for vocab row vbase + 32 a + 16 (r / 8) + (r % 8) and token column
  // j0 + 64 wj + 32 b + l32.  Only the last vocab tile has rows past V: masked there alone.
  const int64_t vbase = i0 + 128 * wi + 8 * h;
  if (i0 + BI > p.V) {
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (vbase + 32 * a + 16 * (r >> 3) + (r & 7) >= p.V) acc[a][b][r] = -INFINITY;
  }
  float mt[2];
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    float mx = -INFINITY;
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, acc[a][b][r]);
    // tile max in log2 units (scaling by log2 e > 0 commutes with the max)
    mx = wave_max_xor32(mx) * kLog2e;
    if (h == 0) red[wi * 256 + 64 * wj + 32 * b + l32] = mx;
  }
  __syncthreads();
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    const int col = 64 * wj + 32 * b + l32;
    mt[b] = fmaxf(red[col], red[256 + col]);
  }
  __syncthreads();
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    const int col = 64 * wj + 32 * b + l32;
    const int64_t tok = j0 + col;
    const bool tv = tok < p.nc;
    // the label logit: held by at most one lane of the workgroup, for one
    // vocab tile in ~600 -- located with one range test per token
    const int64_t rel64 = (tv ? p.y[tok] : -1) - vbase;
    const bool hit = rel64 >= 0 && rel64 < 128 && ((rel64 >> 3) & 1) == 0;
    if (__any(hit)) {
      const int rel = (int)rel64;
      float zsel = 0.f;
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (hit && rel == 32 * a + 16 * (r >> 3) + (r & 7)) zsel = acc[a][b][r];
      if (hit) p.zy[tok] = zsel;
    }
    const float m2 = mt[b];
    float sum = 0.f;
#pragma unroll
    for (int a = 0; a < 4; ++a) {
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const int64_t v0 = vbase + 32 * a + 16 * jj;
        bf16x8 e8;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float e = exp2f_fast(__builtin_fmaf(acc[a][b][8 * jj + i], kLog2e, -m2));
          sum += e;
          e8[i] = (bf16)e;
        }
        if (p.store_e && tv && v0 < p.V) st_bf16x8(p.E + tok * p.V + v0, e8);
      }
    }
    sum = wave_sum_xor32(sum);
    if (h == 0) red[wi * 256 + col] = sum;
  }
  __syncthreads();
  if (wi == 0 && h == 0) {
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int col = 64 * wj + 32 * b + l32;
      const int64_t tok = j0 + col;
      if (tok < p.nc) {
        p.mpart[tok * p.nvt + ti] = mt[b];
        p.spart[tok * p.nvt + ti] = red[col] + red[256 + col];
      }
    }
  }
}

// ---------------------------------------------------------------- row pass
struct RowArgs {
  const float* mpart;    // [nc, nvt] tile max (log2 units)
  const float* spart;    // [nc, nvt] tile sum of exp2(z2 - m)
  const float* zy;
  const int64_t* y;      // chunk labels
  bf16* E;               // [nc, V]: E on entry, dZ on exit
  float* loss_row;       // [nc] (chunk slice)
  const float* invden;
  const int64_t* nvalid;
  int64_t nc, nvt, V, ignore_index, c0;
  int rewrite;           // 0: loss only (E was never stored)
};

// One workgroup (four waves) per token row.  lse2 = M + log2(sum_t s_t
// 2^(m_t - M)); then the row of E becomes dZ = E * f_t - g [v == y], f_t =
// 2^(m_t - lse2) * g, in fp32 and rounded to bf16 once (zero for an ignored
// row: g = 0).  The factors f_t are computed once per tile into LDS, in
// segments of kRowSegTiles tiles, so the streaming loop does one LDS read and
// eight multiplies per 16 bytes.  Four waves per row (rather than one) split
// the per-row reductions over the tile statistics, which precede the
// streaming, four ways.
constexpr int kRowSegTiles = 1024, kRowThreads = 256;
__global__ __launch_bounds__(kRowThreads) void flce_row_kernel(const RowArgs p) {
  constexpr int RT = kRowThreads, NWR = RT / 64;
  __shared__ float fsh[kRowSegTiles];
  __shared__ float red[NWR];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t row = blockIdx.x;
  // rows past the last token tile with a valid row are read by no GEMM
  if (row >= p.nc || row >= ((*p.nvalid - p.c0 + BJ - 1) / BJ) * BJ) return;
  const float* m = p.mpart + row * p.nvt;
  const float* s = p.spart + row * p.nvt;
  float mx = -INFINITY;
  for (int64_t t = tid; t < p.nvt; t += RT) mx = fmaxf(mx, m[t]);
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
  if (lane == 0) red[w] = mx;
  __syncthreads();
#pragma unroll
  for (int i = 0; i < NWR; ++i) mx = fmaxf(mx, red[i]);
  __syncthreads();  // red is reused below
  float sum = 0.f;
  for (int64_t t = tid; t < p.nvt; t += RT) sum += s[t] * exp2f_fast(m[t] - mx);
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) sum += __shfl_xor(sum, o);
  if (lane == 0) red[w] = sum;
  __syncthreads();
  sum = 0.f;
#pragma unroll
  for (int i = 0; i < NWR; ++i) sum += red[i];  // fixed order: every thread gets the same sum
  const float lse2 = mx + __log2f(sum);
  const int64_t yv = p.y[row];
  const bool valid = yv != p.ignore_index && yv >= 0 && yv < p.V;
  const float gv = valid ? *p.invden : 0.f;
  if (tid == 0) p.loss_row[row] = valid ? lse2 * kLn2 - p.zy[row] : 0.f;
  if (!p.rewrite) return;
  // dZ, 8 columns per thread per chunk (V is a multiple of 8, so a chunk never
  // straddles the row end; 8 aligned columns never straddle a 256-column
  // tile: chunk c lies in tile c / 32).  An ignored row's dZ is zero: written
  // without reading E.
  bf16* e = p.E + row * p.V;
  const int64_t nchunk = p.V / 8;
  if (gv == 0.f) {
    for (int64_t c = tid; c < nchunk; c += RT) st_bf16x8(e + 8 * c, zero_bf16x8());
    return;
  }
  auto chunk = [&](const bf16x8& x, float fv, int64_t c) {
    const int64_t v0 = 8 * c;
    bf16x8 o;
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = (bf16)((float)x[i] * fv);
    const int64_t yrel = yv - v0;
    if (yrel >= 0 && yrel < 8) {
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = (i == yrel) ? (bf16)((float)x[i] * fv - gv) : o[i];
    }
    st_bf16x8(e + v0, o);
  };
  // U chunks per thread in flight: thread chunks c + RT u sit in tiles
  // c / 32 + (RT / 32) u (the pass streams E in and dZ out at the device's
  // mixed read / write rate; deeper unrolling, loading the next chunks before
  // this U's stores, and non-temporal accesses measured no faster)
  constexpr int U = 8;
  for (int64_t t0 = 0; t0 < p.nvt; t0 += kRowSegTiles) {
    const int nt = (int)min((int64_t)kRowSegTiles, p.nvt - t0);
    __syncthreads();  // the previous segment's factors are no longer read
    for (int t = tid; t < nt; t += RT) fsh[t] = exp2f_fast(m[t0 + t] - lse2) * gv;
    __syncthreads();
    const int64_t cb = 32 * t0, ce = min(nchunk, 32 * (t0 + nt));
    int64_t c = cb + tid;
    for (; c + RT * (U - 1) < ce; c += RT * U) {
      bf16x8 x[U];
#pragma unroll
      for (int u = 0; u < U; ++u) x[u] = ld_bf16x8(e + 8 * (c + RT * u));
      const int tb = (int)((c - cb) >> 5);
#pragma unroll
      for (int u = 0; u < U; ++u) chunk(x[u], fsh[tb + (RT / 32) * u], c + RT * u);
    }
    for (; c < ce; c += RT) chunk(ld_bf16x8(e + 8 * c), fsh[(c - cb) >> 5], c);
  }
}

// ---------------------------------------------------------------- dH
struct DhArgs {
  GOp Wt;        // W [V, hdim] read as A[i = h][k = v]
  GOp E;         // dZ [nc, V] read as B[j = tok][k = v]
  bf16* dh;      // dhidden rows of the chunk [nc, hdim] (used when splits == 1)
  float* part;   // [splits, nc, hdim]
  const int32_t* rows;    // compacted row -> original row (whole batch)
  const int64_t* nvalid;
  int64_t hdim, nc, kper, c0;
  int nI, nJ, splits;
};

// dH work: a unit is one (token tile, vocab split); its nI hdim tiles share
// the unit's dZ slab, so they run as consecutive blocks on one XCD (block b
// runs on XCD b % 8).  Units are dealt out over the XCDs in turn, splits of a
// token tile on different XCDs: every XCD gets the same number of units, also
// when the token tiles past the valid rows (which return at once) are many --
// a whole token tile per XCD left some XCDs half as loaded as others.  The
// grid is 8 nI ceil(nJ splits / 8) blocks.
__device__ __forceinline__ bool dh_tile_of(int nI, int nJ, int splits, int& ti, int& tj, int& split) {
  const int x = (int)(blockIdx.x % kXcds), k = (int)(blockIdx.x / kXcds);
  ti = k % nI;
  const int unit = x + kXcds * (k / nI);
  tj = unit / splits;
  split = unit - tj * splits;
  return tj < nJ;
}

__global__ __launch_bounds__(NT) void flce_dh_kernel(const DhArgs p) {
  __shared__ __align__(16) bf16 smem[4 * SLAB];
  int ti, tj, split;
  if (!dh_tile_of(p.nI, p.nJ, p.splits, ti, tj, split)) return;
  const int64_t i0 = (int64_t)ti * BI, j0 = (int64_t)tj * BJ;
  const int64_t nv = *p.nvalid - p.c0;
  if (j0 >= nv) return;
  const int64_t kb = split * p.kper;
  const int64_t ke = min(p.E.cols, kb + p.kper);
  f32x16 acc[4][2];
  gemm_core<false, true>(smem, p.Wt, p.E, i0, j0, kb, ke, acc);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, h = lane >> 5, l32 = lane & 31;
  const int wi = w & 1, wj = w >> 1;
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    const int64_t tok = j0 + 64 * wj + 32 * b + l32;
    if (tok >= p.nc) continue;
    if (p.splits == 1 && tok >= nv) continue;  // padding row
    const int64_t orow = p.splits == 1 ? p.rows[p.c0 + tok] : 0;
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const int64_t hh = i0 + 128 * wi + 32 * a + 16 * jj + 8 * h;
        if (hh >= p.hdim) continue;
        if (p.splits == 1) {
          bf16x8 o;
#pragma unroll
          for (int i = 0; i < 8; ++i) o[i] = (bf16)acc[a][b][8 * jj + i];
          st_bf16x8(p.dh + orow * p.hdim + hh, o);
        } else {
          float* dst = p.part + ((int64_t)split * p.nc + tok) * p.hdim + hh;
          f32x4 lo, hi;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            lo[i] = acc[a][b][8 * jj + i];
            hi[i] = acc[a][b][8 * jj + 4 + i];
          }
          *reinterpret_cast<f32x4*>(dst) = lo;
          *reinterpret_cast<f32x4*>(dst + 4) = hi;
        }
      }
  }
}

// dH rows of the chunk: the splits' fp32 partial sums added in split order,
// each compacted row written to its original row.
__global__ __launch_bounds__(256) void flce_dh_sum_kernel(const float* __restrict__ part, bf16* __restrict__ dh,
                                                          const int32_t* __restrict__ rows,
                                                          const int64_t* __restrict__ nvalid, int64_t c0, int64_t nc,
                                                          int64_t hdim, int splits) {
  // part is [splits][nc * hdim]; groups of 8 elements, hdim / 8 per row
  const int64_t nv = min(nc, *nvalid - c0);
  const int64_t gpr = hdim / 8, stride = nc * hdim;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < nv * gpr; i += (int64_t)gridDim.x * 256) {
    f32x4 a = *reinterpret_cast<const f32x4*>(part + 8 * i);
    f32x4 b = *reinterpret_cast<const f32x4*>(part + 8 * i + 4);
    for (int s = 1; s < splits; ++s) {
      a += *reinterpret_cast<const f32x4*>(part + s * stride + 8 * i);
      b += *reinterpret_cast<const f32x4*>(part + s * stride + 8 * i + 4);
    }
    bf16x8 o;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      o[k] = (bf16)a[k];
      o[4 + k] = (bf16)b[k];
    }
    const int64_t r = i / gpr;
    st_bf16x8(dh + (int64_t)rows[c0 + r] * hdim + 8 * (i - r * gpr), o);
  }
}

// ---------------------------------------------------------------- dW
struct DwArgs {
  GOp Ht;        // hidden rows of the chunk [nc, hdim] read as A[i = h][k = tok]
  GOp Et;        // dZ [nc, V] read as B[j = v][k = tok]
  bf16* dw;      // [V, hdim]
  float* acc32;  // [V, hdim] fp32 accumulator across chunks
  const int64_t* nvalid;
  int64_t hdim, V, c0, chunk;
  int nI, nJ;
};

__global__ __launch_bounds__(NT) void flce_dw_kernel(const DwArgs p) {
  __shared__ __align__(16) bf16 smem[4 * SLAB];
  int ti, tj;
  if (!tile_of(p.nI, p.nJ, p.nI, ti, tj)) return;
  const int64_t i0 = (int64_t)ti * BI, j0 = (int64_t)tj * BJ;
  // The chunk's part in the sum over chunks, from the valid-row count: the
  // first chunk starts it, the one holding the last valid row finishes it
  // (bf16 store), chunks past it do nothing.  A single chunk (or no valid
  // row at all) stores bf16 directly.  Over two chunks the first one's sum is
  // kept in dW itself, in bf16, and the second adds to it: dW is rounded
  // twice, and the fp32 [V, hdim] round trip (twice dW's size, written and
  // read back) is saved.  Over more chunks the sum stays in fp32.
  // mode 0: bf16 store; 1: fp32 store; 2: fp32 add; 3: fp32 add + bf16
  // store; 4: bf16 add.
  const int64_t nvt_all = *p.nvalid;
  if (p.c0 > 0 && p.c0 >= nvt_all) return;
  const bool last = p.c0 + p.chunk >= nvt_all;
  const bool two = nvt_all <= 2 * p.chunk;
  const int mode = p.c0 == 0 ? (last || two ? 0 : 1) : (two ? 4 : (last ? 3 : 2));
  // tokens past the last 64-row step with a valid row are skipped (those up to
  // it are zero padding)
  const int64_t nv = nvt_all - p.c0;
  const int64_t ke = min(p.Ht.rows, nv > 0 ? ((nv + BK - 1) / BK) * BK : (int64_t)0);
  f32x16 acc[4][2];
  gemm_core<false, false>(smem, p.Ht, p.Et, i0, j0, 0, ke, acc);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, h = lane >> 5, l32 = lane & 31;
  const int wi = w & 1, wj = w >> 1;
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    const int64_t v = j0 + 64 * wj + 32 * b + l32;
    if (v >= p.V) continue;
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const int64_t hh = i0 + 128 * wi + 32 * a + 16 * jj + 8 * h;
        if (hh >= p.hdim) continue;
        f32x4 lo, hi;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          lo[i] = acc[a][b][8 * jj + i];
          hi[i] = acc[a][b][8 * jj + 4 + i];
        }
        float* a32 = p.acc32 + v * p.hdim + hh;
        if (mode == 2 || mode == 3) {
          lo += *reinterpret_cast<const f32x4*>(a32);
          hi += *reinterpret_cast<const f32x4*>(a32 + 4);
        } else if (mode == 4) {
          const bf16x8 prev = ld_bf16x8(p.dw + v * p.hdim + hh);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            lo[i] += (float)prev[i];
            hi[i] += (float)prev[4 + i];
          }
        }
        if (mode == 1 || mode == 2) {
          *reinterpret_cast<f32x4*>(a32) = lo;
          *reinterpret_cast<f32x4*>(a32 + 4) = hi;
        } else {
          bf16x8 o;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            o[i] = (bf16)lo[i];
            o[4 + i] = (bf16)hi[i];
          }
          st_bf16x8(p.dw + v * p.hdim + hh, o);
        }
      }
  }
}

// ---------------------------------------------------------------- scalars
__global__ __launch_bounds__(1024) void flce_count_kernel(const int64_t* __restrict__ y, int64_t n, int64_t V,
                                                          int64_t ignore_index, int reduction,
                                                          const float* __restrict__ divisor, int64_t* count,
                                                          int64_t* bad, float* invden) {
  __shared__ long long sc[1024], sb[1024];
  long long c = 0, b = 0;
  for (int64_t i = threadIdx.x; i < n; i += 1024) {
    const int64_t v = y[i];
    if (v == ignore_index) continue;
    if (v >= 0 && v < V) ++c;
    else ++b;
  }
  sc[threadIdx.x] = c;
  sb[threadIdx.x] = b;
  __syncthreads();
  for (int s = 512; s >= 1; s >>= 1) {
    if ((int)threadIdx.x < s) {
      sc[threadIdx.x] += sc[threadIdx.x + s];
      sb[threadIdx.x] += sb[threadIdx.x + s];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    *count = sc[0];
    *bad = sb[0];
    *invden = reduction == 0 ? 1.f / (float)sc[0] : 1.f / *divisor;
  }
}

// Valid rows in order, compacted: rows[k] = the k-th row whose label counts,
// *nvalid = their number.  One workgroup; per round 16 chunks of 1024 labels
// are loaded at once, each wave ballots its valid lanes, and one prefix over
// the 256 (chunk, wave) counts places every valid row.
__global__ __launch_bounds__(1024) void flce_compact_kernel(const int64_t* __restrict__ y, int64_t n, int64_t V,
                                                            int64_t ignore_index, int32_t* __restrict__ rows,
                                                            int64_t* __restrict__ nvalid) {
  constexpr int CT = 1024, NWV = CT / 64, PER = 16;
  static_assert(PER * NWV == 256, "one (chunk, wave) count per lane quarter");
  __shared__ int cnt_sh[PER * NWV];  // valid rows of (chunk i, wave w) at i * NWV + w, in row order
  __shared__ long long carry_sh;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const uint64_t below = lane ? (~0ull >> (64 - lane)) : 0ull;  // lanes before this one
  if (tid == 0) carry_sh = 0;
  __syncthreads();
  for (int64_t c0 = 0; c0 < n; c0 += (int64_t)CT * PER) {
    int64_t v[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int64_t r = c0 + (int64_t)i * CT + tid;
      v[i] = r < n ? y[r] : ignore_index;
    }
    uint64_t m[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      m[i] = __ballot(v[i] != ignore_index && v[i] >= 0 && v[i] < V);
      if (lane == 0) cnt_sh[i * NWV + wv] = __popcll(m[i]);
    }
    __syncthreads();
    // exclusive prefix of the 256 counts in row order: lane l holds entries 4 l .. 4 l + 3
    const int a0 = cnt_sh[4 * lane], a1 = cnt_sh[4 * lane + 1], a2 = cnt_sh[4 * lane + 2], a3 = cnt_sh[4 * lane + 3];
    const int lsum = a0 + a1 + a2 + a3;
    int incl = lsum;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int t = __shfl_up(incl, o);
      if (lane >= o) incl += t;
    }
    const int total = __shfl(incl, 63);
    // entry i * NWV + wv sits in lane 4 i + wv / 4 at position wv % 4 (the same position for every i)
    const int k = wv & 3;
    const int mine = incl - lsum + (k > 0 ? a0 : 0) + (k > 1 ? a1 : 0) + (k > 2 ? a2 : 0);
    const long long carry = carry_sh;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const long long r = carry + __shfl(mine, 4 * i + (wv >> 2)) + __popcll(m[i] & below);
      if ((m[i] >> lane) & 1) rows[r] = (int32_t)(c0 + (int64_t)i * CT + tid);
    }
    __syncthreads();
    if (tid == 0) carry_sh += total;
    __syncthreads();
  }
  if (tid == 0) *nvalid = carry_sh;
}

// The compacted operands: Hc[k] = H[rows[k]], yc[k] = y[rows[k]] for k < nvalid,
// zero rows and ignore_index up to the next multiple of 256 (the padding the
// GEMM tiles read); and dH = 0 on every row whose label does not count.  One
// wave per row, 16 bytes per lane per step.
__global__ __launch_bounds__(256) void flce_gather_kernel(const bf16* __restrict__ H, const int64_t* __restrict__ y,
                                                          const int32_t* __restrict__ rows,
                                                          const int64_t* __restrict__ nvalid, int64_t n, int64_t hdim,
                                                          int64_t V, int64_t ignore_index, bf16* __restrict__ Hc,
                                                          int64_t* __restrict__ yc, bf16* __restrict__ dh) {
  const int lane = threadIdx.x & 63;
  const int64_t nvec = hdim / 8, nv = *nvalid, npad = ((nv + 255) / 256) * 256;
  const int64_t wstep = (int64_t)gridDim.x * 4;
  for (int64_t k = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); k < npad; k += wstep) {
    const bool real = k < nv;
    const int64_t src = real ? rows[k] : 0;
    if (lane == 0) yc[k] = real ? y[src] : ignore_index;
    for (int64_t c = lane; c < nvec; c += 64)
      st_bf16x8(Hc + k * hdim + 8 * c, real ? ld_bf16x8(H + src * hdim + 8 * c) : zero_bf16x8());
  }
  if (dh == nullptr) return;  // loss only
  for (int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); t < n; t += wstep) {
    const int64_t v = y[t];
    if (v != ignore_index && v >= 0 && v < V) continue;
    for (int64_t c = lane; c < nvec; c += 64) st_bf16x8(dh + t * hdim + 8 * c, zero_bf16x8());
  }
}

__global__ __launch_bounds__(1024) void flce_loss_kernel(const float* __restrict__ loss_row, int64_t n,
                                                         const int64_t* __restrict__ nvalid,
                                                         const float* __restrict__ invden, float* loss) {
  __shared__ float sm[1024];
  float acc = 0.f;
  const int64_t nv = min(n, *nvalid);
  for (int64_t i = threadIdx.x; i < nv; i += 1024) acc += loss_row[i];
  sm[threadIdx.x] = acc;
  __syncthreads();
  for (int s = 512; s >= 1; s >>= 1) {
    if ((int)threadIdx.x < s) sm[threadIdx.x] += sm[threadIdx.x + s];
    __syncthreads();
  }
  if (threadIdx.x == 0) *loss = sm[0] * *invden;
}

// y = x * scalar in bf16 (rounded once from fp32).  x == y scales in place,
// and then an exact 1.0 returns at once; out of place it is a copy.
__global__ __launch_bounds__(256) void scale_bf16_kernel(const bf16* x, bf16* y, int64_t nvec, int64_t numel,
                                                         const float* __restrict__ scalar) {
  const float s = *scalar;
  if (s == 1.f && x == y) return;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < nvec; i += (int64_t)gridDim.x * 256) {
    if (8 * i + 8 <= numel) {
      bf16x8 v = ld_bf16x8(x + 8 * i);
#pragma unroll
      for (int k = 0; k < 8; ++k) v[k] = (bf16)((float)v[k] * s);
      st_bf16x8(y + 8 * i, v);
    } else {
      for (int64_t k = 8 * i; k < numel; ++k) y[k] = (bf16)((float)x[k] * s);
    }
  }
}

__global__ __launch_bounds__(256) void zero_bf16_kernel(bf16* __restrict__ x, int64_t nvec) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < nvec; i += (int64_t)gridDim.x * 256)
    *reinterpret_cast<u32x4*>(x + 8 * i) = u32x4{0u, 0u, 0u, 0u};
}

// ---------------------------------------------------------------- workspace
struct Layout {
  size_t invden, loss_row, mpart, spart, zy, E, part, acc32, rows, hc, yc, total;
  int64_t chunk, nvt, splits;
};

size_t al(size_t x) { return (x + 255) & ~size_t(255); }

int dh_splits(int64_t hdim, int64_t chunk) {
  const int64_t tiles = ((hdim + BI - 1) / BI) * ((chunk + BJ - 1) / BJ);
  int64_t s = (2048 + tiles - 1) / tiles;
  if (s < 1) s = 1;
  if (s > 8) s = 8;
  return (int)s;
}

// need_dh false: loss only (no E, no gradient buffers); its chunks only bound
// the per-(row, vocab tile) max / sum buffers, so they are large.
constexpr int64_t kLossChunk = 32768;

Layout layout(int64_t n, int64_t hdim, int64_t V, int64_t chunk, bool need_dh, bool need_dw) {
  Layout L{};
  if (!need_dh) {
    need_dw = false;
    chunk = kLossChunk;
  }
  L.chunk = chunk < n ? chunk : (n > 0 ? n : 1);
  L.nvt = (V + kVT - 1) / kVT;
  L.splits = dh_splits(hdim, L.chunk);
  const int64_t nchunks = n > 0 ? (n + L.chunk - 1) / L.chunk : 0;
  size_t off = 0;
  L.invden = off;
  off += 256;
  L.loss_row = off;
  off += al(sizeof(float) * (size_t)(n > 0 ? n : 1));
  L.mpart = off;
  off += al(sizeof(float) * (size_t)(L.chunk * L.nvt));
  L.spart = off;
  off += al(sizeof(float) * (size_t)(L.chunk * L.nvt));
  L.zy = off;
  off += al(sizeof(float) * (size_t)L.chunk);
  L.E = off;
  if (need_dh) off += al(sizeof(bf16) * (size_t)(L.chunk * V));
  L.part = off;
  if (need_dh && L.splits > 1) off += al(sizeof(float) * (size_t)(L.splits * L.chunk * hdim));
  L.acc32 = off;
  // the fp32 dW sum: only when the valid rows may span more than two chunks
  // (over two, the first chunk's sum is kept in dW itself)
  if (need_dw && nchunks > 2) off += al(sizeof(float) * (size_t)(V * hdim));
  const int64_t npad = ((n > 0 ? n : 1) + 255) / 256 * 256;
  L.rows = off;
  off += al(sizeof(int32_t) * (size_t)npad);
  L.hc = off;
  off += al(sizeof(bf16) * (size_t)(npad * hdim));
  L.yc = off;
  off += al(sizeof(int64_t) * (size_t)npad);
  L.total = off;
  return L;
}

}  // namespace

size_t flce_workspace_bytes(int64_t n, int64_t hdim, int64_t vocab, int64_t chunk, bool need_dh, bool need_dw) {
  if (chunk <= 0) return 0;
  return layout(n, hdim, vocab, chunk, need_dh, need_dw).total;
}

hipError_t flce_run(const FlceArgs& a, hipStream_t stream) {
  const bool grads = a.grads;
  const Layout L = layout(a.n, a.hdim, a.vocab, a.chunk, grads, grads && a.dweight != nullptr);
  char* ws = static_cast<char*>(a.ws);
  float* invden = reinterpret_cast<float*>(ws + L.invden);
  float* loss_row = reinterpret_cast<float*>(ws + L.loss_row);
  float* mpart = reinterpret_cast<float*>(ws + L.mpart);
  float* spart = reinterpret_cast<float*>(ws + L.spart);
  float* zy = reinterpret_cast<float*>(ws + L.zy);
  bf16* E = reinterpret_cast<bf16*>(ws + L.E);
  float* part = reinterpret_cast<float*>(ws + L.part);
  float* acc32 = reinterpret_cast<float*>(ws + L.acc32);
  int64_t* nvalid = reinterpret_cast<int64_t*>(ws + L.invden) + 1;
  int32_t* rows = reinterpret_cast<int32_t*>(ws + L.rows);
  bf16* hcomp = reinterpret_cast<bf16*>(ws + L.hc);
  int64_t* ycomp = reinterpret_cast<int64_t*>(ws + L.yc);
  const int64_t V = a.vocab, Hd = a.hdim;

  hipLaunchKernelGGL(flce_count_kernel, dim3(1), dim3(1024), 0, stream, a.labels, a.n, V, a.ignore_index,
                     a.reduction, a.divisor, a.count, a.bad_labels, invden);
  hipLaunchKernelGGL(flce_compact_kernel, dim3(1), dim3(1024), 0, stream, a.labels, a.n, V, a.ignore_index, rows,
                     nvalid);
  if (a.n > 0) {
    int64_t blocks = (a.n + 3) / 4;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(flce_gather_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, a.hidden, a.labels, rows,
                       nvalid, a.n, Hd, V, a.ignore_index, hcomp, ycomp, grads ? a.dhidden : nullptr);
  }
  // chunks of compacted rows: the host sizes them for n rows; those past the
  // valid count return at once
  const int64_t nchunks = a.n > 0 ? (a.n + L.chunk - 1) / L.chunk : 0;
  for (int64_t ci = 0; ci < nchunks; ++ci) {
    const int64_t c0 = ci * L.chunk;
    const int64_t nc = (a.n - c0) < L.chunk ? (a.n - c0) : L.chunk;
    const bf16* Hc = hcomp + c0 * Hd;
    const int64_t* yc = ycomp + c0;

    LogitsArgs lg{};
    lg.W = GOp{a.weight, Hd, V, Hd};
    lg.H = GOp{Hc, Hd, nc, Hd};
    lg.y = yc;
    lg.E = E;
    lg.mpart = mpart;
    lg.spart = spart;
    lg.zy = zy;
    lg.nvalid = nvalid;
    lg.c0 = c0;
    lg.V = V;
    lg.nc = nc;
    lg.nvt = L.nvt;
    lg.nI = (int)L.nvt;
    lg.nJ = (int)((nc + BJ - 1) / BJ);
    lg.store_e = grads ? 1 : 0;
    {
      const int total = lg.nI * lg.nJ;
      const int grid = ((total + kXcds - 1) / kXcds) * kXcds;
      hipLaunchKernelGGL(flce_logits_kernel, dim3(grid), dim3(NT), 0, stream, lg);
    }

    RowArgs rw{};
    rw.mpart = mpart;
    rw.spart = spart;
    rw.zy = zy;
    rw.y = yc;
    rw.E = E;
    rw.loss_row = loss_row + c0;
    rw.invden = invden;
    rw.nvalid = nvalid;
    rw.c0 = c0;
    rw.nc = nc;
    rw.nvt = L.nvt;
    rw.V = V;
    rw.ignore_index = a.ignore_index;
    rw.rewrite = grads ? 1 : 0;
    hipLaunchKernelGGL(flce_row_kernel, dim3((unsigned)nc), dim3(kRowThreads), 0, stream, rw);
    if (!grads) continue;

    DhArgs dh{};
    dh.Wt = GOp{a.weight, Hd, V, Hd};
    dh.E = GOp{E, V, nc, V};
    dh.dh = a.dhidden;
    dh.part = part;
    dh.rows = rows;
    dh.nvalid = nvalid;
    dh.c0 = c0;
    dh.hdim = Hd;
    dh.nc = nc;
    dh.splits = (int)L.splits;
    {
      const int64_t kblocks = (V + BK - 1) / BK;
      dh.kper = ((kblocks + L.splits - 1) / L.splits) * BK;
    }
    dh.nI = (int)((Hd + BI - 1) / BI);
    dh.nJ = (int)((nc + BJ - 1) / BJ);
    {
      const int units = dh.nJ * (int)L.splits;
      const int grid = kXcds * dh.nI * ((units + kXcds - 1) / kXcds);
      hipLaunchKernelGGL(flce_dh_kernel, dim3(grid), dim3(NT), 0, stream, dh);
    }
    if (L.splits > 1) {
      const int64_t nvec = nc * Hd / 8;
      int64_t blocks = (nvec + 255) / 256;
      if (blocks > 4096) blocks = 4096;
      hipLaunchKernelGGL(flce_dh_sum_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, part, a.dhidden, rows,
                         nvalid, c0, nc, Hd, (int)L.splits);
    }

    if (grads && a.dweight != nullptr) {
      DwArgs dw{};
      dw.Ht = GOp{Hc, Hd, nc, Hd};
      dw.Et = GOp{E, V, nc, V};
      dw.dw = a.dweight;
      dw.acc32 = acc32;
      dw.nvalid = nvalid;
      dw.c0 = c0;
      dw.hdim = Hd;
      dw.V = V;
      dw.nI = (int)((Hd + BI - 1) / BI);
      dw.nJ = (int)L.nvt;
      dw.chunk = L.chunk;
      const int total = dw.nI * dw.nJ;
      const int grid = ((total + kXcds - 1) / kXcds) * kXcds;
      hipLaunchKernelGGL(flce_dw_kernel, dim3(grid), dim3(NT), 0, stream, dw);
    }
  }
  if (grads && a.n == 0 && a.dweight != nullptr) {
    // no rows: d loss / d W is zero (a fill kernel, so the call stays graph-capturable)
    const int64_t nvec = V * Hd / 8;
    int64_t blocks = (nvec + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(zero_bf16_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, a.dweight, nvec);
  }
  hipLaunchKernelGGL(flce_loss_kernel, dim3(1), dim3(1024), 0, stream, loss_row, a.n, nvalid, invden, a.loss);
  return hipGetLastError();
}

hipError_t launch_scale_bf16(const bf16* src, bf16* dst, int64_t numel, const float* scalar, hipStream_t stream) {
  const int64_t nvec = (numel + 7) / 8;
  int64_t blocks = (nvec + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(scale_bf16_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, src, dst, nvec, numel, scalar);
  return hipGetLastError();
}

}  // namespace siq
