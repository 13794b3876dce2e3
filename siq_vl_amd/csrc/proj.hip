// Pixel-shuffle projector (forward and backward) for gfx950.
//
// Semantics: SiQ_VLProjector (siq_vl/model/modeling.py:37-106): the vision
// tower's [batch, side * side, dv] patch features are pixel-shuffled by r --
// token (ho, wo) of the side/r x side/r grid gathers the r x r patches
// (ho r + i, wo r + j) into features (i r + j) dv + c (view / reshape /
// permute(0, 1, 3, 2, 4, 5) at :93-98) -- and projected by a bias-free Linear
// (:59, :101-105):  y = Xs W^T,  Xs [m = batch t, k = r r dv],  W [n, k].
// Backward:  dXs = dY W (scattered back to x's layout),  dW = dY^T Xs.
//
// The reference materialises Xs with .contiguous() (one read and one write of
// the features), and autograd materialises dXs before permuting it back.  Here
// the shuffle lives in the operand addressing: a 16-byte chunk of Xs (8
// consecutive features of one token) is 16 contiguous bytes of x, so the
// direct global->LDS loads of the GEMM slabs gather Xs rows straight from x,
// and the dX epilogue scatters its rows straight to x's layout.  The three
// GEMMs are the CE's tiled core (gemm.h: 256 x 256 tiles, 8 waves, bf16 MFMA,
// fp32 accumulation), each computed transposed so that a lane's 8
// consecutive outputs are 8 consecutive elements of the output's row:
//   forward  Y^T [n][m]   = W  . Xs^T  (A = W rows, B = gathered Xs rows)
//   dX       dXs^T [k][m] = W^T . dY^T (A = W read k-major, B = dY rows)
//   dW       dW^T [k][n]  = Xs^T . dY  (A = gathered Xs read k-major, B = dY read k-major)
// The forward and dW have few tiles at projector sizes (96 at m = 4096,
// n = 1536, k = 4096), so their reduction is split over up to 8 workgroups
// per tile with fp32 partial sums added afterwards in split order
// (deterministic).
#include "gemm.h"
#include "proj.h"

namespace siq {

namespace {

using namespace gemm;

// Pixel-shuffle geometry; every index here is < 2^31 (checked on the host).
struct Shuffle {
  int r, side, wo, t, dv, m, k;
  float inv_t, inv_wo, inv_dv;

  // a / d for 0 <= a < 2^24, via the fp32 reciprocal plus one correction
  __device__ __forceinline__ static int divf(int a, int d, float inv) {
    int q = (int)((float)a * inv);
    if (q * d > a) --q;
    else if ((q + 1) * d <= a) ++q;
    return q;
  }
  // row of x holding segment (i, j) = (0, 0) of shuffled token mm
  __device__ __forceinline__ int xrow(int mm) const {
    const int b = divf(mm, t, inv_t), tt = mm - b * t;
    const int ho = divf(tt, wo, inv_wo), w_ = tt - ho * wo;
    return (b * side + ho * r) * side + w_ * r;
  }
  // offset in x, from row xrow(m), of feature kf = (i r + j) dv + c
  __device__ __forceinline__ int featoff(int kf) const {
    const int ij = divf(kf, dv, inv_dv), c = kf - ij * dv;
    const int i = ij / r, j = ij - i * r;
    return (i * side + j) * dv + c;
  }
};

// Xs as a k-contiguous operand (slab rows = shuffled tokens j0 + row,
// 64 features per k-step, inside one (i, j) segment since dv % 64 == 0): the
// layout of SlabLoad<true>, with each row's x address from the shuffle.
struct GatherKC {
  const bf16* x;
  Shuffle sh;
  uint32_t rowoff[4];  // per instruction: xrow(token) * dv + the lane's swizzled chunk
  __device__ __forceinline__ void init(const bf16* xp, const Shuffle& s, int64_t j0, int lane, int w) {
    x = xp;
    sh = s;
    const int lrow = lane / 8, lpc = lane % 8;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int row = 32 * w + 8 * q + lrow;
      const int tok = min((int)j0 + row, s.m - 1);  // rows past the end re-read the last token (never stored)
      rowoff[q] = (uint32_t)(s.xrow(tok) * s.dv + 8 * (lpc ^ swz_kc(row)));
    }
  }
  __device__ __forceinline__ void issue(int64_t k0, bf16* lds, int wu) const {
    const uint32_t delta = (uint32_t)sh.featoff((int)k0);
#pragma unroll
    for (int q = 0; q < 4; ++q) dma16(x, rowoff[q] + delta, lds + (wu * 4 + q) * 512);
  }
};

// Xs^T as a k-major operand (slab rows = shuffled tokens k0 + row, 256
// feature columns i0 .. i0 + 255): the layout of SlabLoad<false>.  A lane's
// chunk columns are fixed per tile; its rows' x addresses are recomputed per
// k-step.
struct GatherNKC {
  const bf16* x;
  Shuffle sh;
  int coloff[4];  // per instruction: offset of the lane's 8 features from the token's row
  int rr[4];      // per instruction: the lane's slab row
  __device__ __forceinline__ void init(const bf16* xp, const Shuffle& s, int64_t i0, int lane, int w) {
    x = xp;
    sh = s;
    const int lrow = lane / 32, lpc = lane % 32;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int row = 8 * w + 2 * q + lrow;
      const int col = min((int)i0 + 8 * (lpc ^ swz_nkc(row)), s.k - 8);  // columns past k: never stored
      coloff[q] = s.featoff(col);
      rr[q] = row;
    }
  }
  __device__ __forceinline__ void issue(int64_t k0, bf16* lds, int wu) const {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int tok = min((int)k0 + rr[q], sh.m - 1);  // past the end: multiplied by the zeroed dY tail
      dma16(x, (uint32_t)(sh.xrow(tok) * sh.dv + coloff[q]), lds + (wu * 4 + q) * 512);
    }
  }
};

struct FwdArgs {
  GOp W;            // [n, k]
  const bf16* x;
  Shuffle sh;
  bf16* y;          // [m, n]
  float* part;      // [splits, m, n] when splits > 1
  int64_t n, kper;
  int nI, nJ, splits;
};

__global__ __launch_bounds__(NT) void proj_fwd_kernel(const FwdArgs p) {
  __shared__ __align__(16) bf16 smem[4 * SLAB];
  int ti, tj;
  if (!tile_of(p.nI, p.nJ, p.nI, ti, tj)) return;
  const int split = blockIdx.y;
  const int64_t i0 = (int64_t)ti * BI, j0 = (int64_t)tj * BJ;
  const int64_t kb = split * p.kper, ke = min((int64_t)p.sh.k, kb + p.kper);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, h = lane >> 5, l32 = lane & 31;
  OpLoad<true> la;
  la.init(p.W, i0, lane, w);
  GatherKC lb;
  lb.init(p.x, p.sh, j0, lane, w);
  f32x16 acc[4][2];
  gemm_core_l<true, true>(smem, la, lb, kb, ke, acc);
  const int wi = w & 1, wj = w >> 1;
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    const int64_t tok = j0 + 64 * wj + 32 * b + l32;
    if (tok >= p.sh.m) continue;
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const int64_t nn = i0 + 128 * wi + 32 * a + 16 * jj + 8 * h;
        if (nn >= p.n) continue;
        if (p.splits == 1) {
          bf16x8 o;
#pragma unroll
          for (int i = 0; i < 8; ++i) o[i] = (bf16)acc[a][b][8 * jj + i];
          st_bf16x8(p.y + tok * p.n + nn, o);
        } else {
          float* dst = p.part + ((int64_t)split * p.sh.m + tok) * p.n + nn;
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

struct DxArgs {
  GOp Wt;           // W [n, k] read as A[i = feature][kk = output feature]
  GOp dY;           // [m, n]
  Shuffle sh;
  bf16* dx;         // [batch, side * side, dv]
  int nI, nJ;
};

__global__ __launch_bounds__(NT) void proj_dx_kernel(const DxArgs p) {
  __shared__ __align__(16) bf16 smem[4 * SLAB];
  int ti, tj;
  if (!tile_of(p.nI, p.nJ, p.nI, ti, tj)) return;
  const int64_t i0 = (int64_t)ti * BI, j0 = (int64_t)tj * BJ;
  f32x16 acc[4][2];
  gemm_core<false, true>(smem, p.Wt, p.dY, i0, j0, 0, p.dY.cols, acc);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, h = lane >> 5, l32 = lane & 31;
  const int wi = w & 1, wj = w >> 1;
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    const int tok = (int)(j0 + 64 * wj + 32 * b + l32);
    if (tok >= p.sh.m) continue;
    bf16* row = p.dx + (int64_t)p.sh.xrow(tok) * p.sh.dv;
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const int kf = (int)(i0 + 128 * wi + 32 * a + 16 * jj + 8 * h);
        if (kf >= p.sh.k) continue;
        bf16x8 o;
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = (bf16)acc[a][b][8 * jj + i];
        st_bf16x8(row + p.sh.featoff(kf), o);
      }
  }
}

struct DwArgs {
  const bf16* x;
  Shuffle sh;
  GOp dY;           // [m, n] read as B[j = output feature][kk = token]
  bf16* dw;         // [n, k]
  float* part;      // [splits, n, k] when splits > 1
  int64_t n, kper;
  int nI, nJ, splits;
};

__global__ __launch_bounds__(NT) void proj_dw_kernel(const DwArgs p) {
  __shared__ __align__(16) bf16 smem[4 * SLAB];
  int ti, tj;
  if (!tile_of(p.nI, p.nJ, p.nI, ti, tj)) return;
  const int split = blockIdx.y;
  const int64_t i0 = (int64_t)ti * BI, j0 = (int64_t)tj * BJ;
  const int64_t kb = split * p.kper, ke = min((int64_t)p.sh.m, kb + p.kper);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, h = lane >> 5, l32 = lane & 31;
  GatherNKC la;
  la.init(p.x, p.sh, i0, lane, w);
  OpLoad<false> lb;
  lb.init(p.dY, j0, lane, w);
  f32x16 acc[4][2];
  gemm_core_l<false, false>(smem, la, lb, kb, ke, acc);
  const int wi = w & 1, wj = w >> 1;
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    const int64_t nn = j0 + 64 * wj + 32 * b + l32;
    if (nn >= p.n) continue;
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const int64_t kf = i0 + 128 * wi + 32 * a + 16 * jj + 8 * h;
        if (kf >= p.sh.k) continue;
        if (p.splits == 1) {
          bf16x8 o;
#pragma unroll
          for (int i = 0; i < 8; ++i) o[i] = (bf16)acc[a][b][8 * jj + i];
          st_bf16x8(p.dw + nn * p.sh.k + kf, o);
        } else {
          float* dst = p.part + ((int64_t)split * p.n + nn) * p.sh.k + kf;
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

// out[e] = bf16(sum over s of part[s][e]), s in order; nvec groups of 8.
__global__ __launch_bounds__(256) void proj_sum_kernel(const float* __restrict__ part, bf16* __restrict__ out,
                                                       int64_t nvec, int64_t stride, int splits) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < nvec; i += (int64_t)gridDim.x * 256) {
    f32x4 a = *reinterpret_cast<const f32x4*>(part + 8 * i);
    f32x4 b = *reinterpret_cast<const f32x4*>(part + 8 * i + 4);
    for (int s = 1; s < splits; ++s) {
      a += *reinterpret_cast<const f32x4*>(part + s * stride + 8 * i);
      b += *reinterpret_cast<const f32x4*>(part + s * stride + 8 * i + 4);
    }
    bf16x8 o;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      o[q] = (bf16)a[q];
      o[4 + q] = (bf16)b[q];
    }
    st_bf16x8(out + 8 * i, o);
  }
}

__global__ __launch_bounds__(256) void proj_zero_kernel(bf16* __restrict__ out, int64_t nvec) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < nvec; i += (int64_t)gridDim.x * 256)
    *reinterpret_cast<u32x4*>(out + 8 * i) = u32x4{0u, 0u, 0u, 0u};
}

int cu_count() {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) dev = 0;
  int cu = dev < 64 ? cus[dev] : 0;
  if (cu <= 0) {
    if (hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cu <= 0) cu = 256;
    if (dev < 64) cus[dev] = cu;
  }
  return cu;
}

Shuffle shuffle_of(const ProjArgs& a) {
  Shuffle s;
  s.r = a.r;
  s.side = (int)a.side;
  s.wo = (int)(a.side / a.r);
  s.t = s.wo * s.wo;
  s.dv = (int)a.dv;
  s.m = (int)(a.batch * s.t);
  s.k = a.r * a.r * s.dv;
  s.inv_t = 1.f / (float)s.t;
  s.inv_wo = 1.f / (float)s.wo;
  s.inv_dv = 1.f / (float)s.dv;
  return s;
}

// Split-K factor: enough workgroups to cover the CUs once, each keeping at
// least 8 k-steps, at most 8 splits.
int splits_for(int64_t tiles, int64_t kdim, int cus) {
  int64_t s = tiles > 0 ? cus / tiles : 1;
  const int64_t ksteps = (kdim + BK - 1) / BK;
  if (s > ksteps / 8) s = ksteps / 8;
  if (s > 8) s = 8;
  return s < 1 ? 1 : (int)s;
}

int64_t kper_for(int64_t kdim, int splits) {
  const int64_t ksteps = (kdim + BK - 1) / BK;
  return ((ksteps + splits - 1) / splits) * BK;
}

unsigned grid_of(int nI, int nJ) { return (unsigned)(((nI * nJ + kXcds - 1) / kXcds) * kXcds); }

void launch_sum(const float* part, bf16* out, int64_t elems, int splits, hipStream_t stream) {
  const int64_t nvec = elems / 8;
  int64_t blocks = (nvec + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(proj_sum_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, part, out, nvec, elems, splits);
}

}  // namespace

size_t proj_workspace_bytes(int64_t batch, int64_t side, int64_t dv, int r, int64_t n) {
  const int64_t t = (side / r) * (side / r), m = batch * t, k = (int64_t)r * r * dv;
  const int cus = cu_count();
  const int64_t tiles_f = ((n + BI - 1) / BI) * ((m + BJ - 1) / BJ);
  const int64_t tiles_w = ((k + BI - 1) / BI) * ((n + BJ - 1) / BJ);
  const int sf = splits_for(tiles_f, k, cus), sw = splits_for(tiles_w, m, cus);
  const int64_t f = sf > 1 ? (int64_t)sf * m * n : 0, w = sw > 1 ? (int64_t)sw * n * k : 0;
  return (size_t)((f > w ? f : w) * 4);
}

hipError_t proj_fwd(const ProjArgs& a, hipStream_t stream) {
  const Shuffle sh = shuffle_of(a);
  FwdArgs p{};
  p.W = GOp{a.weight, sh.k, a.n, sh.k};
  p.x = a.x;
  p.sh = sh;
  p.y = a.y;
  p.part = a.part;
  p.n = a.n;
  p.nI = (int)((a.n + BI - 1) / BI);
  p.nJ = (int)((sh.m + BJ - 1) / BJ);
  p.splits = splits_for((int64_t)p.nI * p.nJ, sh.k, cu_count());
  p.kper = kper_for(sh.k, p.splits);
  hipLaunchKernelGGL(proj_fwd_kernel, dim3(grid_of(p.nI, p.nJ), (unsigned)p.splits), dim3(NT), 0, stream, p);
  if (p.splits > 1) launch_sum(a.part, a.y, (int64_t)sh.m * a.n, p.splits, stream);
  return hipGetLastError();
}

hipError_t proj_bwd(const ProjArgs& a, hipStream_t stream) {
  const Shuffle sh = shuffle_of(a);
  if (sh.m == 0) {
    // no tokens: d loss / d weight is zero (a fill kernel, so the call stays graph-capturable)
    if (a.dweight != nullptr) {
      const int64_t nvec = a.n * sh.k / 8;
      int64_t blocks = (nvec + 255) / 256;
      if (blocks > 4096) blocks = 4096;
      if (nvec > 0) hipLaunchKernelGGL(proj_zero_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, a.dweight, nvec);
    }
    return hipGetLastError();
  }
  if (a.dx != nullptr) {
    DxArgs p{};
    p.Wt = GOp{a.weight, sh.k, a.n, sh.k};
    p.dY = GOp{a.dy, a.n, sh.m, a.n};
    p.sh = sh;
    p.dx = a.dx;
    p.nI = (int)((sh.k + BI - 1) / BI);
    p.nJ = (int)((sh.m + BJ - 1) / BJ);
    hipLaunchKernelGGL(proj_dx_kernel, dim3(grid_of(p.nI, p.nJ)), dim3(NT), 0, stream, p);
  }
  if (a.dweight != nullptr) {
    DwArgs p{};
    p.x = a.x;
    p.sh = sh;
    p.dY = GOp{a.dy, a.n, sh.m, a.n};
    p.dw = a.dweight;
    p.part = a.part;
    p.n = a.n;
    p.nI = (int)((sh.k + BI - 1) / BI);
    p.nJ = (int)((a.n + BJ - 1) / BJ);
    p.splits = splits_for((int64_t)p.nI * p.nJ, sh.m, cu_count());
    p.kper = kper_for(sh.m, p.splits);
    hipLaunchKernelGGL(proj_dw_kernel, dim3(grid_of(p.nI, p.nJ), (unsigned)p.splits), dim3(NT), 0, stream, p);
    if (p.splits > 1) launch_sum(a.part, a.dweight, a.n * sh.k, p.splits, stream);
  }
  return hipGetLastError();
}

}  // namespace siq
