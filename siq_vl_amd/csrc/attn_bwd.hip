// Varlen flash attention backward for gfx950 (deterministic: no atomics).
//
// Math (the gradient of the reference's eager attention,
// transformers models/qwen2/modeling_qwen2.py:150-172): with P = softmax(S),
// S = scale * Q K^T + mask, and Delta_i = sum_d dO_id O_id,
//   dV = P^T dO,  dP = dO V^T,  dS = P o (dP - Delta),
//   dQ = scale * dS K,  dK = scale * dS^T Q.
// P is recomputed from the forward's LSE: P = exp2(S * scale * log2e - LSE * log2e).
//
// Three kernels:
//  * preprocess: Delta = rowsum(dO o O)                      (HBM-bound)
//  * dK/dV: one workgroup = 32 kv rows of one kv-head.  K and V of those rows
//    sit in every wave's registers as B operands of S = Q K^T and dP = dO V^T
//    (lane = kv column).  The workgroup walks every q-head of the GQA group and
//    every q block that can see the rows, 128 q rows per step (32 per wave),
//    with Q and dO tiles staged row-major in LDS; dV^T += dO^T P and
//    dK^T += Q^T dS read dO^T / Q^T with ds_read_b64_tr_b16.  The four waves'
//    partial dK/dV are summed through LDS at the end and written once.
//  * dQ: one workgroup = 128 q rows of one q-head (same schedule as the
//    forward); Q and dO in registers as B operands of S^T = K Q^T and
//    dP^T = V dO^T, K and V tiles row-major in LDS, dQ^T += K^T dS^T with K^T
//    read by ds_read_b64_tr_b16.
#include "attn.h"

namespace siq {

namespace {

template <int D>
__global__ __launch_bounds__(256) void attn_bwd_preprocess_kernel(const AttnParams p) {
  constexpr int TPR = D / 8;         // threads per (token, head) row
  constexpr int RPB = 256 / TPR;     // rows per block iteration
  const int tid = threadIdx.x, sub = tid % TPR;
  const int64_t nrows = p.total_q * p.hq;
  for (int64_t row = (int64_t)blockIdx.x * RPB + tid / TPR; row < nrows; row += (int64_t)gridDim.x * RPB) {
    const int64_t t = row / p.hq;
    const int hh = (int)(row - t * p.hq);
    const bf16x8 o = ld_bf16x8(p.o + t * p.o_tok + hh * p.o_head + 8 * sub);
    const bf16x8 g = ld_bf16x8(p.dout + t * p.do_tok + hh * p.do_head + 8 * sub);
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc += (float)o[i] * (float)g[i];
#pragma unroll
    for (int m = TPR / 2; m >= 1; m >>= 1) acc += __shfl_xor(acc, m);
    if (sub == 0) p.delta[(int64_t)hh * p.lse_head + t] = acc;
  }
}

template <int D, bool CAUSAL>
__global__ __launch_bounds__(256) void attn_bwd_dkdv_kernel(const AttnParams p) {
  constexpr int BN = kBwdBN, BM = kBwdBM, NT = 256;
  static_assert(BN == 32 && BM == 128, "one 32-row kv tile, 32 q rows per wave");
  using QTile = RowTile<BM, D, NT>;
  constexpr int RS = QTile::RS, TSZ = BM * RS;
  constexpr int STAGE = 2 * TSZ;  // Q, dO (bf16 elements)
  __shared__ __align__(16) bf16 smem[2 * STAGE];
  __shared__ __align__(16) float rowv[2][2][BM];  // [stage][lse2 | delta][q]

  const int2 tl = p.kvtiles[blockIdx.x];
  if (tl.x < 0) return;
  const SeqInfo si = p.seq[tl.x];
  const int hk = blockIdx.y;
  const int k0 = tl.y * BN;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, h = lane >> 5, l32 = lane & 31;
  const int off = si.k_len - si.q_len;
  const float c = p.scale_log2;

  const int kvrow = k0 + l32;
  const bool kvvalid = kvrow < si.k_len;
  bf16x8 kf[D / 16], vf[D / 16];
  {
    const int64_t r = si.k_start + (kvvalid ? kvrow : 0);
    const bf16* kp = p.k + r * p.k_tok + (int64_t)hk * p.k_head + 8 * h;
    const bf16* vp = p.v + r * p.v_tok + (int64_t)hk * p.v_head + 8 * h;
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
      const bf16x8 a = ld_bf16x8(kp + 16 * ks), b = ld_bf16x8(vp + 16 * ks);
      kf[ks] = kvvalid ? a : zero_bf16x8();
      vf[ks] = kvvalid ? b : zero_bf16x8();
    }
  }
  f32x16 dk[D / 32], dv[D / 32];
#pragma unroll
  for (int i = 0; i < D / 32; ++i) {
    dk[i] = zero16();
    dv[i] = zero16();
  }

  // q blocks that can see any of this tile's kv rows
  int qb0 = 0;
  if (CAUSAL) qb0 = max(0, k0 - off) / BM;
  const int nqb = si.q_len > qb0 * BM ? (si.q_len - qb0 * BM + BM - 1) / BM : 0;
  const int nsteps = (k0 < si.k_len) ? nqb * p.n_rep : 0;

  QTile qt, gt;
  qt.init(p.q_tok, tid);
  gt.init(p.do_tok, tid);
  TrRead tr;
  tr.init(RS, lane);
  float rl = 0.f, rd = 0.f;  // this thread's lse2 / delta prefetch (threads < BM)
  auto fetch = [&](int step) {
    const int j = step / nqb, qb = qb0 + step - j * nqb;
    const int hq = hk * p.n_rep + j;
    const int q0 = qb * BM;
    const int nrows = si.q_len - q0;
    const int64_t r0 = si.q_start + q0;
    qt.load(p.q + r0 * p.q_tok + (int64_t)hq * p.q_head, p.q_tok, nrows);
    gt.load(p.dout + r0 * p.do_tok + (int64_t)hq * p.do_head, p.do_tok, nrows);
    if (tid < BM) {
      const bool ok = tid < nrows;
      const int64_t idx = (int64_t)hq * p.lse_head + r0 + (ok ? tid : 0);
      const float l = p.lse[idx], dl = p.delta[idx];
      rl = ok ? l * kLog2e : INFINITY;  // invalid rows: P = exp2(-inf) = 0
      rd = ok ? dl : 0.f;
    }
  };
  auto stash = [&](int buf) {
    bf16* base = smem + buf * STAGE;
    qt.store(base, tid);
    gt.store(base + TSZ, tid);
    if (tid < BM) {
      rowv[buf][0][tid] = rl;
      rowv[buf][1][tid] = rd;
    }
  };

  if (nsteps > 0) {
    fetch(0);
    stash(0);
  }
  __syncthreads();

  for (int step = 0; step < nsteps; ++step) {
    const int buf = step & 1;
    const bf16* Qs = smem + buf * STAGE;
    const bf16* Gs = Qs + TSZ;
    const float* lse2 = rowv[buf][0];
    const float* dlt = rowv[buf][1];
    const int q0 = (qb0 + step % nqb) * BM;
    const bool more = step + 1 < nsteps;
    if (more) fetch(step + 1);

    const int wq0 = q0 + 32 * w;  // first q row of this wave
    const bool active = !CAUSAL || (wq0 + 31 + off >= k0);
    if (active) {
      const bool need_mask = CAUSAL && (wq0 + off < k0 + 31);
      // accumulator r (= 8j + i) holds q = wq0 + 16j + krow(i, h), kv = kvrow
      f32x16 s = zero16(), dp = zero16();
      const bf16* qr = Qs + (32 * w + l32) * RS + 8 * h;
      const bf16* gr = Gs + (32 * w + l32) * RS + 8 * h;
#pragma unroll
      for (int ks = 0; ks < D / 16; ++ks) {
        s = mfma32(ld_bf16x8(qr + 16 * ks), kf[ks], s);
        dp = mfma32(ld_bf16x8(gr + 16 * ks), vf[ks], dp);
      }
      const int rel = kvrow - off - wq0 - 4 * h;  // causal: keep q offsets >= rel
      bf16x8 pb[2], db[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int qo = 32 * w + 16 * j + 4 * h;  // krow(i, h) = 4h + i (i < 4), 8 + 4h + i - 4
        const f32x4 l0 = *reinterpret_cast<const f32x4*>(lse2 + qo);
        const f32x4 l1 = *reinterpret_cast<const f32x4*>(lse2 + qo + 8);
        const f32x4 d0 = *reinterpret_cast<const f32x4*>(dlt + qo);
        const f32x4 d1 = *reinterpret_cast<const f32x4*>(dlt + qo + 8);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float lv = i < 4 ? l0[i] : l1[i - 4];
          const float dv_ = i < 4 ? d0[i] : d1[i - 4];
          float pv = exp2f_fast(__builtin_fmaf(s[8 * j + i], c, -lv));
          if (need_mask) pv = (16 * j + 8 * (i >> 2) + (i & 3) < rel) ? 0.f : pv;
          s[8 * j + i] = pv;
          dp[8 * j + i] = pv * (dp[8 * j + i] - dv_);
        }
        pb[j] = pack8(s, 8 * j);
        db[j] = pack8(dp, 8 * j);
      }
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          dv[dt] = mfma32(tr.read(Gs, RS, 32 * w + 16 * j, 32 * dt), pb[j], dv[dt]);
          dk[dt] = mfma32(tr.read(Qs, RS, 32 * w + 16 * j, 32 * dt), db[j], dk[dt]);
        }
      }
    }
    if (more) stash(buf ^ 1);
    __syncthreads();
  }

  // Sum the four waves' partial dK^T / dV^T through LDS (all waves hold the same
  // 32 kv columns); wave w then finishes d-tiles w, w + 4, ...
  constexpr int NDT = D / 32;
  float* red = reinterpret_cast<float*>(smem);  // [2][4 waves][NDT][16][64]
  static_assert(2 * 4 * NDT * 16 * 64 * 4 <= 2 * STAGE * 2, "reduction fits the staging buffers");
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      red[(((0 * 4 + w) * NDT + dt) * 16 + r) * 64 + lane] = dk[dt][r];
      red[(((1 * 4 + w) * NDT + dt) * 16 + r) * 64 + lane] = dv[dt][r];
    }
  __syncthreads();
  if (kvvalid) {
    const int64_t row = si.k_start + kvrow;
    for (int dt = w; dt < NDT; dt += 4) {
#pragma unroll
      for (int which = 0; which < 2; ++which) {
        float acc[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float a = 0.f;
#pragma unroll
          for (int ww = 0; ww < 4; ++ww) a += red[(((which * 4 + ww) * NDT + dt) * 16 + r) * 64 + lane];
          acc[r] = a;
        }
        const float sc = which == 0 ? p.scale : 1.f;
        bf16* dst = which == 0 ? p.dk + row * p.dk_tok + (int64_t)hk * p.dk_head
                               : p.dv + row * p.dv_tok + (int64_t)hk * p.dv_head;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          bf16x8 o;
#pragma unroll
          for (int i = 0; i < 8; ++i) o[i] = (bf16)(acc[8 * j + i] * sc);
          st_bf16x8(dst + 32 * dt + 16 * j + 8 * h, o);
        }
      }
    }
  }
}

template <int D, bool CAUSAL>
__global__ __launch_bounds__(256) void attn_bwd_dq_kernel(const AttnParams p) {
  constexpr int BM = kFwdBM, BN = kFwdBN, NT = 256;
  using Tile = RowTile<BN, D, NT>;
  constexpr int RS = Tile::RS, TSZ = BN * RS;
  constexpr int STAGE = 2 * TSZ;  // Ks, Vs
  __shared__ __align__(16) bf16 smem[2 * STAGE];

  const int2 tl = p.qtiles[blockIdx.x];
  if (tl.x < 0) return;
  const SeqInfo si = p.seq[tl.x];
  const int hqi = blockIdx.y, hk = hqi / p.n_rep;
  const int q0 = tl.y * BM;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, h = lane >> 5, l32 = lane & 31;
  const int off = si.k_len - si.q_len;
  int kv_end = si.k_len;
  if (CAUSAL) kv_end = min(kv_end, q0 + BM + off);
  const int nblk = kv_end > 0 ? (kv_end + BN - 1) / BN : 0;

  const int qrow = q0 + 32 * w + l32;
  const bool qvalid = qrow < si.q_len;
  const int lim = CAUSAL ? min(si.k_len - 1, qrow + off) : si.k_len - 1;
  bf16x8 qf[D / 16], gf[D / 16];
  float lse2, dlt;
  {
    const int64_t r = si.q_start + (qvalid ? qrow : 0);
    const bf16* qp = p.q + r * p.q_tok + (int64_t)hqi * p.q_head + 8 * h;
    const bf16* gp = p.dout + r * p.do_tok + (int64_t)hqi * p.do_head + 8 * h;
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
      const bf16x8 a = ld_bf16x8(qp + 16 * ks), b = ld_bf16x8(gp + 16 * ks);
      qf[ks] = qvalid ? a : zero_bf16x8();
      gf[ks] = qvalid ? b : zero_bf16x8();
    }
    const int64_t idx = (int64_t)hqi * p.lse_head + r;
    const float l = p.lse[idx], dl = p.delta[idx];
    lse2 = qvalid ? l * kLog2e : INFINITY;
    dlt = qvalid ? dl : 0.f;
  }
  f32x16 dq[D / 32];
#pragma unroll
  for (int i = 0; i < D / 32; ++i) dq[i] = zero16();
  const float c = p.scale_log2;

  const bf16* kbase = p.k + (int64_t)si.k_start * p.k_tok + (int64_t)hk * p.k_head;
  const bf16* vbase = p.v + (int64_t)si.k_start * p.v_tok + (int64_t)hk * p.v_head;
  Tile kt, vt;
  kt.init(p.k_tok, tid);
  vt.init(p.v_tok, tid);
  TrRead tr;
  tr.init(RS, lane);
  if (nblk > 0) {
    kt.load(kbase, p.k_tok, si.k_len);
    vt.load(vbase, p.v_tok, si.k_len);
    kt.store(smem, tid);
    vt.store(smem + TSZ, tid);
  }
  __syncthreads();

  const int wq_last = q0 + 32 * w + 31;
  for (int kb = 0; kb < nblk; ++kb) {
    const bf16* Ks = smem + (kb & 1) * STAGE;
    const bf16* Vs = Ks + TSZ;
    const int k0 = kb * BN;
    const bool more = kb + 1 < nblk;
    if (more) {
      kt.load(kbase + (int64_t)(k0 + BN) * p.k_tok, p.k_tok, si.k_len - k0 - BN);
      vt.load(vbase + (int64_t)(k0 + BN) * p.v_tok, p.v_tok, si.k_len - k0 - BN);
    }
    const bool active = !CAUSAL || (k0 <= wq_last + off);
    if (active) {
      const bool need_mask = (k0 + BN > si.k_len) || (CAUSAL && k0 + BN - 1 > q0 + 32 * w + off);
      // accumulator (t, r) holds kv = k0 + 32t + nrow(r, h) for q = qrow
      f32x16 s[BN / 32], dp[BN / 32];
#pragma unroll
      for (int t = 0; t < BN / 32; ++t) {
        s[t] = zero16();
        dp[t] = zero16();
        const bf16* kr = Ks + (32 * t + l32) * RS + 8 * h;
        const bf16* vr = Vs + (32 * t + l32) * RS + 8 * h;
#pragma unroll
        for (int ks = 0; ks < D / 16; ++ks) {
          s[t] = mfma32(ld_bf16x8(kr + 16 * ks), qf[ks], s[t]);
          dp[t] = mfma32(ld_bf16x8(vr + 16 * ks), gf[ks], dp[t]);
        }
      }
      const int rel = lim - k0 - 4 * h;
      bf16x8 db[BN / 16];
#pragma unroll
      for (int t = 0; t < BN / 32; ++t) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float pv = exp2f_fast(__builtin_fmaf(s[t][r], c, -lse2));
          if (need_mask) pv = (32 * t + 8 * (r >> 2) + (r & 3) > rel) ? 0.f : pv;
          dp[t][r] = pv * (dp[t][r] - dlt);
        }
        db[2 * t] = pack8(dp[t], 0);
        db[2 * t + 1] = pack8(dp[t], 8);
      }
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt) {
#pragma unroll
        for (int st = 0; st < BN / 16; ++st) dq[dt] = mfma32(tr.read(Ks, RS, 16 * st, 32 * dt), db[st], dq[dt]);
      }
    }
    if (more) {
      bf16* nx = smem + ((kb + 1) & 1) * STAGE;
      kt.store(nx, tid);
      vt.store(nx + TSZ, tid);
    }
    __syncthreads();
  }

  if (qvalid) {
    bf16* dqp = p.dq + (int64_t)(si.q_start + qrow) * p.dq_tok + (int64_t)hqi * p.dq_head;
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        bf16x8 a;
#pragma unroll
        for (int i = 0; i < 8; ++i) a[i] = (bf16)(dq[dt][8 * j + i] * p.scale);
        st_bf16x8(dqp + 32 * dt + 16 * j + 8 * h, a);
      }
    }
  }
}

template <int D, bool CAUSAL>
hipError_t launch_bwd_t(const AttnParams& p, int qcap, int kvcap, hipStream_t stream) {
  const int64_t rows = p.total_q * p.hq;
  if (rows > 0) {
    const int rpb = 256 / (D / 8);
    int64_t blocks = (rows + rpb - 1) / rpb;
    if (blocks > 8192) blocks = 8192;
    hipLaunchKernelGGL((attn_bwd_preprocess_kernel<D>), dim3((unsigned)blocks), dim3(256), 0, stream, p);
  }
  hipLaunchKernelGGL((attn_bwd_dkdv_kernel<D, CAUSAL>), dim3(kvcap, p.hkv), dim3(256), 0, stream, p);
  hipLaunchKernelGGL((attn_bwd_dq_kernel<D, CAUSAL>), dim3(qcap, p.hq), dim3(256), 0, stream, p);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_attn_bwd(const AttnParams& p, int d, int causal, int qcap, int kvcap, hipStream_t stream) {
  if (d == 128) return causal ? launch_bwd_t<128, true>(p, qcap, kvcap, stream) : launch_bwd_t<128, false>(p, qcap, kvcap, stream);
  if (d == 64) return causal ? launch_bwd_t<64, true>(p, qcap, kvcap, stream) : launch_bwd_t<64, false>(p, qcap, kvcap, stream);
  return hipErrorInvalidValue;
}

}  // namespace siq
