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
//  * dK/dV: one workgroup = 128 kv rows (4 waves x 32) of one kv-head; it
//    loops over every q-head of the GQA group and every q block that can see
//    those kv rows, so dK/dV are complete in registers and written once.
//    K and V live in registers as B operands of S = Q K^T and dP = dO V^T
//    (each lane then holds one kv column); Q and dO tiles are staged in LDS
//    both row-major (A of S, dP) and transposed (A of dK^T += Q^T dS,
//    dV^T += dO^T P).
//  * dQ: one workgroup = 128 q rows of one q-head (same schedule as the
//    forward); Q and dO in registers as B operands of S^T = K Q^T and
//    dP^T = V dO^T, K row-major + transposed and V row-major in LDS;
//    dQ^T += K^T dS^T.
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
  using QTile = Tile4x8<BM, D, NT, true>;
  constexpr int RS = QTile::RS, TS = QTile::TS;
  constexpr int RSZ = BM * RS, TSZ = D * TS;
  constexpr int STAGE = 2 * RSZ + 2 * TSZ;  // Qs, Qt, dOs, dOt (bf16 elements)
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

  // K, V rows of this wave as B operands (lane = kv column k0 + 32w + l32).
  const int kvrow = k0 + 32 * w + l32;
  const bool kvvalid = kvrow < si.k_len;
  bf16x8 kf[D / 16], vf[D / 16];
  {
    const int64_t r = si.k_start + (kvvalid ? kvrow : 0);
    const bf16* kp = p.k + r * p.k_tok + (int64_t)hk * p.k_head + 8 * h;
    const bf16* vp = p.v + r * p.v_tok + (int64_t)hk * p.v_head + 8 * h;
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
      kf[ks] = kvvalid ? ld_bf16x8(kp + 16 * ks) : zero_bf16x8();
      vf[ks] = kvvalid ? ld_bf16x8(vp + 16 * ks) : zero_bf16x8();
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
  float rl = 0.f, rd = 0.f;  // this thread's lse2 / delta prefetch (threads < BM)
  auto fetch = [&](int step) {
    const int j = step / nqb, qb = qb0 + step % nqb;
    const int hq = hk * p.n_rep + j;
    const int q0 = qb * BM;
    const int nrows = si.q_len - q0;
    const int64_t r0 = si.q_start + q0;
    qt.load(p.q + r0 * p.q_tok + (int64_t)hq * p.q_head, p.q_tok, nrows, tid);
    gt.load(p.dout + r0 * p.do_tok + (int64_t)hq * p.do_head, p.do_tok, nrows, tid);
    if (tid < BM) {
      const bool ok = tid < nrows;
      rl = ok ? p.lse[(int64_t)hq * p.lse_head + r0 + tid] * kLog2e : 0.f;
      rd = ok ? p.delta[(int64_t)hq * p.lse_head + r0 + tid] : 0.f;
    }
  };
  auto stash = [&](int buf) {
    bf16* base = smem + buf * STAGE;
    qt.store_rows(base, tid);
    qt.store_cols(base + RSZ, tid);
    gt.store_rows(base + RSZ + TSZ, tid);
    gt.store_cols(base + 2 * RSZ + TSZ, tid);
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

  const int wk_first = k0 + 32 * w;  // first kv row of this wave
  for (int step = 0; step < nsteps; ++step) {
    const int buf = step & 1;
    const bf16* Qs = smem + buf * STAGE;
    const bf16* Qt = Qs + RSZ;
    const bf16* Gs = Qt + TSZ;
    const bf16* Gt = Gs + RSZ;
    const float* lse2 = rowv[buf][0];
    const float* dlt = rowv[buf][1];
    const int q0 = (qb0 + step % nqb) * BM;
    const bool more = step + 1 < nsteps;
    if (more) fetch(step + 1);

    const bool active = !CAUSAL || (q0 + BM - 1 + off >= wk_first);
    if (active) {
      const bool need_mask = CAUSAL && (q0 + off < wk_first + 31);
      f32x16 s[BM / 32], dp[BM / 32];
#pragma unroll
      for (int t = 0; t < BM / 32; ++t) {
        s[t] = zero16();
        dp[t] = zero16();
        const bf16* qr = Qs + (32 * t + perm32(l32)) * RS + 8 * h;
        const bf16* gr = Gs + (32 * t + perm32(l32)) * RS + 8 * h;
#pragma unroll
        for (int ks = 0; ks < D / 16; ++ks) {
          s[t] = mfma32(ld_bf16x8(qr + 16 * ks), kf[ks], s[t]);
          dp[t] = mfma32(ld_bf16x8(gr + 16 * ks), vf[ks], dp[t]);
        }
      }
      bf16x8 pb[BM / 16], db[BM / 16];
#pragma unroll
      for (int t = 0; t < BM / 32; ++t) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int qb = 32 * t + 16 * j + 8 * h;  // first of 8 consecutive q rows
          const f32x4 l0 = *reinterpret_cast<const f32x4*>(lse2 + qb);
          const f32x4 l1 = *reinterpret_cast<const f32x4*>(lse2 + qb + 4);
          const f32x4 d0 = *reinterpret_cast<const f32x4*>(dlt + qb);
          const f32x4 d1 = *reinterpret_cast<const f32x4*>(dlt + qb + 4);
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const float lv = i < 4 ? l0[i] : l1[i - 4];
            const float dv_ = i < 4 ? d0[i] : d1[i - 4];
            float pv = exp2f_fast(s[t][8 * j + i] * c - lv);
            if (need_mask && kvrow > q0 + qb + i + off) pv = 0.f;
            s[t][8 * j + i] = pv;
            dp[t][8 * j + i] = pv * (dp[t][8 * j + i] - dv_);
          }
          pb[2 * t + j] = pack8(s[t], 8 * j);
          db[2 * t + j] = pack8(dp[t], 8 * j);
        }
      }
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt) {
        const bf16* gtr = Gt + (32 * dt + perm32(l32)) * TS + 8 * h;
        const bf16* qtr = Qt + (32 * dt + perm32(l32)) * TS + 8 * h;
#pragma unroll
        for (int st = 0; st < BM / 16; ++st) {
          dv[dt] = mfma32(ld_bf16x8(gtr + 16 * st), pb[st], dv[dt]);
          dk[dt] = mfma32(ld_bf16x8(qtr + 16 * st), db[st], dk[dt]);
        }
      }
    }
    if (more) stash(buf ^ 1);
    __syncthreads();
  }

  if (kvvalid) {
    const int64_t r = si.k_start + kvrow;
    bf16* dkp = p.dk + r * p.dk_tok + (int64_t)hk * p.dk_head;
    bf16* dvp = p.dv + r * p.dv_tok + (int64_t)hk * p.dv_head;
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        bf16x8 a, b;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          a[i] = (bf16)(dk[dt][8 * j + i] * p.scale);
          b[i] = (bf16)dv[dt][8 * j + i];
        }
        st_bf16x8(dkp + 32 * dt + 16 * j + 8 * h, a);
        st_bf16x8(dvp + 32 * dt + 16 * j + 8 * h, b);
      }
    }
  }
}

template <int D, bool CAUSAL>
__global__ __launch_bounds__(256) void attn_bwd_dq_kernel(const AttnParams p) {
  constexpr int BM = kFwdBM, BN = kFwdBN, NT = 256;
  using KTile = Tile4x8<BN, D, NT, true>;
  using VTile = Tile4x8<BN, D, NT, false>;
  constexpr int RS = KTile::RS, TS = KTile::TS;
  constexpr int RSZ = BN * RS, TSZ = D * TS;
  constexpr int STAGE = 2 * RSZ + TSZ;  // Ks, Kt, Vs
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
  bf16x8 qf[D / 16], gf[D / 16];
  float lse2 = 0.f, dlt = 0.f;
  {
    const int64_t r = si.q_start + (qvalid ? qrow : 0);
    const bf16* qp = p.q + r * p.q_tok + (int64_t)hqi * p.q_head + 8 * h;
    const bf16* gp = p.dout + r * p.do_tok + (int64_t)hqi * p.do_head + 8 * h;
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
      qf[ks] = qvalid ? ld_bf16x8(qp + 16 * ks) : zero_bf16x8();
      gf[ks] = qvalid ? ld_bf16x8(gp + 16 * ks) : zero_bf16x8();
    }
    if (qvalid) {
      lse2 = p.lse[(int64_t)hqi * p.lse_head + r] * kLog2e;
      dlt = p.delta[(int64_t)hqi * p.lse_head + r];
    }
  }
  f32x16 dq[D / 32];
#pragma unroll
  for (int i = 0; i < D / 32; ++i) dq[i] = zero16();
  const float c = p.scale_log2;

  const bf16* kbase = p.k + (int64_t)si.k_start * p.k_tok + (int64_t)hk * p.k_head;
  const bf16* vbase = p.v + (int64_t)si.k_start * p.v_tok + (int64_t)hk * p.v_head;
  KTile kt;
  VTile vt;
  if (nblk > 0) {
    kt.load(kbase, p.k_tok, si.k_len, tid);
    vt.load(vbase, p.v_tok, si.k_len, tid);
    kt.store_rows(smem, tid);
    kt.store_cols(smem + RSZ, tid);
    vt.store_rows(smem + RSZ + TSZ, tid);
  }
  __syncthreads();

  const int wq_last = q0 + 32 * w + 31;
  for (int kb = 0; kb < nblk; ++kb) {
    const bf16* Ks = smem + (kb & 1) * STAGE;
    const bf16* Kt = Ks + RSZ;
    const bf16* Vs = Kt + TSZ;
    const int k0 = kb * BN;
    const bool more = kb + 1 < nblk;
    if (more) {
      kt.load(kbase + (int64_t)(k0 + BN) * p.k_tok, p.k_tok, si.k_len - k0 - BN, tid);
      vt.load(vbase + (int64_t)(k0 + BN) * p.v_tok, p.v_tok, si.k_len - k0 - BN, tid);
    }
    const bool active = !CAUSAL || (k0 <= wq_last + off);
    if (active) {
      const bool need_mask = (k0 + BN > si.k_len) || (CAUSAL && k0 + BN - 1 > q0 + 32 * w + off);
      f32x16 s[BN / 32], dp[BN / 32];
#pragma unroll
      for (int t = 0; t < BN / 32; ++t) {
        s[t] = zero16();
        dp[t] = zero16();
        const bf16* kr = Ks + (32 * t + perm32(l32)) * RS + 8 * h;
        const bf16* vr = Vs + (32 * t + perm32(l32)) * RS + 8 * h;
#pragma unroll
        for (int ks = 0; ks < D / 16; ++ks) {
          s[t] = mfma32(ld_bf16x8(kr + 16 * ks), qf[ks], s[t]);
          dp[t] = mfma32(ld_bf16x8(vr + 16 * ks), gf[ks], dp[t]);
        }
      }
      bf16x8 db[BN / 16];
#pragma unroll
      for (int t = 0; t < BN / 32; ++t) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float pv = exp2f_fast(s[t][r] * c - lse2);
          if (need_mask) {
            const int kv = k0 + 32 * t + drow(r, h);
            if (kv >= si.k_len || (CAUSAL && kv > qrow + off)) pv = 0.f;
          }
          dp[t][r] = pv * (dp[t][r] - dlt);
        }
        db[2 * t] = pack8(dp[t], 0);
        db[2 * t + 1] = pack8(dp[t], 8);
      }
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt) {
        const bf16* ktr = Kt + (32 * dt + perm32(l32)) * TS + 8 * h;
#pragma unroll
        for (int st = 0; st < BN / 16; ++st) dq[dt] = mfma32(ld_bf16x8(ktr + 16 * st), db[st], dq[dt]);
      }
    }
    if (more) {
      bf16* nx = smem + ((kb + 1) & 1) * STAGE;
      kt.store_rows(nx, tid);
      kt.store_cols(nx + RSZ, tid);
      vt.store_rows(nx + RSZ + TSZ, tid);
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
