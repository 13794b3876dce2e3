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
//    with Q and dO tiles staged in LDS by direct global->LDS loads; dV^T +=
//    dO^T P and dK^T += Q^T dS read dO^T / Q^T with ds_read_b64_tr_b16.  The four waves'
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
  using QTile = LdsTile<BM, D, NT / 64>;
  constexpr int TE = QTile::ELEMS;
  constexpr int STAGE = 2 * TE;  // Q, dO (bf16 elements)
  __shared__ __align__(16) bf16 smem[2 * STAGE];
  __shared__ __align__(16) float rowv[2][2][BM];  // [stage][lse | delta][q] (raw, as loaded)

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, h = lane >> 5, l32 = lane & 31;
  const int wu = wave_uniform(w);
  QTile qt, gt;
  qt.init(p.q_tok, lane);
  gt.init(p.do_tok, lane);
  RowRead<D> rr;
  rr.init(lane);
  TrRead<D> tr;
  tr.init(lane);
  const float c = p.scale_log2;

  const int2 tl = p.kvtiles[blockIdx.x];
  if (tl.x < 0) return;
  const SeqInfo si = p.seq[tl.x];
  const int hk = blockIdx.y;
  const int k0 = tl.y * BN;
  const int off = si.k_len - si.q_len;

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

  // Stage step `step` into buffer `buf`: Q and dO tiles, plus the 128 LSE and
  // Delta values (one 64-lane dword direct load per wave; rows past the end
  // read the last valid row and are fixed at use).
  auto issue = [&](int step, int buf) {
    const int j = step / nqb, qb = qb0 + step - j * nqb;
    const int hq = hk * p.n_rep + j;
    const int q0 = qb * BM;
    const int nrows = si.q_len - q0;
    const int64_t r0 = si.q_start + q0;
    bf16* base = smem + buf * STAGE;
    qt.issue(p.q + r0 * p.q_tok + (int64_t)hq * p.q_head, p.q_tok, nrows, base, wu);
    gt.issue(p.dout + r0 * p.do_tok + (int64_t)hq * p.do_head, p.do_tok, nrows, base + TE, wu);
    const int which = wu >> 1, half = wu & 1;
    const int r = min(64 * half + lane, nrows - 1);
    const float* src = (which == 0 ? p.lse : p.delta) + (int64_t)hq * p.lse_head + r0 + r;
    __builtin_amdgcn_global_load_lds(src, (lds_void*)(&rowv[buf][which][64 * half]), 4, 0, 0);
  };

  if (nsteps > 0) issue(0, 0);
  wait_vmem();
  __syncthreads();

  for (int step = 0; step < nsteps; ++step) {
    const int buf = step & 1;
    const bf16* Qs = smem + buf * STAGE;
    const bf16* Gs = Qs + TE;
    const float* lse = rowv[buf][0];
    const float* dlt = rowv[buf][1];
    const int q0 = (qb0 + step % nqb) * BM;
    const int qvalid = si.q_len - q0;  // rows of this block that exist
    const bool tail = qvalid < BM;
    const bool more = step + 1 < nsteps;
    if (more) issue(step + 1, buf ^ 1);

    const int wq0 = q0 + 32 * w;  // first q row of this wave
    const bool active = !CAUSAL || (wq0 + 31 + off >= k0);
    if (active) {
      const bool need_mask = CAUSAL && (wq0 + off < k0 + 31);
      // accumulator r (= 8j + i) holds q = wq0 + 16j + krow(i, h), kv = kvrow
      f32x16 s = zero16(), dp = zero16();
#pragma unroll
      for (int ks = 0; ks < D / 16; ++ks) {
        s = mfma32(rr.read(Qs, 32 * w, ks), kf[ks], s);
        dp = mfma32(rr.read(Gs, 32 * w, ks), vf[ks], dp);
      }
      const int rel = kvrow - off - wq0 - 4 * h;  // causal: keep q offsets >= rel
      bf16x8 pb[2], db[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int qo = 32 * w + 16 * j + 4 * h;  // krow(i, h) = 4h + i (i < 4), 8 + 4h + i - 4
        const f32x4 l0 = *reinterpret_cast<const f32x4*>(lse + qo);
        const f32x4 l1 = *reinterpret_cast<const f32x4*>(lse + qo + 8);
        const f32x4 d0 = *reinterpret_cast<const f32x4*>(dlt + qo);
        const f32x4 d1 = *reinterpret_cast<const f32x4*>(dlt + qo + 8);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          float lv = (i < 4 ? l0[i] : l1[i - 4]) * kLog2e;
          float dv_ = i < 4 ? d0[i] : d1[i - 4];
          if (tail) {  // rows past the end of the sequence: P = exp2(-inf) = 0, Delta = 0
            const bool ok = qo + 8 * (i >> 2) + (i & 3) < qvalid;
            lv = ok ? lv : INFINITY;
            dv_ = ok ? dv_ : 0.f;
          }
          float pv = exp2f_fast(__builtin_fmaf(s[8 * j + i], c, -lv));
          if (need_mask) pv = (16 * j + 8 * (i >> 2) + (i & 3) < rel) ? 0.f : pv;
          s[8 * j + i] = pv;
          dp[8 * j + i] = pv * (dp[8 * j + i] - dv_);
        }
        pb[j] = pack8(s, 8 * j);
        db[j] = pack8(dp, 8 * j);
      }
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) {
          dv[dt] = mfma32(tr.read(Gs, 32 * w + 16 * j, dt), pb[j], dv[dt]);
          dk[dt] = mfma32(tr.read(Qs, 32 * w + 16 * j, dt), db[j], dk[dt]);
        }
    }
    wait_vmem();
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
  using Tile = LdsTile<BN, D, NT / 64>;
  constexpr int TE = Tile::ELEMS, STAGE = 2 * TE;  // K, V
  __shared__ __align__(16) bf16 smem[2 * STAGE];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, h = lane >> 5, l32 = lane & 31;
  const int wu = wave_uniform(w);
  Tile kt, vt;
  kt.init(p.k_tok, lane);
  vt.init(p.v_tok, lane);
  RowRead<D> rr;
  rr.init(lane);
  TrRead<D> tr;
  tr.init(lane);
  const float c = p.scale_log2;

  const int2 tl = p.qtiles[blockIdx.x];
  if (tl.x < 0) return;
  const SeqInfo si = p.seq[tl.x];
  const int hqi = blockIdx.y, hk = hqi / p.n_rep;
  const int q0 = tl.y * BM;
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

  const bf16* kbase = p.k + (int64_t)si.k_start * p.k_tok + (int64_t)hk * p.k_head;
  const bf16* vbase = p.v + (int64_t)si.k_start * p.v_tok + (int64_t)hk * p.v_head;
  if (nblk > 0) {
    kt.issue(kbase, p.k_tok, si.k_len, smem, wu);
    vt.issue(vbase, p.v_tok, si.k_len, smem + TE, wu);
  }
  wait_vmem();
  __syncthreads();

  const int wq_last = q0 + 32 * w + 31;
  for (int kb = 0; kb < nblk; ++kb) {
    const bf16* Ks = smem + (kb & 1) * STAGE;
    const bf16* Vs = Ks + TE;
    const int k0 = kb * BN;
    const bool more = kb + 1 < nblk;
    if (more) {
      bf16* nx = smem + ((kb + 1) & 1) * STAGE;
      kt.issue(kbase + (int64_t)(k0 + BN) * p.k_tok, p.k_tok, si.k_len - k0 - BN, nx, wu);
      vt.issue(vbase + (int64_t)(k0 + BN) * p.v_tok, p.v_tok, si.k_len - k0 - BN, nx + TE, wu);
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
      }
#pragma unroll
      for (int ks = 0; ks < D / 16; ++ks)
#pragma unroll
        for (int t = 0; t < BN / 32; ++t) {
          s[t] = mfma32(rr.read(Ks, 32 * t, ks), qf[ks], s[t]);
          dp[t] = mfma32(rr.read(Vs, 32 * t, ks), gf[ks], dp[t]);
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
      for (int st = 0; st < BN / 16; ++st)
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) dq[dt] = mfma32(tr.read(Ks, 16 * st, dt), db[st], dq[dt]);
    }
    wait_vmem();
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
