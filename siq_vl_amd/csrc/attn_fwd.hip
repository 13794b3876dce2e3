// Varlen (cu_seqlens-packed) flash attention forward for gfx950.
//
// Semantics follow the reference path's eager definition
// (transformers models/qwen2/modeling_qwen2.py:150-172, siglip
// modeling_siglip.py:227-247): O = softmax(scale * Q K^T + mask) V per
// sequence, fp32 softmax, GQA with q-head h reading kv-head h / (Hq / Hkv)
// (repeat_kv, modeling_qwen2.py:138-147); causal masking is bottom-right
// aligned as in the flash-attention varlen contract
// (modeling_flash_attention_utils.py:796-822), identical to top-left when
// len_q == len_k.  Also writes the natural-log LSE the backward needs.
//
// One workgroup = 4 waves = 128 q rows of one q-head of one sequence; the
// (sequence, q-tile) comes from the device-side schedule (heaviest first).
// Each wave owns 32 q rows and keeps its Q fragment in registers as the B
// operand of S^T = K Q^T (v_mfma_f32_32x32x16_bf16), so each lane holds 16
// scores of ONE q row: the online-softmax max is in-lane plus one cross-half
// swap.  P^T then feeds O^T += V^T P^T straight from registers, with V^T read
// from the row-major V tile by ds_read_b64_tr_b16 in the row order of the
// score accumulators (no shuffles).  K and V tiles of 64 kv rows are
// double-buffered in LDS and staged with direct global->LDS loads: the next
// tile is in flight while the current one is multiplied, at no register cost.
//
// Rescaling is lazy: a row's reference max only moves when a block's max
// exceeds it by more than 2^8 (so unnormalised P stays <= 256, exact in the
// fp32 accumulators and in bf16), and the O rescale is skipped for the whole
// wave when no row moved -- after the first block it practically never runs.
//
// The softmax costs few VALU instructions per score: one v_fma_f32 (scale *
// log2(e) and the row's reference, applied to the fp32 score, so large
// logits keep fp32 accuracy) feeding v_exp_f32; the row sum is taken over
// the bf16 P with v_dot2c_f32_bf16 (two per instruction), the cross-half max
// / sum with v_permlane32_swap, and the next block's K / V load offsets are
// computed once per workgroup.
//
// With the rotary embedding fused (ROPE), q arrives before rotation: each lane
// rotates its Q fragment in registers with the cos / sin rows of its token
// (the same bf16 roundings as transformers' apply_rotary_pos_emb, so the
// result is bitwise the separate RoPE pass's) and writes the rotated rows
// once, for the backward.
#include "attn.h"

namespace siq {

namespace {

constexpr float kRescaleLog2 = 8.f;

template <int D, bool CAUSAL, bool ROPE>
__global__ __launch_bounds__(256, 2) void attn_fwd_kernel(const AttnParams p) {
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

  // 1-D grid over (q tile, q-head), q-head fastest: the heads that share a
  // kv-head read the same K / V blocks, so each XCD takes whole tiles (runs
  // of hq entries, sharing K / V through its L2) -- and only one tile per
  // run, so that the heaviest-first tiles are dealt out over the XCDs in
  // turn (longer runs hand the first XCD the heaviest tiles of every round)
  const int e = xcd_order(blockIdx.x, gridDim.x, p.hq);
  const int ti = e / p.hq, hqi = e - ti * p.hq, hk = hqi / p.n_rep;
  const PlanHeader ph = plan_header(p);
  const QTile tl = p.qtiles[ti];
  // every field of the entry and the plan header loaded before the idle
  // test (the compiler would otherwise fetch b alone, wait for it, then
  // fetch the rest)
  asm volatile("" : : "s"(tl.s.q_start), "s"(tl.s.q_len), "s"(tl.s.k_start), "s"(tl.s.k_len), "s"(tl.t),
               "v"(ph.magic));
  if (!plan_header_ok(ph, p, CAUSAL, false) || tl.b < 0) return;
  const SeqInfo si = tl.s;
  const int q0 = tl.t * BM;
  const int off = si.k_len - si.q_len;
  int kv_end = si.k_len;
  if (CAUSAL) kv_end = min(kv_end, q0 + BM + off);
  const int nblk = kv_end > 0 ? (kv_end + BN - 1) / BN : 0;

  const int qrow = q0 + 32 * w + l32;
  const bool qvalid = qrow < si.q_len;
  // last kv row this lane's q row may see
  const int lim = CAUSAL ? min(si.k_len - 1, qrow + off) : si.k_len - 1;
  // The first K / V block goes out before the Q chunks: the loads are
  // untracked (each block's wait_vmem + barrier orders them), so the wait the
  // compiler puts before the first use of Q (or, with the rotation, before
  // rotating it) also covers them, and their latency overlaps Q's.
  const bf16* kbase = p.k + (int64_t)si.k_start * p.k_tok + (int64_t)hk * p.k_head;
  const bf16* vbase = p.v + (int64_t)si.k_start * p.v_tok + (int64_t)hk * p.v_head;
  if (nblk > 0) {
    kt.template issue<true>(kbase, p.k_tok, si.k_len, smem, wu);
    vt.template issue<true>(vbase, p.v_tok, si.k_len, smem + TE, wu);
  }
  bf16x8 qf[D / 16];
  using QStage = LdsTile<BM, D, NT / 64>;
  static_assert(QStage::ELEMS == STAGE && QStage::PERW * QStage::RPI == 32,
                "the q tile fills one K / V stage, and each wave stages its own 32 rows");
  if constexpr (!ROPE) {
    // The q tile goes through LDS, in the second K / V stage (free until the
    // first prefetch of the block loop): the direct loads read whole
    // 256-byte rows, where loading the MFMA operand layout straight into
    // registers touches 32 rows per instruction.  Each wave stages its own 32
    // rows and reads them back after its own load wait.
    QStage qs;
    qs.init(p.q_tok, lane);
    qs.template issue<true>(p.q + (int64_t)(si.q_start + q0) * p.q_tok + (int64_t)hqi * p.q_head, p.q_tok,
                            si.q_len - q0, smem + STAGE, wu);
  } else {
    const int64_t r = si.q_start + (qvalid ? qrow : 0);
    const bf16* qp = p.q + r * p.q_tok + (int64_t)hqi * p.q_head + 8 * h;
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
      const bf16x8 x = ld_bf16x8(qp + 16 * ks);
      qf[ks] = qvalid ? x : zero_bf16x8();
    }
    if constexpr (ROPE) {
      // lane holds d = 16 ks + 8 h + i; its rotation partner d + D / 2 is chunk ks + HK of the same lane
      constexpr int HK = D / 32;
      const bf16* cp = p.rcos + r * p.rc_tok + 8 * h;
      const bf16* sp = p.rsin + r * p.rs_tok + 8 * h;
      // every cos / sin chunk in flight with the q chunks before the first use
      bf16x8 cs[D / 16], sn[D / 16];
#pragma unroll
      for (int ks = 0; ks < D / 16; ++ks) {
        cs[ks] = ld_bf16x8(cp + 16 * ks);
        sn[ks] = ld_bf16x8(sp + 16 * ks);
      }
#pragma unroll
      for (int ks = 0; ks < HK; ++ks) {
        bf16x8 o1, o2;
        rope_fwd8(qf[ks], qf[ks + HK], cs[ks], cs[ks + HK], sn[ks], sn[ks + HK], o1, o2);
        qf[ks] = o1;
        qf[ks + HK] = o2;
      }
      // the rotated rows, for the backward (their stores only join the first
      // block's wait for its K / V loads)
      if (qvalid) {
        bf16* qe = p.qe + (int64_t)(si.q_start + qrow) * p.qe_tok + (int64_t)hqi * p.qe_head + 8 * h;
#pragma unroll
        for (int ks = 0; ks < D / 16; ++ks) st_bf16x8(qe + 16 * ks, qf[ks]);
      }
    }
  }
  // full-tile K / V load offsets, computed once
  uint32_t koff[Tile::PERW], voff[Tile::PERW];
  kt.full_offsets(p.k_tok, wu, koff);
  vt.full_offsets(p.v_tok, wu, voff);

  f32x16 oacc[D / 32];
#pragma unroll
  for (int i = 0; i < D / 32; ++i) oacc[i] = zero16();
  // Scores are taken relative to a per-row reference max mref (log2 units;
  // -inf until the row sees its first key); msafe = mref, or 0 while mref is -inf.
  float mref = -INFINITY, msafe = 0.f, lsum = 0.f;  // lsum: this lane's partial row sum

  wait_vmem();
  asm volatile("" ::: "memory");  // the LDS reads below stay after the wait
  if constexpr (!ROPE) {
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
      const bf16x8 x = rr.read(smem + STAGE, 32 * w, ks);
      qf[ks] = qvalid ? x : zero_bf16x8();
    }
  }
  // every wave's rows read (the first prefetch overwrites the q stage) and
  // the first K / V block visible
  __syncthreads();

  const int wq_last = q0 + 32 * w + 31;  // last q row of this wave
  for (int kb = 0; kb < nblk; ++kb) {
    const bf16* Ks = smem + (kb & 1) * STAGE;
    const bf16* Vs = Ks + TE;
    const int k0 = kb * BN;
    const bool more = kb + 1 < nblk;
    if (more) {
      bf16* nx = smem + ((kb + 1) & 1) * STAGE;
      const bf16* kn = kbase + (int64_t)(k0 + BN) * p.k_tok;
      const bf16* vn = vbase + (int64_t)(k0 + BN) * p.v_tok;
      const int rem = si.k_len - k0 - BN;
      if (rem >= BN) {
        kt.issue_full(kn, koff, nx, wu);
        vt.issue_full(vn, voff, nx + TE, wu);
      } else {
        kt.template issue<true>(kn, p.k_tok, rem, nx, wu);
        vt.template issue<true>(vn, p.v_tok, rem, nx + TE, wu);
      }
    }
    // a wave whose 32 q rows all lie past the sequence end (the tail of the
    // last q-tile) has nothing to compute; it still stages its loads
    const bool active = q0 + 32 * w < si.q_len && (!CAUSAL || (k0 <= wq_last + off));
    if (active) {
      // independent accumulators innermost, so consecutive MFMAs never wait on each other
      f32x16 s[BN / 32];
      // software pipeline: operand reads run two k-steps ahead of the MFMAs
      constexpr int KS = D / 16, NTL = BN / 32;
      bf16x8 ka[KS][NTL];
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int t = 0; t < NTL; ++t) ka[ks][t] = rr.read(Ks, 32 * t, ks);
#pragma unroll
      for (int t = 0; t < NTL; ++t) s[t] = mfma32(ka[0][t], qf[0], zero16());
#pragma unroll
      for (int ks = 1; ks < KS; ++ks)
#pragma unroll
        for (int t = 0; t < NTL; ++t) s[t] = mfma32(ka[ks][t], qf[ks], s[t]);
      __builtin_amdgcn_sched_group_barrier(0x100, 2 * NTL, 0);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        if (ks + 2 < KS) __builtin_amdgcn_sched_group_barrier(0x100, NTL, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, NTL, 0);
      }
      // accumulator (t, r) holds kv = k0 + 32t + nrow(r, h)
      const bool need_mask = (k0 + BN > si.k_len) || (CAUSAL && k0 + BN - 1 > q0 + 32 * w + off);
      if (need_mask) {
        const int rel = lim - k0 - 4 * h;
#pragma unroll
        for (int t = 0; t < BN / 32; ++t)
#pragma unroll
          for (int r = 0; r < 16; ++r) s[t][r] = (32 * t + 8 * (r >> 2) + (r & 3) > rel) ? -INFINITY : s[t][r];
      }
      float mx = -INFINITY;
#pragma unroll
      for (int t = 0; t < BN / 32; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[t][r]);
      mx = half_max(mx) * c;  // block max, log2 units
      // a row moves its reference when it sees its first key or when the
      // block max exceeds the reference by more than 2^kRescaleLog2
      const bool grow = mx > mref + kRescaleLog2;
      if (__any(grow)) {
        // rows that did not grow keep alpha = 1 (also when their max is still -inf)
        const float alpha = grow ? exp2f_fast(mref - mx) : 1.f;
        mref = grow ? mx : mref;
        msafe = mref == -INFINITY ? 0.f : mref;
        lsum *= alpha;
        if (kb > 0) {
#pragma unroll
          for (int i = 0; i < D / 32; ++i) oacc[i] *= alpha;
        }
      }
      bf16x8 pb[BN / 16];
#pragma unroll
      for (int t = 0; t < BN / 32; ++t) {
#pragma unroll
        for (int r = 0; r < 16; ++r) s[t][r] = exp2f_fast(__builtin_fmaf(s[t][r], c, -msafe));
        pb[2 * t] = pack8(s[t], 0);
        pb[2 * t + 1] = pack8(s[t], 8);
      }
      // the row sum over the bf16 P that the PV products use
#pragma unroll
      for (int st = 0; st < BN / 16; ++st) lsum = sum8_bf16(pb[st], lsum);
#pragma unroll
      for (int st = 0; st < BN / 16; ++st)
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) oacc[dt] = mfma32(tr.read(Vs, 16 * st, dt), pb[st], oacc[dt]);
    }
    wait_vmem();
    __syncthreads();
  }

  const float ltot = half_sum(lsum);
  if (qvalid && h == 0) {
    p.lse[(int64_t)hqi * p.lse_head + si.q_start + qrow] = ltot > 0.f ? (mref + __log2f(ltot)) * kLn2 : -INFINITY;
  }
  // O through LDS, so that it leaves as whole 256-byte rows: after the block
  // loop's last barrier no wave reads K / V, and each wave writes and reads
  // back only its own 32 rows (the wave's LDS accesses run in order, so no
  // barrier).  Lane (l32, h) holds d = 32 dt + 16 j + 8 h + i of its row:
  // logical chunk 4 dt + 2 j + h.
  {
    const float inv = ltot > 0.f ? 1.f / ltot : 0.f;
    RowWrite<D> rw;
    rw.init(lane);
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        bf16x8 ov;
#pragma unroll
        for (int i = 0; i < 8; ++i) ov[i] = (bf16)(oacc[dt][8 * j + i] * inv);
        rw.write(smem, 32 * w, 4 * dt + 2 * j + h, ov);
      }
    }
    RowSpan<D> rs;
    rs.init(lane);
    bf16* obase = p.out + (int64_t)(si.q_start + q0) * p.o_tok + (int64_t)hqi * p.o_head + 8 * rs.c;
#pragma unroll
    for (int i = 0; i < RowSpan<D>::N32; ++i) {
      const int r = rs.row(32 * w, i);
      const bf16x8 v = ld_bf16x8(smem + rs.lds(r));
      if (q0 + r < si.q_len) st_bf16x8(obase + (int64_t)r * p.o_tok, v);
    }
  }
}

}  // namespace

template <int D, bool CAUSAL>
hipError_t launch_fwd_t(const AttnParams& p, int qcap, hipStream_t stream) {
  const dim3 grid((unsigned)((int64_t)qcap * p.hq));
  if (p.rcos != nullptr)
    hipLaunchKernelGGL((attn_fwd_kernel<D, CAUSAL, true>), grid, dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL((attn_fwd_kernel<D, CAUSAL, false>), grid, dim3(256), 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_attn_fwd(const AttnParams& p, int d, int causal, int qcap, hipStream_t stream) {
  if (d == 128) return causal ? launch_fwd_t<128, true>(p, qcap, stream) : launch_fwd_t<128, false>(p, qcap, stream);
  if (d == 64) return causal ? launch_fwd_t<64, true>(p, qcap, stream) : launch_fwd_t<64, false>(p, qcap, stream);
  return hipErrorInvalidValue;
}

}  // namespace siq
