// Varlen flash attention backward for gfx950, deterministic (no atomics) or
// with atomic dQ.
//
// Math (the gradient of the reference's eager attention,
// transformers models/qwen2/modeling_qwen2.py:150-172): with P = softmax(S),
// S = scale * Q K^T + mask, and Delta_i = sum_d dO_id O_id,
//   dV = P^T dO,  dP = dO V^T,  dS = P o (dP - Delta),
//   dQ = scale * dS K,  dK = scale * dS^T Q.
// P is recomputed from the forward's LSE: P = exp2(S * scale * log2e - LSE * log2e).
//
// Kernels, in launch order:
//  * dQ: one workgroup = 4 waves = 128 q rows of one q-head (same schedule as
//    the forward); wave g owns q rows 32 g .. 32 g + 31 with Q and dO in
//    registers as B operands of S^T = K Q^T and dP^T = V dO^T.  Each lane
//    also reads its row's O to form Delta = rowsum(dO o O), and the kernel
//    publishes Delta and LSE * log2(e) for the dK/dV kernel.  K and V tiles
//    of 64 rows are double-buffered row-major in LDS and taken 32 rows at a
//    time (operand reads one k-step ahead of the MFMAs); dQ^T += K^T dS^T reads
//    K^T with ds_read_b64_tr_b16.
//  * dK/dV (D = 128, and the atomic backward): one workgroup = 8 waves =
//    128 kv rows of one kv-head.  Wave
//    (g, kq) owns kv rows 32 kq .. 32 kq + 31 and q rows 32 g .. 32 g + 31 of
//    each 64-row step, so every staged Q / dO tile feeds all 128 kv rows and
//    every SIMD runs two waves.  K and V of the tile sit in LDS as the B
//    operands of S = Q K^T and dP = dO V^T.  A work item walks steps (q block,
//    q-head of the GQA group) of its kv tile, with Q / dO / LSE2 / Delta
//    double-buffered in LDS by direct global->LDS loads and the operand reads
//    one k-step ahead of the MFMAs; dV^T += dO^T P and dK^T += Q^T dS read
//    dO^T / Q^T with ds_read_b64_tr_b16.  The two q-group waves' partial
//    dK/dV of each kv quarter are summed through LDS.  Tiles heavier than the
//    scheduler's piece length run as several work items writing fp32 sums to
//    workspace slots,
//  * which the partial-sum kernel adds in piece order afterwards.
// At D = 64 the deterministic backward's dK/dV kernel is
// attn_bwd_dkdv_w4_kernel (one wave per SIMD, K and V in registers); the
// atomic backward replaces the dQ kernel with a Delta / LSE2 pass, dQ formed
// in the 8-wave dK/dV kernel, and a conversion of the fp32 sums.
// With the rotary embedding fused, the dQ kernel reads the rotated q the
// forward wrote and stores dq through the rotation's backward (the separate
// RoPE backward pass's exact roundings); dK stays the gradient of the rotated
// k, for a k-only RoPE backward pass.
#include "attn.h"

namespace siq {

namespace {

// Atomic dQ (DQ = true, the non-deterministic backward): the dK/dV kernel
// also forms dQ = dS K, so no second kernel recomputes S and dP.  Each wave
// writes its 32 x 32 block of dS (bf16) to an LDS exchange buffer [64 q][128
// kv] (rows padded to 136 elements: consecutive rows start one 16-byte bank
// group apart, so the row reads below are conflict free and every write of a
// lane is its base plus a constant); after a barrier wave (g, kq) multiplies
// the q rows of group g by K for d-tile kq % NDT over the kv quarters of part
// kq / NDT (all four at D = 128, two at D = 64) and adds the fp32 result to a
// dQ workspace with vector atomics, issued after the step's closing barrier so
// that its load wait does not also wait for them.  kv offset o of each 16-kv
// group is stored at slot o with bits 2 and 3 swapped, so that a row read
// returns the kv order of a transposed K read (TrRead's krow).
constexpr int kDsxLd = kBwdBN + 8;
__device__ __forceinline__ int dsx_slot(int kv) {
  return (kv & ~15) | (kv & 3) | ((kv & 4) << 1) | ((kv & 8) >> 1);
}

template <int D, bool CAUSAL, bool DQ>
__global__ __launch_bounds__(512, 1) void attn_bwd_dkdv_kernel(const AttnParams p) {
  constexpr int BN = kBwdBN, BM = kBwdBM, NT = 512, NW = NT / 64, NS = 2;
  static_assert(BN == 128 && BM == 64, "128 kv rows (4 x 32) by 64 q rows (2 x 32) per step");
  using StTile = LdsTile<BM, D, NW / 2>;  // Q staged by waves 0-3, dO by waves 4-7
  using KVTile = LdsTile<BN, D, NW>;
  constexpr int TE = StTile::ELEMS;
  constexpr int STAGE = 2 * TE;  // Q, dO (bf16 elements)
  constexpr int NDT = D / 32;
  constexpr int SMEM = NS * STAGE + 2 * KVTile::ELEMS;  // stages, K, V
  static_assert(2 * 4 * NDT * 16 * 64 * 4 <= SMEM * 2, "one reduction round fits the LDS");
  __shared__ __align__(16) bf16 smem[SMEM];
  __shared__ __align__(16) float rowv[NS][2][BM];  // [stage][lse2 | delta][q] (raw, as loaded)
  __shared__ __align__(16) bf16 dsx[DQ ? BM * kDsxLd : 8];  // dS exchange (atomic dQ)

  const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, l32 = lane & 31;
  const int wu = wave_uniform(tid >> 6);
  const int g = wu & 1, kq = wu >> 1;     // q group (32 rows of a step), kv quarter (32 rows of the tile)
  const bool stages_q = wu < 4;           // waves 0-3 stage Q, waves 4-7 stage dO
  const bool stages_row = (wu & 3) == 0;  // waves 0 / 4 also stage the step's LSE2 / Delta
  StTile st;
  st.init(stages_q ? p.q_tok : p.do_tok, lane);
  KVTile kt, vt;
  kt.init(p.k_tok, lane);
  vt.init(p.v_tok, lane);
  RowRead<D> rr;
  rr.init(lane);
  TrRead<D> tr;
  tr.init(lane);
  const float c = p.scale_log2;
  bf16* Ks = smem + NS * STAGE;
  bf16* Vs = Ks + KVTile::ELEMS;

  // 1-D grid over (item, kv-head), kv-head fastest; each XCD takes one item
  // (all its kv-heads) per run, so the heaviest-first items go round the XCDs
  const int e = xcd_order(blockIdx.x, gridDim.x, p.hkv);
  const int ii = e / p.hkv, hk = e - ii * p.hkv;
  const PlanHeader ph = plan_header(p);
  const KvItem it = p.kvitems[ii];
  // every field of the entry and the plan header loaded before the idle
  // test (the compiler would otherwise fetch b alone, wait for it, then
  // fetch the rest)
  asm volatile("" : : "s"(it.s.q_start), "s"(it.s.q_len), "s"(it.s.k_start), "s"(it.s.k_len), "s"(it.t), "s"(it.s0),
               "s"(it.s1), "v"(ph.magic));
  if (!plan_header_ok(ph, p, CAUSAL, true) || it.b < 0) return;
  const SeqInfo si = it.s;
  const int k0 = it.t * BN;
  const int kb = k0 + 32 * kq;  // first kv row of this wave
  const int off = si.k_len - si.q_len;

  const int kvrow = kb + l32;
  const bool kvvalid = kvrow < si.k_len;
  // K and V of the tile in LDS (rows past the end repeat the last row: they
  // only reach dK / dV rows that are never written)
  kt.template issue<true>(p.k + (int64_t)(si.k_start + k0) * p.k_tok + (int64_t)hk * p.k_head, p.k_tok, si.k_len - k0,
                          Ks, wu);
  vt.template issue<true>(p.v + (int64_t)(si.k_start + k0) * p.v_tok + (int64_t)hk * p.v_head, p.v_tok, si.k_len - k0,
                          Vs, wu);
  f32x16 dk[NDT], dv[NDT];
#pragma unroll
  for (int i = 0; i < NDT; ++i) {
    dk[i] = zero16();
    dv[i] = zero16();
  }

  // The tile's steps are (q block qb, q-head j of the GQA group) for the q
  // blocks that can see any of its rows, q blocks from the last one down, the
  // n_rep heads inside; this item runs steps [s0, s1).
  const int qb_last = (si.q_len - 1) / BM;
  const int s0 = it.s0, ns = it.s1 - it.s0;

  // this wave's source tensor (Q or dO, and LSE2 or Delta), pinned so the
  // step loop does not re-read the kernel arguments
  const bf16* sbase = stages_q ? p.q : p.dout;
  int64_t stok = stages_q ? p.q_tok : p.do_tok;
  int64_t shead = stages_q ? p.q_head : p.do_head;
  const float* rbase = stages_q ? p.lse2 : p.delta;
  int64_t lhead = p.lse_head;
  pin_sgpr(sbase);
  pin_sgpr(stok);
  pin_sgpr(shead);
  pin_sgpr(rbase);
  pin_sgpr(lhead);
  // Loads untracked: the step loop's wait_vmem + barrier order them.  A step's
  // loads are described once (src, nrows, buf) and issued one instruction at
  // a time (issue_k), spread over the previous step's S / dP MFMAs so that the
  // waves do not all wait on the load queue at the start of a step.
  struct StepLoad {
    const bf16* src;
    const float* rsrc;
    int nrows, buf;
  };
  auto describe = [&](int step, int buf) {
    const int j = step % p.n_rep, qb = qb_last - step / p.n_rep;
    const int hq = hk * p.n_rep + j;
    const int q0 = qb * BM;
    const int64_t r0 = si.q_start + q0;
    return StepLoad{sbase + r0 * stok + (int64_t)hq * shead, rbase + (int64_t)hq * lhead + r0, si.q_len - q0, buf};
  };
  auto issue_k = [&](const StepLoad& l, int k) {
    st.template issue_one<true>(k, l.src, stok, l.nrows, smem + l.buf * STAGE + (stages_q ? 0 : TE), wu & 3);
    if (k == 0 && stages_row)
      dma4_untracked(l.rsrc + min(lane, l.nrows - 1), &rowv[l.buf][stages_q ? 0 : 1][0]);
  };
  auto issue = [&](int step, int buf) {
    const StepLoad l = describe(step, buf);
#pragma unroll
    for (int k = 0; k < StTile::PERW; ++k) issue_k(l, k);
  };
  constexpr int KPI = (D / 16) / StTile::PERW;  // S / dP k-steps per spread load instruction
  static_assert(KPI >= 1 && (D / 16) % StTile::PERW == 0, "loads spread evenly over the k-steps");

  // atomic dQ: this wave's d-tile and kv quarters
  constexpr int WPT = 4 / NDT;                  // waves per d-tile
  const int qdt = kq % NDT, qpart = kq / NDT;   // d-tile, kv-quarter part

  if (ns > 0) issue(s0, 0);
  wait_vmem();
  __syncthreads();
  // At D = 64 this wave's 32 kv rows of K and V stay in registers as the B
  // operands of S = Q K^T and dP = dO V^T for every step of the item (a third
  // of the step's LDS reads); at D = 128 they do not fit beside the dK / dV
  // accumulators and are read from LDS each step.
  constexpr bool KVREG = D <= 64;
  bf16x8 kreg[KVREG ? D / 16 : 1], vreg[KVREG ? D / 16 : 1];
  if constexpr (KVREG) {
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
      kreg[ks] = rr.read(Ks, 32 * kq, ks);
      vreg[ks] = rr.read(Vs, 32 * kq, ks);
    }
  }

  for (int i = 0; i < ns; ++i) {
    const int step = s0 + i;
    const int buf = i % NS;
    const bf16* Qs = smem + buf * STAGE;
    const bf16* Gs = Qs + TE;
    const float* lse2 = rowv[buf][0];
    const float* dlt = rowv[buf][1];
    const int q0 = (qb_last - step / p.n_rep) * BM;
    const int qvalid = si.q_len - q0;  // rows of this block that exist
    const bool pf = i + 1 < ns;
    const StepLoad nl = describe(step + 1, buf ^ 1);

    const int wq0 = q0 + 32 * g;  // first q row of this wave
    // kv quarters past the sequence end have nothing to accumulate
    auto quarter_active = [&](int qq) {
      const int kq0 = k0 + 32 * qq;
      return 32 * g < qvalid && kq0 < si.k_len && (!CAUSAL || wq0 + 31 + off >= kq0);
    };
    const bool active = quarter_active(kq);
    if (!active && pf) {
#pragma unroll
      for (int k = 0; k < StTile::PERW; ++k) issue_k(nl, k);
    }
    if (active) {
      // accumulator r (= 8j + i) holds q = wq0 + 16j + 8(i / 4) + 4h + i % 4, kv = kvrow
      // operand fragments double-buffered one k-step ahead of the MFMAs
      f32x16 s = zero16(), dp = zero16();
      bf16x8 fq[2], fg[2], fk[2], fv[2];
      fq[0] = rr.read(Qs, 32 * g, 0);
      fg[0] = rr.read(Gs, 32 * g, 0);
      if constexpr (!KVREG) {
        fk[0] = rr.read(Ks, 32 * kq, 0);
        fv[0] = rr.read(Vs, 32 * kq, 0);
      }
#pragma unroll
      for (int ks = 0; ks < D / 16; ++ks) {
        const int cur = ks & 1;
        if (pf && ks % KPI == 0) issue_k(nl, ks / KPI);
        if (ks + 1 < D / 16) {
          fq[cur ^ 1] = rr.read(Qs, 32 * g, ks + 1);
          fg[cur ^ 1] = rr.read(Gs, 32 * g, ks + 1);
          if constexpr (!KVREG) {
            fk[cur ^ 1] = rr.read(Ks, 32 * kq, ks + 1);
            fv[cur ^ 1] = rr.read(Vs, 32 * kq, ks + 1);
          }
        }
        if constexpr (KVREG) {
          s = mfma32(fq[cur], kreg[ks], s);
          dp = mfma32(fg[cur], vreg[ks], dp);
        } else {
          s = mfma32(fq[cur], fk[cur], s);
          dp = mfma32(fg[cur], fv[cur], dp);
        }
      }
      // P = exp2(S scale log2e - LSE2), dS = P (dP - Delta), in place; on the
      // causal diagonal and past the end of the sequence the exponent is -inf
      // (P = 0, hence dS = 0)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int qo = 32 * g + 16 * j + 4 * h;
        const f32x4 l0 = *reinterpret_cast<const f32x4*>(lse2 + qo);
        const f32x4 l1 = *reinterpret_cast<const f32x4*>(lse2 + qo + 8);
        const f32x4 d0 = *reinterpret_cast<const f32x4*>(dlt + qo);
        const f32x4 d1 = *reinterpret_cast<const f32x4*>(dlt + qo + 8);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          s[8 * j + e] = __builtin_fmaf(s[8 * j + e], c, -(e < 4 ? l0[e] : l1[e - 4]));
          dp[8 * j + e] -= e < 4 ? d0[e] : d1[e - 4];
        }
      }
      if (32 * g + 32 > qvalid || (CAUSAL && wq0 + off < kb + 31)) {
        const int rel = CAUSAL ? kvrow - off - wq0 - 4 * h : -(1 << 30);  // keep q offsets >= rel
        const int lim = qvalid - 32 * g - 4 * h;                            // keep q offsets < lim
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int qoff = 8 * (r >> 2) + (r & 3);
          s[r] = (qoff >= rel && qoff < lim) ? s[r] : -INFINITY;
        }
      }
      bf16x8 pb[2], db[2];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        s[r] = exp2f_fast(s[r]);
        dp[r] *= s[r];
      }
      pb[0] = pack8(s, 0);
      pb[1] = pack8(s, 8);
      db[0] = pack8(dp, 0);
      db[1] = pack8(dp, 8);
      if constexpr (DQ) {
        // this wave's dS block into the exchange buffer: q = 32 g + 4 h + 8 (r / 4) + r % 4, kv = 32 kq + l32.
        // kv rows past the sequence end hold the last row's K (their dK / dV rows are never written, but
        // dQ sums over kv): their dS is written as zero
        bf16* w = dsx + (32 * g + 4 * h) * kDsxLd + dsx_slot(32 * kq + l32);
#pragma unroll
        for (int r = 0; r < 16; ++r) w[(8 * (r >> 2) + (r & 3)) * kDsxLd] = kvvalid ? db[r >> 3][r & 7] : (bf16)0.f;
      }
      bf16x8 tg[2], tq[2];
      tg[0] = tr.read(Gs, 32 * g, 0);
      tq[0] = tr.read(Qs, 32 * g, 0);
#pragma unroll
      for (int u = 0; u < 2 * NDT; ++u) {
        const int j = u / NDT, dt = u % NDT, cur = u & 1;
        if (u + 1 < 2 * NDT) {
          const int j1 = (u + 1) / NDT, dt1 = (u + 1) % NDT;
          tg[cur ^ 1] = tr.read(Gs, 32 * g + 16 * j1, dt1);
          tq[cur ^ 1] = tr.read(Qs, 32 * g + 16 * j1, dt1);
        }
        dv[dt] = mfma32(tg[cur], pb[j], dv[dt]);
        dk[dt] = mfma32(tq[cur], db[j], dk[dt]);
      }
    }
    if constexpr (DQ) {
      // every wave's dS block is in the exchange buffer after this barrier
      __syncthreads();
      // dQ[q][d] = sum dS[q][kv] K[kv][d] for q rows 32 g .., d-tile qdt, this part's kv quarters
      f32x16 dqa = zero16();
      bool any = false;
#pragma unroll
      for (int u = 0; u < 4 / WPT; ++u) {
        const int qq = qpart * (4 / WPT) + u;
        if (!quarter_active(qq)) continue;
        any = true;
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          const bf16x8 a = ld_bf16x8(dsx + (32 * g + l32) * kDsxLd + 8 * h + 16 * (2 * qq + kk));
          const bf16x8 b = tr.read(Ks, 32 * qq + 16 * kk, qdt);
          dqa = mfma32(a, b, dqa);
        }
      }
      // the next stage's loads first (the atomics below also count in vmcnt), then the sums
      wait_vmem();
      if (any) {
        // wave-uniform base (first row of the group, its q-head) plus a 32-bit lane offset
        float* base = p.dq_acc + ((int64_t)(si.q_start + wq0) * p.hq + hk * p.n_rep + step % p.n_rep) * D;
        uint32_t rs = (uint32_t)(p.hq * D);
        uint32_t lo = (uint32_t)(32 * qdt + perm32(l32)) + (uint32_t)(4 * h) * rs;
        // recomputed here each step: hoisted out of the loop, the 16 row offsets would hold 16 registers
        asm volatile("" : "+s"(rs), "+v"(lo));
        const int rows = qvalid - 32 * g;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int i = 8 * (r >> 2) + (r & 3);
          if (i + 4 * h < rows) __builtin_amdgcn_global_atomic_fadd_f32(base + lo + (uint32_t)i * rs, dqa[r]);
        }
      }
    } else {
      wait_vmem();
    }
    __syncthreads();
  }

  // Sum the two q-group waves' partial dK^T / dV^T of each kv quarter in one
  // exchange through LDS: wave g finishes d-tiles [g NDT / 2, (g + 1) NDT / 2)
  // of both tensors and hands the other half of its partials to its partner
  // (wave 1 - g of the quarter), with 16-byte LDS stores of 1 KB per
  // instruction.  Each sum is g = 0's partial plus g = 1's.  A whole tile
  // (np == 1) is scaled and written as bf16; a piece of a split tile writes
  // its fp32 sums to its slot ([dK | dV][kv row][d]) for
  // attn_bwd_dkv_sum_kernel.
  const bool split = it.np > 1;
  const bool slot_ok = split && it.slot0 >= 0 && (it.slot0 + it.np) * p.hkv <= kSplitSlots;
  float* slot = p.dkv_part + (int64_t)((it.slot0 + it.piece) * p.hkv + hk) * (2 * BN * D);
  const int64_t row = si.k_start + kvrow;
  constexpr int HT = NDT / 2;             // d-tiles a wave finishes
  constexpr int XR = 2 * HT * 16 * 64;    // floats a wave hands its partner: [dK | dV][HT][16][64 lanes]
  static_assert(8 * XR * 4 <= SMEM * 2, "the exchange fits the LDS");
  float* inbox = reinterpret_cast<float*>(smem) + (2 * kq + g) * XR;
  float* outbox = reinterpret_cast<float*>(smem) + (2 * kq + (1 - g)) * XR;
  // the step loop ends on a barrier; an item without steps has only read K / V (D = 64) since the last one
  if (ns == 0) __syncthreads();
  // d-tiles are indexed statically (a wave-uniform branch picks them), so
  // the accumulators stay in registers
#pragma unroll
  for (int t = 0; t < NDT; ++t) {
    if (t / HT == g) continue;  // this wave finishes tile t itself
    const int u = t % HT;
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      *reinterpret_cast<f32x4*>(outbox + ((0 * HT + u) * 4 + q4) * 256 + 4 * lane) =
          f32x4{dk[t][4 * q4], dk[t][4 * q4 + 1], dk[t][4 * q4 + 2], dk[t][4 * q4 + 3]};
      *reinterpret_cast<f32x4*>(outbox + ((1 * HT + u) * 4 + q4) * 256 + 4 * lane) =
          f32x4{dv[t][4 * q4], dv[t][4 * q4 + 1], dv[t][4 * q4 + 2], dv[t][4 * q4 + 3]};
    }
  }
  __syncthreads();
#pragma unroll
  for (int which = 0; which < 2; ++which) {
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      if (dt / HT != g) continue;  // the partner finishes tile dt
      const int u = dt % HT;
      const f32x16& mine = which == 0 ? dk[dt] : dv[dt];
      float sum[16];
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const f32x4 o = *reinterpret_cast<const f32x4*>(inbox + ((which * HT + u) * 4 + q4) * 256 + 4 * lane);
#pragma unroll
        for (int i = 0; i < 4; ++i) sum[4 * q4 + i] = g == 0 ? mine[4 * q4 + i] + o[i] : o[i] + mine[4 * q4 + i];
      }
      if (!split) {
        if (kvvalid) {
          bf16* dst = which == 0 ? p.dk + row * p.dk_tok + (int64_t)hk * p.dk_head
                                 : p.dv + row * p.dv_tok + (int64_t)hk * p.dv_head;
          const float sc = which == 0 ? p.scale : 1.f;
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            bf16x8 o;
#pragma unroll
            for (int q = 0; q < 8; ++q) o[q] = (bf16)(sum[8 * j + q] * sc);
            st_bf16x8(dst + 32 * dt + 16 * j + 8 * h, o);
          }
        }
      } else if (slot_ok) {
        float* dst = slot + ((int64_t)which * BN + 32 * kq + l32) * D + 32 * dt + 8 * h;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          *reinterpret_cast<f32x4*>(dst + 16 * j) = f32x4{sum[8 * j], sum[8 * j + 1], sum[8 * j + 2], sum[8 * j + 3]};
          *reinterpret_cast<f32x4*>(dst + 16 * j + 4) =
              f32x4{sum[8 * j + 4], sum[8 * j + 5], sum[8 * j + 6], sum[8 * j + 7]};
        }
      }
    }
  }
}

// dK/dV with one wave per SIMD (the deterministic backward's kernel at D =
// 64; measured 15% faster than attn_bwd_dkdv_kernel on the SigLIP shape): one
// workgroup = 4 waves = 128 kv rows of one kv-head, wave w owning kv rows
// 32 w .. 32 w + 31 of the tile for the whole work item.  K and V of those
// rows stay in registers as the B operands of S = Q K^T and dP = dO V^T (a
// wave has the SIMD's 512 registers), and each wave accumulates dK^T / dV^T
// over both 32-row q groups of every 64-row step, so no partial sums cross
// waves.  The products of the two groups are interleaved (four independent
// accumulator chains).  Q / dO / LSE2 / Delta of each step are
// double-buffered in LDS by direct global->LDS loads, spread over the
// previous step's S / dP products; dV^T += dO^T P and dK^T += Q^T dS read
// dO^T / Q^T with ds_read_b64_tr_b16.  Work items, steps and split-tile slots
// are those of attn_bwd_dkdv_kernel.
template <int D, bool CAUSAL>
__global__ __launch_bounds__(256, 1) void attn_bwd_dkdv_w4_kernel(const AttnParams p) {
  constexpr int BN = kBwdBN, BM = kBwdBM, NT = 256, NW = NT / 64, NS = 2;
  static_assert(BN == 128 && BM == 64, "128 kv rows (4 x 32) by 64 q rows (2 x 32) per step");
  using StTile = LdsTile<BM, D, NW>;  // Q and dO, each staged by all four waves
  constexpr int TE = StTile::ELEMS;
  constexpr int STAGE = 2 * TE;  // Q, dO (bf16 elements)
  constexpr int NDT = D / 32, KS = D / 16;
  __shared__ __align__(16) bf16 smem[NS * STAGE];
  __shared__ __align__(16) float rowv[NS][2][BM];  // [stage][lse2 | delta][q] (raw, as loaded)

  const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, l32 = lane & 31;
  const int wu = wave_uniform(tid >> 6);
  StTile st;
  st.init(p.q_tok, lane);
  RowRead<D> rr;
  rr.init(lane);
  TrRead<D> tr;
  tr.init(lane);
  const float c = p.scale_log2;

  // 1-D grid over (item, kv-head), kv-head fastest; each XCD takes one item
  // (all its kv-heads) per run, so the heaviest-first items go round the XCDs
  const int e = xcd_order(blockIdx.x, gridDim.x, p.hkv);
  const int ii = e / p.hkv, hk = e - ii * p.hkv;
  const PlanHeader ph = plan_header(p);
  const KvItem it = p.kvitems[ii];
  asm volatile("" : : "s"(it.s.q_start), "s"(it.s.q_len), "s"(it.s.k_start), "s"(it.s.k_len), "s"(it.t), "s"(it.s0),
               "s"(it.s1), "v"(ph.magic));
  if (!plan_header_ok(ph, p, CAUSAL, true) || it.b < 0) return;
  const SeqInfo si = it.s;
  const int k0 = it.t * BN;
  const int kb = k0 + 32 * wu;  // first kv row of this wave
  const int off = si.k_len - si.q_len;
  const int kvrow = kb + l32;
  const bool kvvalid = kvrow < si.k_len;

  // K and V rows of this wave in registers, in the row-operand layout (lane:
  // row l32, d = 16 ks + 8 h .. +7); rows past the end repeat the last row
  // (they only reach dK / dV rows that are never written)
  bf16x8 kreg[KS], vreg[KS];
  {
    const int r = max(0, min(kvrow, si.k_len - 1));
    const bf16* kp = p.k + (int64_t)(si.k_start + r) * p.k_tok + (int64_t)hk * p.k_head + 8 * h;
    const bf16* vp = p.v + (int64_t)(si.k_start + r) * p.v_tok + (int64_t)hk * p.v_head + 8 * h;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      kreg[ks] = ld_bf16x8(kp + 16 * ks);
      vreg[ks] = ld_bf16x8(vp + 16 * ks);
    }
  }
  f32x16 dk[NDT], dv[NDT];
#pragma unroll
  for (int i = 0; i < NDT; ++i) {
    dk[i] = zero16();
    dv[i] = zero16();
  }

  // steps (q block qb, q-head j of the GQA group): q blocks from the last one
  // down, the n_rep heads inside; this item runs steps [s0, s1)
  const int qb_last = (si.q_len - 1) / BM;
  const int s0 = it.s0, ns = it.s1 - it.s0;
  int64_t qtok = p.q_tok, qhead = p.q_head, gtok = p.do_tok, ghead = p.do_head, lhead = p.lse_head;
  pin_sgpr(qtok);
  pin_sgpr(qhead);
  pin_sgpr(gtok);
  pin_sgpr(ghead);
  pin_sgpr(lhead);
  struct StepLoad {
    const bf16* q;
    const bf16* g;
    const float* rsrc;  // LSE2 (wave 0) or Delta (wave 1) of the step's rows
    int nrows, buf;
  };
  auto describe = [&](int step, int buf) {
    const int j = step % p.n_rep, qb = qb_last - step / p.n_rep;
    const int hq = hk * p.n_rep + j;
    const int q0 = qb * BM;
    const int64_t r0 = si.q_start + q0;
    const float* rb = (wu == 0 ? p.lse2 : p.delta) + (int64_t)hq * lhead + r0;
    return StepLoad{p.q + r0 * qtok + (int64_t)hq * qhead, p.dout + r0 * gtok + (int64_t)hq * ghead, rb, si.q_len - q0,
                    buf};
  };
  // instruction k < PERW: Q, PERW .. 2 PERW - 1: dO; waves 0 / 1 also stage LSE2 / Delta with k == 0
  auto issue_k = [&](const StepLoad& l, int k) {
    bf16* dst = smem + l.buf * STAGE;
    if (k < StTile::PERW)
      st.template issue_one<true>(k, l.q, qtok, l.nrows, dst, wu);
    else
      st.template issue_one<true>(k - StTile::PERW, l.g, gtok, l.nrows, dst + TE, wu);
    if (k == 0 && wu < 2) dma4_untracked(l.rsrc + min(lane, l.nrows - 1), &rowv[l.buf][wu][0]);
  };
  constexpr int NLD = 2 * StTile::PERW;
  static_assert(KS % NLD == 0, "loads spread evenly over the k-steps");
  constexpr int KPI = KS / NLD;  // S / dP k-steps per spread load instruction

  if (ns > 0) {
    const StepLoad l = describe(s0, 0);
#pragma unroll
    for (int k = 0; k < NLD; ++k) issue_k(l, k);
  }
  wait_vmem();
  __syncthreads();

  for (int i = 0; i < ns; ++i) {
    const int step = s0 + i;
    const int buf = i % NS;
    const bf16* Qs = smem + buf * STAGE;
    const bf16* Gs = Qs + TE;
    const float* lse2 = rowv[buf][0];
    const float* dlt = rowv[buf][1];
    const int q0 = (qb_last - step / p.n_rep) * BM;
    const int qvalid = si.q_len - q0;  // rows of this block that exist
    const bool pf = i + 1 < ns;
    const StepLoad nl = describe(step + 1, buf ^ 1);
    // a q group contributes when it has rows and, causally, some row sees this wave's kv rows
    auto group_active = [&](int g) {
      return 32 * g < qvalid && kb < si.k_len && (!CAUSAL || q0 + 32 * g + 31 + off >= kb);
    };
    const bool act0 = group_active(0), act1 = group_active(1);
    if (!act0 && !act1) {
      if (pf) {
#pragma unroll
        for (int k = 0; k < NLD; ++k) issue_k(nl, k);
      }
    } else {
      // S_g = Q_g K^T, dP_g = dO_g V^T for both q groups, interleaved; accumulator r (= 8j + i)
      // holds q = q0 + 32 g + 16 j + 8 (i / 4) + 4 h + i % 4, kv = kvrow.  Q / dO fragments one
      // k-step ahead of the MFMAs.
      f32x16 s[2], dp[2];
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        s[g] = zero16();
        dp[g] = zero16();
      }
      bf16x8 fq[2][2], fg[2][2];  // [buffer][group]
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        fq[0][g] = rr.read(Qs, 32 * g, 0);
        fg[0][g] = rr.read(Gs, 32 * g, 0);
      }
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int cur = ks & 1;
        if (pf && ks % KPI == 0) issue_k(nl, ks / KPI);
        if (ks + 1 < KS) {
#pragma unroll
          for (int g = 0; g < 2; ++g) {
            fq[cur ^ 1][g] = rr.read(Qs, 32 * g, ks + 1);
            fg[cur ^ 1][g] = rr.read(Gs, 32 * g, ks + 1);
          }
        }
#pragma unroll
        for (int g = 0; g < 2; ++g) {
          s[g] = mfma32(fq[cur][g], kreg[ks], s[g]);
          dp[g] = mfma32(fg[cur][g], vreg[ks], dp[g]);
        }
      }
      // P = exp2(S scale log2e - LSE2), dS = P (dP - Delta); masked entries (causal, past the
      // end of the sequence) get P = 0, hence dS = 0
      bf16x8 pb[2][2], db[2][2];  // [group][j]
#pragma unroll
      for (int g = 0; g < 2; ++g) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int qo = 32 * g + 16 * j + 4 * h;
          const f32x4 l0 = *reinterpret_cast<const f32x4*>(lse2 + qo);
          const f32x4 l1 = *reinterpret_cast<const f32x4*>(lse2 + qo + 8);
          const f32x4 d0 = *reinterpret_cast<const f32x4*>(dlt + qo);
          const f32x4 d1 = *reinterpret_cast<const f32x4*>(dlt + qo + 8);
#pragma unroll
          for (int e2 = 0; e2 < 8; ++e2) {
            s[g][8 * j + e2] = __builtin_fmaf(s[g][8 * j + e2], c, -(e2 < 4 ? l0[e2] : l1[e2 - 4]));
            dp[g][8 * j + e2] -= e2 < 4 ? d0[e2] : d1[e2 - 4];
          }
        }
        const int wq0 = q0 + 32 * g;
        if (32 * g + 32 > qvalid || (CAUSAL && wq0 + off < kb + 31)) {
          const int rel = CAUSAL ? kvrow - off - wq0 - 4 * h : -(1 << 30);  // keep q offsets >= rel
          const int lim = qvalid - 32 * g - 4 * h;                            // keep q offsets < lim
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int qoff = 8 * (r >> 2) + (r & 3);
            s[g][r] = (qoff >= rel && qoff < lim) ? s[g][r] : -INFINITY;
          }
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          s[g][r] = exp2f_fast(s[g][r]);
          dp[g][r] *= s[g][r];
        }
        pb[g][0] = pack8(s[g], 0);
        pb[g][1] = pack8(s[g], 8);
        db[g][0] = pack8(dp[g], 0);
        db[g][1] = pack8(dp[g], 8);
      }
      // dV^T += dO^T P, dK^T += Q^T dS over the step's 64 q rows (transposed reads one ahead)
      constexpr int NU = 4 * NDT;  // (group, j, d-tile)
      bf16x8 tg[2], tq[2];
      tg[0] = tr.read(Gs, 0, 0);
      tq[0] = tr.read(Qs, 0, 0);
#pragma unroll
      for (int u = 0; u < NU; ++u) {
        const int gj = u / NDT, dt = u % NDT, cur = u & 1;
        if (u + 1 < NU) {
          const int gj1 = (u + 1) / NDT, dt1 = (u + 1) % NDT;
          tg[cur ^ 1] = tr.read(Gs, 16 * gj1, dt1);
          tq[cur ^ 1] = tr.read(Qs, 16 * gj1, dt1);
        }
        dv[dt] = mfma32(tg[cur], pb[gj >> 1][gj & 1], dv[dt]);
        dk[dt] = mfma32(tq[cur], db[gj >> 1][gj & 1], dk[dt]);
      }
    }
    wait_vmem();
    __syncthreads();
  }

  // A whole tile (np == 1): dK (scaled) and dV of this wave's rows as bf16; a
  // piece of a split tile: its fp32 sums to its slot ([dK | dV][kv row][d])
  // for attn_bwd_dkv_sum_kernel.  Lane holds d = 32 dt + 16 j + 8 h + q.
  const bool split = it.np > 1;
  const bool slot_ok = split && it.slot0 >= 0 && (it.slot0 + it.np) * p.hkv <= kSplitSlots;
  float* slot = p.dkv_part + (int64_t)((it.slot0 + it.piece) * p.hkv + hk) * (2 * BN * D);
  const int64_t row = si.k_start + kvrow;
  auto store = [&](const f32x16 (&acc)[NDT], int which) {
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      if (!split) {
        if (kvvalid) {
          bf16* dst = which == 0 ? p.dk + row * p.dk_tok + (int64_t)hk * p.dk_head
                                 : p.dv + row * p.dv_tok + (int64_t)hk * p.dv_head;
          const float sc = which == 0 ? p.scale : 1.f;
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            bf16x8 o;
#pragma unroll
            for (int q = 0; q < 8; ++q) o[q] = (bf16)(acc[dt][8 * j + q] * sc);
            st_bf16x8(dst + 32 * dt + 16 * j + 8 * h, o);
          }
        }
      } else if (slot_ok) {
        float* dst = slot + ((int64_t)which * BN + 32 * wu + l32) * D + 32 * dt + 8 * h;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const f32x16& a = acc[dt];
          *reinterpret_cast<f32x4*>(dst + 16 * j) = f32x4{a[8 * j], a[8 * j + 1], a[8 * j + 2], a[8 * j + 3]};
          *reinterpret_cast<f32x4*>(dst + 16 * j + 4) = f32x4{a[8 * j + 4], a[8 * j + 5], a[8 * j + 6], a[8 * j + 7]};
        }
      }
    }
  };
  store(dk, 0);
  store(dv, 1);
}

// dK / dV of split tiles: the pieces' fp32 sums added in piece order (so the
// result does not depend on which piece ran when), scaled and written as bf16.
// A work unit = ROWS rows of one split tile and kv-head (unit = tile * NCH +
// row chunk, kv-head = blockIdx.y); the workgroups stride over the units of
// the split tiles that exist.  Thread x owns float4 column x % COLS of
// [dK | dV] and rows x / COLS + RSTEP u (u < U) of the chunk, whose loads are
// in flight together.
template <int D>
struct DkvSum {
  static constexpr int C4 = D / 4, COLS = 2 * C4, RSTEP = 256 / COLS, U = 8, ROWS = RSTEP * U, NCH = kBwdBN / ROWS;
  static_assert(kBwdBN % ROWS == 0, "rows split evenly");
};

template <int D, bool CAUSAL>
__global__ __launch_bounds__(256) void attn_bwd_dkv_sum_kernel(const AttnParams p) {
  using S = DkvSum<D>;
  constexpr int BN = kBwdBN;
  // the call's own causality: a plan built for the other one leaves dK / dV alone here too
  if (!plan_matches(p, CAUSAL, true)) return;
  const int units = *p.nsplit * S::NCH;
  for (int unit = blockIdx.x; unit < units; unit += gridDim.x) {
  const int tile = unit / S::NCH, ch = unit % S::NCH;
  const SplitTile st = p.splits[tile];
  const SeqInfo si = p.seq[st.b];
  const int hk = blockIdx.y;
  if ((st.slot0 + st.np) * p.hkv > kSplitSlots) continue;
  const int col = threadIdx.x % S::COLS, which = col / S::C4, c = col - which * S::C4;
  const int k0 = st.t * BN;
  const int rows = min(BN, si.k_len - k0);
  const int r0 = ch * S::ROWS + threadIdx.x / S::COLS;
  const float* base = p.dkv_part + (int64_t)(st.slot0 * p.hkv + hk) * (2 * BN * D) + (int64_t)which * BN * D + 4 * c;
  const int64_t pstride = (int64_t)p.hkv * (2 * BN * D);
  const float sc = which == 0 ? p.scale : 1.f;
  f32x4 acc[S::U];
#pragma unroll
  for (int u = 0; u < S::U; ++u) acc[u] = *reinterpret_cast<const f32x4*>(base + (int64_t)(r0 + S::RSTEP * u) * D);
  for (int pc = 1; pc < st.np; ++pc)
#pragma unroll
    for (int u = 0; u < S::U; ++u)
      acc[u] += *reinterpret_cast<const f32x4*>(base + pc * pstride + (int64_t)(r0 + S::RSTEP * u) * D);
#pragma unroll
  for (int u = 0; u < S::U; ++u) {
    const int r = r0 + S::RSTEP * u;
    if (r >= rows) continue;
    const int64_t row = si.k_start + k0 + r;
    bf16* dst = which == 0 ? p.dk + row * p.dk_tok + (int64_t)hk * p.dk_head + 4 * c
                           : p.dv + row * p.dv_tok + (int64_t)hk * p.dv_head + 4 * c;
    *reinterpret_cast<bf16x4*>(dst) = bf16x4{(bf16)(acc[u][0] * sc), (bf16)(acc[u][1] * sc), (bf16)(acc[u][2] * sc),
                                             (bf16)(acc[u][3] * sc)};
  }
  }
}

template <int D, bool CAUSAL, bool ROPE>
__global__ __launch_bounds__(256, 2) void attn_bwd_dq_kernel(const AttnParams p) {
  constexpr int BM = kFwdBM, BN = kFwdBN, NT = 256, NW = NT / 64;
  static_assert(BM == 128 && BN == 64, "128 q rows (4 x 32) by 64 kv rows (2 x 32) per step");
  using Tile = LdsTile<BN, D, NW>;
  constexpr int TE = Tile::ELEMS, STAGE = 2 * TE;  // K, V
  constexpr int NDT = D / 32;
  __shared__ __align__(16) bf16 smem[2 * STAGE];
  __shared__ __align__(16) float dsh[BM];  // Delta of the tile's rows, handed from the row pass to the MFMA layout

  const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, l32 = lane & 31;
  const int g = wave_uniform(tid >> 6);  // q group: rows 32 g .. 32 g + 31 of the tile
  Tile kt, vt;
  kt.init(p.k_tok, lane);
  vt.init(p.v_tok, lane);
  RowRead<D> rr;
  rr.init(lane);
  TrRead<D> tr;
  tr.init(lane);
  const float c = p.scale_log2;

  // 1-D grid over (q tile, q-head), q-head fastest; each XCD takes whole
  // tiles, one per run, so the heaviest-first tiles go round the XCDs
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

  const int qrow = q0 + 32 * g + l32;
  const bool qvalid = qrow < si.q_len;
  const int lim = CAUSAL ? min(si.k_len - 1, qrow + off) : si.k_len - 1;  // last kv row qrow sees
  const bf16* kbase = p.k + (int64_t)si.k_start * p.k_tok + (int64_t)hk * p.k_head;
  const bf16* vbase = p.v + (int64_t)si.k_start * p.v_tok + (int64_t)hk * p.v_head;
  // loads untracked: the block loop's wait_vmem + barrier order them
  auto issue = [&](int kb, int buf) {
    kt.template issue<true>(kbase + (int64_t)(kb * BN) * p.k_tok, p.k_tok, si.k_len - kb * BN, smem + buf * STAGE, g);
    vt.template issue<true>(vbase + (int64_t)(kb * BN) * p.v_tok, p.v_tok, si.k_len - kb * BN,
                            smem + buf * STAGE + TE, g);
  };
  // Q and dO of the tile go through LDS (the two K / V stages, free until
  // the first block is loaded): the direct loads read whole 256-byte rows,
  // where loading the MFMA operand layout straight into registers touches 32
  // rows per instruction.  O is only needed for Delta = rowsum(dO o O): it
  // is read the same whole-row way into registers and multiplied with the
  // staged dO chunk by chunk.  Each wave stages and reads back its own 32
  // rows, so only its own load wait orders them.
  using QStage = LdsTile<BM, D, NT / 64>;
  static_assert(QStage::ELEMS == STAGE && QStage::PERW * QStage::RPI == 32,
                "a q tile fills one K / V stage, and each wave stages its own 32 rows");
  bf16* Qst = smem;
  bf16* Gst = smem + STAGE;
  {
    QStage qs;
    qs.init(p.q_tok, lane);
    qs.template issue<true>(p.q + (int64_t)(si.q_start + q0) * p.q_tok + (int64_t)hqi * p.q_head, p.q_tok,
                            si.q_len - q0, Qst, g);
    QStage gs;
    gs.init(p.do_tok, lane);
    gs.template issue<true>(p.dout + (int64_t)(si.q_start + q0) * p.do_tok + (int64_t)hqi * p.do_head, p.do_tok,
                            si.q_len - q0, Gst, g);
  }
  RowSpan<D> rs;
  rs.init(lane);
  bf16x8 ov[RowSpan<D>::N32];
  {
    const bf16* obase = p.o + (int64_t)si.q_start * p.o_tok + (int64_t)hqi * p.o_head + 8 * rs.c;
#pragma unroll
    for (int i = 0; i < RowSpan<D>::N32; ++i) {
      const int r = min(q0 + rs.row(32 * g, i), si.q_len - 1);  // rows past the end re-read the last one
      ov[i] = ld_bf16x8(obase + (int64_t)r * p.o_tok);
    }
  }
  const int64_t lidx = (int64_t)hqi * p.lse_head + si.q_start + (qvalid ? qrow : 0);
  const float l2 = p.lse[lidx] * kLog2e;
  wait_vmem();
  asm volatile("" ::: "memory");  // the LDS reads below stay after the wait
  // Delta of each of the wave's rows: the CH lanes of a row sum their chunks
  // (in the order d = 8 c + i, then the lanes' partial sums pairwise), and
  // one of them hands it on through LDS to the lane that owns the row
#pragma unroll
  for (int i = 0; i < RowSpan<D>::N32; ++i) {
    const int r = rs.row(32 * g, i);
    const bf16x8 gv = ld_bf16x8(Gst + rs.lds(r));
    float acc = 0.f;
#pragma unroll
    for (int k = 0; k < 8; ++k) acc = __builtin_fmaf((float)gv[k], (float)ov[i][k], acc);
#pragma unroll
    for (int o = 1; o < RowSpan<D>::CH; o <<= 1) acc += __shfl_xor(acc, o);
    if (rs.c == 0) dsh[r] = acc;
  }
  bf16x8 qf[D / 16], gf[D / 16];
#pragma unroll
  for (int ks = 0; ks < D / 16; ++ks) {
    const bf16x8 a = rr.read(Qst, 32 * g, ks), b = rr.read(Gst, 32 * g, ks);
    qf[ks] = qvalid ? a : zero_bf16x8();
    gf[ks] = qvalid ? b : zero_bf16x8();
  }
  const float lse2 = qvalid ? l2 : INFINITY;
  const float dlt = qvalid ? dsh[32 * g + l32] : 0.f;
  // every wave's staged rows read: the first K / V block may overwrite them
  __syncthreads();
  if (nblk > 0) issue(0, 0);

  f32x16 dq[NDT];
#pragma unroll
  for (int i = 0; i < NDT; ++i) dq[i] = zero16();

  wait_vmem();
  __syncthreads();

  // The next block's K (instructions 0 .. PERW - 1 of this wave) and V (PERW
  // .. 2 PERW - 1) go out one at a time between this block's S / dP MFMAs: K
  // during the first kv half, V during the second.
  constexpr int KPI = (D / 16) / Tile::PERW;
  static_assert(KPI >= 1 && (D / 16) % Tile::PERW == 0, "loads spread evenly over the k-steps");
  const int wq0 = q0 + 32 * g;
  for (int kb = 0; kb < nblk; ++kb) {
    const bf16* Ks = smem + (kb & 1) * STAGE;
    const bf16* Vs = Ks + TE;
    const bool pf = kb + 1 < nblk;
    const int nb = (kb + 1) * BN;  // first kv row of the next block
    bf16* nx = smem + ((kb + 1) & 1) * STAGE;
    auto issue_k = [&](int idx) {
      if (idx < Tile::PERW)
        kt.template issue_one<true>(idx, kbase + (int64_t)nb * p.k_tok, p.k_tok, si.k_len - nb, nx, g);
      else
        vt.template issue_one<true>(idx - Tile::PERW, vbase + (int64_t)nb * p.v_tok, p.v_tok, si.k_len - nb, nx + TE,
                                    g);
    };
    // the step's two 32-row kv halves in turn
#pragma unroll
    for (int kh = 0; kh < 2; ++kh) {
    const int kw = kb * BN + 32 * kh;  // first kv row of this half
    const bool active = wq0 < si.q_len && kw < si.k_len && (!CAUSAL || kw <= wq0 + 31 + off);
    if (!active && pf) {
#pragma unroll
      for (int k = 0; k < Tile::PERW; ++k) issue_k(kh * Tile::PERW + k);
    }
    if (active) {
      // accumulator r holds kv = kw + nrow(r, h) for q = qrow (operands one k-step ahead)
      f32x16 s = zero16(), dp = zero16();
      bf16x8 fk[2], fv[2];
      fk[0] = rr.read(Ks, 32 * kh, 0);
      fv[0] = rr.read(Vs, 32 * kh, 0);
#pragma unroll
      for (int ks = 0; ks < D / 16; ++ks) {
        const int cur = ks & 1;
        if (pf && ks % KPI == 0) issue_k(kh * Tile::PERW + ks / KPI);
        if (ks + 1 < D / 16) {
          fk[cur ^ 1] = rr.read(Ks, 32 * kh, ks + 1);
          fv[cur ^ 1] = rr.read(Vs, 32 * kh, ks + 1);
        }
        s = mfma32(fk[cur], qf[ks], s);
        dp = mfma32(fv[cur], gf[ks], dp);
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        s[r] = __builtin_fmaf(s[r], c, -lse2);
        dp[r] -= dlt;
      }
      if (kw + 31 > si.k_len - 1 || (CAUSAL && kw + 31 > wq0 + off)) {
        // kv rows past the end of the sequence or after the causal limit of some row
        const int rel = lim - kw - 4 * h;  // keep kv offsets <= rel
#pragma unroll
        for (int r = 0; r < 16; ++r) s[r] = (8 * (r >> 2) + (r & 3) > rel) ? -INFINITY : s[r];
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) dp[r] *= exp2f_fast(s[r]);
      bf16x8 db[2];
      db[0] = pack8(dp, 0);
      db[1] = pack8(dp, 8);
      bf16x8 tk[2];
      tk[0] = tr.read(Ks, 32 * kh, 0);
#pragma unroll
      for (int u = 0; u < 2 * NDT; ++u) {
        const int sub = u / NDT, dt = u % NDT, cur = u & 1;
        if (u + 1 < 2 * NDT) tk[cur ^ 1] = tr.read(Ks, 32 * kh + 16 * ((u + 1) / NDT), (u + 1) % NDT);
        dq[dt] = mfma32(tk[cur], db[sub], dq[dt]);
      }
    }
    }
    wait_vmem();
    __syncthreads();
  }

  if (qvalid && h == 0) {
    p.delta[lidx] = dlt;
    p.lse2[lidx] = lse2;
  }
  // dq through LDS, so that it leaves as whole 256-byte rows: after the
  // block loop's last barrier no wave reads K / V, and each wave writes and
  // reads back only its own 32 rows (no barrier).  Lane (l32, h) holds
  // d = 32 dt + 16 j + 8 h + i of its row: logical chunk 4 dt + 2 j + h.  The
  // staged values are bf16(scale * dQ), the attention's own output rounding.
  RowWrite<D> rw;
  rw.init(lane);
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      bf16x8 a;
#pragma unroll
      for (int i = 0; i < 8; ++i) a[i] = (bf16)(dq[dt][8 * j + i] * p.scale);
      rw.write(smem, 32 * g, 4 * dt + 2 * j + h, a);
    }
  }
  bf16* dbase = p.dq + (int64_t)(si.q_start + q0) * p.dq_tok + (int64_t)hqi * p.dq_head + 8 * rs.c;
#pragma unroll
  for (int i = 0; i < RowSpan<D>::N32; ++i) {
    const int r = rs.row(32 * g, i);
    const bf16x8 v = ld_bf16x8(smem + rs.lds(r));
    if (q0 + r >= si.q_len) continue;
    if constexpr (!ROPE) {
      st_bf16x8(dbase + (int64_t)r * p.dq_tok, v);
    } else {
      // dq of the q before rotation, through the rotation's backward (the
      // separate RoPE backward pass's roundings): d pairs with d + D / 2, so
      // chunk c with chunk c ^ CH / 2, read back from the staged row
      constexpr int HC = RowSpan<D>::CH / 2;
      const bool lo = rs.c < HC;
      const int cl = lo ? rs.c : rs.c - HC;
      const bf16x8 w = ld_bf16x8(smem + (uint32_t)(r * D + 8 * ((rs.c ^ HC) ^ swz<D>(r))));
      const int64_t tok = si.q_start + q0 + r;
      const bf16* cp = p.rcos + tok * p.rc_tok + 8 * cl;
      const bf16* sp = p.rsin + tok * p.rs_tok + 8 * cl;
      bf16x8 o1, o2;
      rope_bwd8(lo ? v : w, lo ? w : v, ld_bf16x8(cp), ld_bf16x8(cp + D / 2), ld_bf16x8(sp), ld_bf16x8(sp + D / 2), o1,
                o2);
      st_bf16x8(dbase + (int64_t)r * p.dq_tok, lo ? o1 : o2);
    }
  }
}

// Atomic backward, before the dK/dV kernel: Delta = rowsum(dO o O) and LSE *
// log2(e) of every (row, q-head), which the dQ kernel publishes in the
// deterministic backward, and the fp32 dQ sums cleared.  D / 8 lanes per
// (row, head), lane c summing the 8 elements of chunk c in order and the
// lanes' sums added pairwise (xor 1, 2, 4, ...), as the dQ kernel does, so
// that Delta -- and with it dK and dV -- is bitwise that of the deterministic
// backward.
template <int D>
__global__ __launch_bounds__(256) void attn_bwd_prep_kernel(const AttnParams p) {
  constexpr int LP = D / 8, PPB = 256 / LP;  // lanes per (row, head), pairs per block
  const int c = threadIdx.x % LP;
  const int64_t npairs = p.total_q * p.hq;
  // the lanes of a pair share pi, so they take the same trips and the shuffles below stay within active pairs
  for (int64_t pi = (int64_t)blockIdx.x * PPB + threadIdx.x / LP; pi < npairs; pi += (int64_t)gridDim.x * PPB) {
    const int64_t row = pi / p.hq;
    const int hq = (int)(pi - row * p.hq);
    const bf16x8 o = ld_bf16x8(p.o + row * p.o_tok + (int64_t)hq * p.o_head + 8 * c);
    const bf16x8 g = ld_bf16x8(p.dout + row * p.do_tok + (int64_t)hq * p.do_head + 8 * c);
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc = __builtin_fmaf((float)g[i], (float)o[i], acc);
#pragma unroll
    for (int k = 1; k < LP; k <<= 1) acc += __shfl_xor(acc, k);
    float* z = p.dq_acc + pi * D + 8 * c;
    *reinterpret_cast<f32x4*>(z) = f32x4{0.f, 0.f, 0.f, 0.f};
    *reinterpret_cast<f32x4*>(z + 4) = f32x4{0.f, 0.f, 0.f, 0.f};
    if (c == 0) {
      const int64_t idx = (int64_t)hq * p.lse_head + row;
      p.delta[idx] = acc;
      p.lse2[idx] = p.lse[idx] * kLog2e;
    }
  }
}

// Atomic backward, last: dq = bf16(scale * dQ sums).  Checks the plan like
// the other kernels, so a mismatched call leaves dq alone.
template <int D, bool CAUSAL>
__global__ __launch_bounds__(256) void attn_bwd_dq_convert_kernel(const AttnParams p) {
  constexpr int LP = D / 8, PPB = 256 / LP;
  if (!plan_matches(p, CAUSAL, true)) return;
  const int sub = threadIdx.x % LP;
  const int64_t npairs = p.total_q * p.hq;
  for (int64_t pi = (int64_t)blockIdx.x * PPB + threadIdx.x / LP; pi < npairs; pi += (int64_t)gridDim.x * PPB) {
    const int64_t row = pi / p.hq;
    const int hq = (int)(pi - row * p.hq);
    const float* a = p.dq_acc + pi * D + 8 * sub;
    const f32x4 x0 = *reinterpret_cast<const f32x4*>(a), x1 = *reinterpret_cast<const f32x4*>(a + 4);
    bf16x8 o;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      o[i] = (bf16)(x0[i] * p.scale);
      o[i + 4] = (bf16)(x1[i] * p.scale);
    }
    st_bf16x8(p.dq + row * p.dq_tok + (int64_t)hq * p.dq_head + 8 * sub, o);
  }
}

template <int D, bool CAUSAL>
hipError_t launch_bwd_t(const AttnParams& p, int qcap, int kvcap, hipStream_t stream) {
  const dim3 kvgrid((unsigned)((int64_t)kvcap * p.hkv));
  if (p.dq_acc != nullptr) {
    // atomic: Delta / LSE2 and cleared sums, dK/dV with dQ, partial sums, dq
    const int64_t pairs = p.total_q * p.hq;
    const int64_t ppb = 256 / (D / 8);  // (row, head) pairs per prep block
    const int64_t pblocks = std::min<int64_t>((pairs + ppb - 1) / ppb, 8192);
    const int64_t blocks = std::min<int64_t>((pairs + 256 / (D / 8) - 1) / (256 / (D / 8)), 8192);
    if (pblocks > 0) hipLaunchKernelGGL((attn_bwd_prep_kernel<D>), dim3((unsigned)pblocks), dim3(256), 0, stream, p);
    hipLaunchKernelGGL((attn_bwd_dkdv_kernel<D, CAUSAL, true>), kvgrid, dim3(512), 0, stream, p);
    hipLaunchKernelGGL((attn_bwd_dkv_sum_kernel<D, CAUSAL>), dim3(min(kMaxSplitTiles * DkvSum<D>::NCH, 512), p.hkv), dim3(256),
                       0, stream, p);
    if (blocks > 0)
      hipLaunchKernelGGL((attn_bwd_dq_convert_kernel<D, CAUSAL>), dim3((unsigned)blocks), dim3(256), 0, stream, p);
    return hipGetLastError();
  }
  // dQ first: it also writes Delta and LSE2, which the dK/dV kernel reads
  const dim3 qgrid((unsigned)((int64_t)qcap * p.hq));
  if (p.rcos != nullptr)
    hipLaunchKernelGGL((attn_bwd_dq_kernel<D, CAUSAL, true>), qgrid, dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL((attn_bwd_dq_kernel<D, CAUSAL, false>), qgrid, dim3(256), 0, stream, p);
  // D = 64: one wave per SIMD (K, V, dK, dV and both groups' S / dP fit the
  // registers); D = 128: two waves per SIMD (one wave per SIMD measured 5-10%
  // slower with the accumulators or with K and V in AGPRs)
  if constexpr (D == 64)
    hipLaunchKernelGGL((attn_bwd_dkdv_w4_kernel<D, CAUSAL>), kvgrid, dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL((attn_bwd_dkdv_kernel<D, CAUSAL, false>), kvgrid, dim3(512), 0, stream, p);
  hipLaunchKernelGGL((attn_bwd_dkv_sum_kernel<D, CAUSAL>), dim3(min(kMaxSplitTiles * DkvSum<D>::NCH, 512), p.hkv), dim3(256), 0, stream,
                     p);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_attn_bwd(const AttnParams& p, int d, int causal, int qcap, int kvcap, hipStream_t stream) {
  if (d == 128) return causal ? launch_bwd_t<128, true>(p, qcap, kvcap, stream) : launch_bwd_t<128, false>(p, qcap, kvcap, stream);
  if (d == 64) return causal ? launch_bwd_t<64, true>(p, qcap, kvcap, stream) : launch_bwd_t<64, false>(p, qcap, kvcap, stream);
  return hipErrorInvalidValue;
}

}  // namespace siq
