"""fp64 varlen attention oracle (test infrastructure only; see package header).

Restates the reference path's attention definition for a packed batch:

* scores, mask, fp32 softmax, product with V:
  transformers models/qwen2/modeling_qwen2.py:150-172 (eager_attention_forward),
  models/siglip/modeling_siglip.py:227-247 (same, bidirectional);
* GQA: q-head h reads kv-head h // (Hq // Hkv) -- repeat_kv,
  models/qwen2/modeling_qwen2.py:138-147;
* packing: sequences never see each other (block-diagonal mask built from
  packed position_ids, masking_utils.py:728-757; the varlen contract
  modeling_flash_attention_utils.py:796-822 with cu_seqlens);
* causal alignment: bottom-right, q row i of a sequence sees k rows
  j <= i + (Lk - Lq) (flash-attention varlen); the usual j <= i when Lq == Lk.

Backward: the exact gradient of that function in fp64 (dV = P^T dO,
dP = dO V^T, dS = P o (dP - rowsum(P o dP)), dQ = s dS K, dK = s dS^T Q,
summed over the q-heads of a GQA group).

Pinning (tests/test_oracle_attention.py): closed forms (q = 0 gives the mean of
the visible values and lse = log(#visible); a single-token sequence gives
o = v; all-equal keys give the mean of V), invariants (perturbing another
sequence leaves a sequence bit-identical; permuting sequences permutes the
output; GQA heads with equal q give equal o; shifting K by a constant leaves O
unchanged), a library cross-check against torch scaled_dot_product_attention
with an explicit block-diagonal mask, central finite differences of the
backward, and the identity that each row of dS sums to zero; the stored-output
form of the backward's row term matches the exact one when given the exact
output.
"""

from __future__ import annotations

import numpy as np


def _f64(x) -> np.ndarray:
    if hasattr(x, "detach"):
        x = x.detach().to("cpu")
        if str(x.dtype) == "torch.bfloat16":
            x = x.float()
        x = x.numpy()
    return np.asarray(x, dtype=np.float64)


def _cu(cu) -> list[int]:
    if hasattr(cu, "tolist"):
        return [int(c) for c in cu.tolist()]
    return [int(c) for c in cu]


def _visible(lq: int, lk: int, causal: bool) -> np.ndarray:
    """[lq, lk] boolean: key j visible to query i."""
    if not causal:
        return np.ones((lq, lk), dtype=bool)
    off = lk - lq
    i = np.arange(lq)[:, None]
    j = np.arange(lk)[None, :]
    return j <= i + off


def _probs(qb: np.ndarray, kb: np.ndarray, scale: float, vis: np.ndarray):
    """qb [n, lq, d], kb [lk, d] -> (P [n, lq, lk], lse [n, lq]) with masked
    entries 0 and lse = -inf for rows that see no key."""
    s = scale * np.einsum("nqd,kd->nqk", qb, kb)
    s = np.where(vis[None], s, -np.inf)
    m = s.max(axis=-1, keepdims=True)
    m_safe = np.where(np.isfinite(m), m, 0.0)
    e = np.where(vis[None], np.exp(s - m_safe), 0.0)
    l = e.sum(axis=-1, keepdims=True)
    p = np.divide(e, l, out=np.zeros_like(e), where=l > 0)
    with np.errstate(divide="ignore"):
        lse = np.where(l[..., 0] > 0, m_safe[..., 0] + np.log(np.where(l[..., 0] > 0, l[..., 0], 1.0)), -np.inf)
    return p, lse


def attention_fwd(q, k, v, cu_q, cu_k, scale: float, causal: bool, q_block: int = 512):
    """q [Tq, Hq, D], k/v [Tk, Hkv, D] -> (out [Tq, Hq, D] fp64, lse [Hq, Tq] fp64)."""
    q, k, v = _f64(q), _f64(k), _f64(v)
    cq, ck = _cu(cu_q), _cu(cu_k)
    tq, hq, d = q.shape
    hkv = k.shape[1]
    rep = hq // hkv
    out = np.zeros((tq, hq, d))
    lse = np.full((hq, tq), -np.inf)
    for b in range(len(cq) - 1):
        qs, qe, ks, ke = cq[b], cq[b + 1], ck[b], ck[b + 1]
        lq, lk = qe - qs, ke - ks
        if lq <= 0:
            continue
        vis_all = _visible(lq, lk, causal)
        for hk in range(hkv):
            heads = slice(hk * rep, (hk + 1) * rep)
            kb, vb = k[ks:ke, hk], v[ks:ke, hk]
            for r0 in range(0, lq, q_block):
                r1 = min(lq, r0 + q_block)
                qb = np.transpose(q[qs + r0:qs + r1, heads], (1, 0, 2))
                p, l = _probs(qb, kb, scale, vis_all[r0:r1])
                out[qs + r0:qs + r1, heads] = np.transpose(p @ vb, (1, 0, 2))
                lse[heads, qs + r0:qs + r1] = l
    return out, lse


def attention_bwd(dout, q, k, v, cu_q, cu_k, scale: float, causal: bool, q_block: int = 512, out=None):
    """Exact fp64 gradients (dq, dk, dv) of attention_fwd's output w.r.t. q, k, v.

    With ``out`` ([Tq, Hq, D], the forward output as stored, e.g. rounded to
    bf16) the row term rowsum(P o dP) is taken as rowsum(dO o out) instead --
    FlashAttention-2's D_i = rowsum(dO_i o O_i) (Dao 2023, Algorithm 2), which
    fused attention backwards compute from the stored output.  The two agree
    exactly when ``out`` is the exact output; they part where P is close to
    one-hot and K is large, since the rounding of ``out`` then dominates
    dP - D."""
    dout, q, k, v = _f64(dout), _f64(q), _f64(k), _f64(v)
    o_st = None if out is None else _f64(out)
    cq, ck = _cu(cu_q), _cu(cu_k)
    tq, hq, d = q.shape
    hkv = k.shape[1]
    rep = hq // hkv
    dq = np.zeros_like(q)
    dk = np.zeros_like(k)
    dv = np.zeros_like(v)
    for b in range(len(cq) - 1):
        qs, qe, ks, ke = cq[b], cq[b + 1], ck[b], ck[b + 1]
        lq, lk = qe - qs, ke - ks
        if lq <= 0 or lk <= 0:
            continue
        vis_all = _visible(lq, lk, causal)
        for hk in range(hkv):
            heads = slice(hk * rep, (hk + 1) * rep)
            kb, vb = k[ks:ke, hk], v[ks:ke, hk]
            for r0 in range(0, lq, q_block):
                r1 = min(lq, r0 + q_block)
                qb = np.transpose(q[qs + r0:qs + r1, heads], (1, 0, 2))      # [rep, n, d]
                gb = np.transpose(dout[qs + r0:qs + r1, heads], (1, 0, 2))   # [rep, n, d]
                p, _ = _probs(qb, kb, scale, vis_all[r0:r1])                 # [rep, n, lk]
                dv[ks:ke, hk] += np.einsum("rnk,rnd->kd", p, gb)
                dp = np.einsum("rnd,kd->rnk", gb, vb)
                if o_st is None:
                    delta = (p * dp).sum(axis=-1, keepdims=True)
                else:
                    ob = np.transpose(o_st[qs + r0:qs + r1, heads], (1, 0, 2))
                    delta = (gb * ob).sum(axis=-1, keepdims=True)
                ds = p * (dp - delta)
                dq[qs + r0:qs + r1, heads] = np.transpose(scale * (ds @ kb), (1, 0, 2))
                dk[ks:ke, hk] += scale * np.einsum("rnk,rnd->kd", ds, qb)
    return dq, dk, dv


def attention_bwd_ds_rowsums(dout, q, k, v, cu_q, cu_k, scale: float, causal: bool) -> np.ndarray:
    """Row sums of dS = P o (dP - rowsum(P o dP)) for every (head, q row): the
    identity sum_j dS_ij = 0 that the backward must respect."""
    dout, q, k, v = _f64(dout), _f64(q), _f64(k), _f64(v)
    cq, ck = _cu(cu_q), _cu(cu_k)
    hq = q.shape[1]
    rep = hq // k.shape[1]
    sums = []
    for b in range(len(cq) - 1):
        qs, qe, ks, ke = cq[b], cq[b + 1], ck[b], ck[b + 1]
        if qe <= qs or ke <= ks:
            continue
        vis = _visible(qe - qs, ke - ks, causal)
        for hk in range(k.shape[1]):
            heads = slice(hk * rep, (hk + 1) * rep)
            qb = np.transpose(q[qs:qe, heads], (1, 0, 2))
            gb = np.transpose(dout[qs:qe, heads], (1, 0, 2))
            p, _ = _probs(qb, k[ks:ke, hk], scale, vis)
            dp = np.einsum("rnd,kd->rnk", gb, v[ks:ke, hk])
            ds = p * (dp - (p * dp).sum(axis=-1, keepdims=True))
            sums.append(ds.sum(axis=-1).ravel())
    return np.concatenate(sums) if sums else np.zeros(0)
