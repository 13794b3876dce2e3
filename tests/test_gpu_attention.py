"""GPU parity of the varlen attention kernels (through the C ABI).

Small and medium cases compare against the fp64 CPU oracle on the same
bf16 inputs; full BASELINE sizes compare against a per-sequence fp32 torch
reference on the GPU and check size-independent properties (no leakage
across sequences, determinism).  Tolerance (the hot path's contract):
||x - x_ref||_F / ||x_ref||_F <= 2e-2 for O, LSE, dQ, dK, dV.
"""

import numpy as np
import pytest
import torch

from oracle import attention as oa
from siq_vl_amd import attention as A
from siq_vl_amd import workloads as W

pytestmark = pytest.mark.gpu

TOL = 2e-2
DEV = "cuda"


def rel(x, ref) -> float:
    x = np.asarray(x, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.linalg.norm(x - ref) / max(np.linalg.norm(ref), 1e-30))


def make(lengths, hq, hkv, d, seed=0):
    g = torch.Generator().manual_seed(seed)
    t = sum(lengths)
    mk = lambda h: torch.randn(t, h, d, generator=g).to(torch.bfloat16)
    q, k, v, do = mk(hq), mk(hkv), mk(hkv), mk(hq)
    cu = [0]
    for n in lengths:
        cu.append(cu[-1] + n)
    return q, k, v, do, torch.tensor(cu, dtype=torch.int32)


def run_gpu(q, k, v, do, cu, causal, backward=True):
    scale = q.shape[-1] ** -0.5
    qg, kg, vg, dog = (x.to(DEV) for x in (q, k, v, do))
    cug = cu.to(DEV)
    mx = int((cu[1:] - cu[:-1]).max()) if cu.numel() > 1 else 0
    out, lse = A.varlen_attn_fwd(qg, kg, vg, cug, cug, mx, mx, scale, causal)
    res = {"out": out, "lse": lse}
    if backward:
        dq, dk, dv = A.varlen_attn_bwd(dog, qg, kg, vg, out, lse, cug, cug, mx, mx, scale, causal)
        res.update(dq=dq, dk=dk, dv=dv)
    torch.cuda.synchronize()
    return {k_: t.float().cpu().numpy() for k_, t in res.items()}


def check_vs_oracle(lengths, hq, hkv, d, causal, backward=True, seed=0):
    q, k, v, do, cu = make(lengths, hq, hkv, d, seed)
    print(f"case lengths={lengths[:6]}... hq={hq} hkv={hkv} d={d} causal={causal}", flush=True)
    got = run_gpu(q, k, v, do, cu, causal, backward)
    scale = d**-0.5
    o_ref, lse_ref = oa.attention_fwd(q, k, v, cu, cu, scale, causal)
    assert rel(got["out"], o_ref) <= TOL, rel(got["out"], o_ref)
    fin = np.isfinite(lse_ref)
    assert np.array_equal(np.isfinite(got["lse"]), fin)
    assert rel(got["lse"][fin], lse_ref[fin]) <= TOL
    if backward:
        dq, dk, dv = oa.attention_bwd(do, q, k, v, cu, cu, scale, causal)
        for name, ref in (("dq", dq), ("dk", dk), ("dv", dv)):
            r = rel(got[name], ref)
            assert r <= TOL, (name, r)
    return got


@pytest.mark.parametrize("d", [128, 64])
def test_causal_gqa_ragged(d):
    check_vs_oracle([1, 17, 130, 257, 64, 300, 2], 12, 2, d, True)


def test_causal_gqa7_config1_fwd():
    cfg = W.attn_config(1)
    check_vs_oracle(list(cfg.lengths), cfg.hq, cfg.hkv, cfg.d, True, backward=False, seed=42)


def test_bidirectional_mha():
    check_vs_oracle([1024, 1024, 5, 100], 16, 16, 64, False)


def test_bidirectional_d128_gqa():
    check_vs_oracle([200, 33, 129], 8, 4, 128, False)


def test_empty_and_single_token_sequences():
    check_vs_oracle([0, 1, 1, 0, 65, 0, 128, 1], 6, 2, 128, True)


def test_long_sequence_tiles():
    check_vs_oracle([1500, 700], 4, 2, 128, True)


def test_no_cross_sequence_leakage():
    lengths = [300, 200, 513]
    q, k, v, do, cu = make(lengths, 12, 2, 128, seed=3)
    base = run_gpu(q, k, v, do, cu, True)
    k2, v2 = k.clone(), v.clone()
    k2[300:500] = torch.randn(200, 2, 128).to(torch.bfloat16)
    v2[300:500] = torch.randn(200, 2, 128).to(torch.bfloat16)
    pert = run_gpu(q, k2, v2, do, cu, True)
    for s, e in ((0, 300), (500, 1013)):
        for name in ("out", "dq", "dk", "dv"):
            assert np.array_equal(base[name][s:e], pert[name][s:e]), name
        assert np.array_equal(base["lse"][:, s:e], pert["lse"][:, s:e])


def test_backward_is_deterministic():
    q, k, v, do, cu = make([700, 300, 24], 12, 2, 128, seed=5)
    a = run_gpu(q, k, v, do, cu, True)
    b = run_gpu(q, k, v, do, cu, True)
    for name in ("out", "lse", "dq", "dk", "dv"):
        assert np.array_equal(a[name], b[name]), name


def test_strided_views_match_contiguous():
    lengths = [100, 157]
    t = sum(lengths)
    g = torch.Generator().manual_seed(7)
    qkv = torch.randn(t, 12 + 2 + 2, 128, generator=g).to(torch.bfloat16).to(DEV)
    q, k, v = qkv[:, :12], qkv[:, 12:14], qkv[:, 14:]
    cu = torch.tensor([0, 100, t], dtype=torch.int32, device=DEV)
    o1, l1 = A.varlen_attn_fwd(q, k, v, cu, cu, 157, 157, 128**-0.5, True)
    o2, l2 = A.varlen_attn_fwd(q.contiguous(), k.contiguous(), v.contiguous(), cu, cu, 157, 157, 128**-0.5, True)
    assert torch.equal(o1, o2) and torch.equal(l1, l2)


def torch_reference(q, k, v, do, cu, causal):
    """Per-sequence fp32 torch attention on the GPU with autograd (GQA by
    repeating K/V), returning out, lse, dq, dk, dv in fp32."""
    scale = q.shape[-1] ** -0.5
    hq, hkv = q.shape[1], k.shape[1]
    rep = hq // hkv
    qf, kf, vf = (x.float().detach().requires_grad_(True) for x in (q, k, v))
    outs, lses = [], []
    cl = cu.tolist()
    for b in range(len(cl) - 1):
        s, e = cl[b], cl[b + 1]
        if e == s:
            continue
        qb = qf[s:e].transpose(0, 1)
        kb = kf[s:e].transpose(0, 1).repeat_interleave(rep, 0)
        vb = vf[s:e].transpose(0, 1).repeat_interleave(rep, 0)
        sc = torch.matmul(qb, kb.transpose(1, 2).contiguous()) * scale
        if causal:
            n = e - s
            m = torch.ones(n, n, dtype=torch.bool, device=q.device).tril()
            sc = sc.masked_fill(~m, float("-inf"))
        lses.append(torch.logsumexp(sc, -1))
        outs.append(torch.matmul(torch.softmax(sc, -1), vb).transpose(0, 1))
    out = torch.cat(outs, 0)
    lse = torch.cat(lses, 1)
    out.backward(do.float())
    return out.detach(), lse.detach(), qf.grad, kf.grad, vf.grad


@pytest.mark.slow
@pytest.mark.parametrize("idx", [2, 3, 5])
def test_full_size_vs_torch_fp32(idx):
    cfg = W.attn_config(idx)
    print(f"full-size config {idx}: T={cfg.total} hq={cfg.hq} hkv={cfg.hkv} d={cfg.d}", flush=True)
    x = W.attn_inputs(cfg, device=DEV)
    cu = cfg.cu_seqlens().to(DEV)
    scale = cfg.d**-0.5
    out, lse = A.varlen_attn_fwd(x["q"], x["k"], x["v"], cu, cu, cfg.max_seqlen, cfg.max_seqlen, scale, cfg.causal)
    dq, dk, dv = A.varlen_attn_bwd(x["dout"], x["q"], x["k"], x["v"], out, lse, cu, cu, cfg.max_seqlen,
                                   cfg.max_seqlen, scale, cfg.causal)
    ro, rl, rdq, rdk, rdv = torch_reference(x["q"], x["k"], x["v"], x["dout"], cu, cfg.causal)
    for name, a, b in (("out", out, ro), ("lse", lse, rl), ("dq", dq, rdq), ("dk", dk, rdk), ("dv", dv, rdv)):
        r = float((a.float() - b).norm() / b.norm())
        print(f"  {name}: rel {r:.3e}", flush=True)
        assert r <= TOL, (name, r)
