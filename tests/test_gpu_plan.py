"""GPU checks of attention plans (the per-batch schedule, built once and reused
by every layer, as the reference forwards the same cu_seq_lens kwargs to each
decoder layer, siq_vl/model/modeling.py:278-288):

* a reused plan gives bitwise the outputs of a plan built for the call, and
  of the self-scheduling entry points siq_attn_varlen_fwd / _bwd;
* one plan serves several layers' tensors (forward and backward);
* the plan is cached on the cu_seqlens tensor and rebuilt after an in-place
  change of it;
* the scheduler's overflow tripwires stay clear on the BASELINE workloads;
* a kernel handed a plan built for other heads writes nothing and flags it.
"""

import ctypes

import numpy as np
import pytest
import torch

from siq_vl_amd import _lib
from siq_vl_amd import attention as A
from siq_vl_amd import workloads as W

pytestmark = pytest.mark.gpu

DEV = "cuda"


def make(lengths, hq, hkv, d, seed=0):
    g = torch.Generator().manual_seed(seed)
    t = sum(lengths)
    mk = lambda h: torch.randn(t, h, d, generator=g).to(torch.bfloat16).to(DEV)
    cu = [0]
    for n in lengths:
        cu.append(cu[-1] + n)
    return mk(hq), mk(hkv), mk(hkv), mk(hq), torch.tensor(cu, dtype=torch.int32, device=DEV)


def legacy_fwd_bwd(q, k, v, do, cu, causal):
    """The self-scheduling entry points (schedule built inside each call)."""
    L = _lib.lib()
    total, hq, d = q.shape
    hkv = k.shape[1]
    batch = cu.numel() - 1
    scale = d**-0.5
    out = torch.empty_like(q)
    lse = torch.empty((hq, total), dtype=torch.float32, device=DEV)
    ws = torch.empty(L.siq_attn_fwd_workspace_bytes(batch, total, total, hq, hkv, d), dtype=torch.uint8, device=DEV)
    st = _lib.int64_array([q.stride(0), q.stride(1), k.stride(0), k.stride(1), v.stride(0), v.stride(1),
                           out.stride(0), out.stride(1)])
    s = torch.cuda.current_stream().cuda_stream
    _lib.check(L.siq_attn_varlen_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), lse.data_ptr(),
                                     cu.data_ptr(), cu.data_ptr(), batch, 0, 0, total, total, hq, hkv, d, st, scale,
                                     int(causal), ws.data_ptr(), ws.numel(), s), "fwd")
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    wsb = torch.empty(L.siq_attn_bwd_workspace_bytes(batch, total, total, hq, hkv, d, 1), dtype=torch.uint8,
                      device=DEV)
    st16 = _lib.int64_array([q.stride(0), q.stride(1), k.stride(0), k.stride(1), v.stride(0), v.stride(1),
                             out.stride(0), out.stride(1), do.stride(0), do.stride(1), dq.stride(0), dq.stride(1),
                             dk.stride(0), dk.stride(1), dv.stride(0), dv.stride(1)])
    _lib.check(L.siq_attn_varlen_bwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), lse.data_ptr(),
                                     do.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), cu.data_ptr(),
                                     cu.data_ptr(), batch, 0, 0, total, total, hq, hkv, d, st16, scale, int(causal),
                                     1, wsb.data_ptr(), wsb.numel(), s), "bwd")
    return out, lse, dq, dk, dv


def planned_fwd_bwd(q, k, v, do, cu, causal, plan):
    mx = 0
    scale = q.shape[-1] ** -0.5
    out, lse = A.varlen_attn_fwd(q, k, v, cu, cu, mx, mx, scale, causal, plan=plan)
    dq, dk, dv = A.varlen_attn_bwd(do, q, k, v, out, lse, cu, cu, mx, mx, scale, causal, plan=plan)
    return out, lse, dq, dk, dv


@pytest.mark.parametrize("causal,hq,hkv,d", [(True, 12, 2, 128), (False, 16, 16, 64), (True, 14, 2, 64)])
def test_reused_plan_is_bitwise_a_fresh_schedule(causal, hq, hkv, d):
    lengths = [1, 17, 130, 257, 64, 600, 2, 1000]
    print(f"plan reuse causal={causal} hq={hq} hkv={hkv} d={d}", flush=True)
    plan = A.build_attn_plan(make(lengths, hq, hkv, d)[4], make(lengths, hq, hkv, d)[4], sum(lengths),
                             sum(lengths), hq, hkv, causal)
    for layer in range(3):  # three layers' tensors, one plan
        q, k, v, do, cu = make(lengths, hq, hkv, d, seed=layer)
        got = planned_fwd_bwd(q, k, v, do, cu, causal, plan)
        ref = legacy_fwd_bwd(q, k, v, do, cu, causal)
        for a, b in zip(got, ref):
            assert torch.equal(a, b)
    torch.cuda.synchronize()
    st = plan.status()
    assert st["status_q"] == 0 and st["status_kv"] == 0 and st["status_use"] == 0


def test_plan_cached_on_the_offsets_tensor():
    lengths = [100, 200, 300]
    q, k, v, do, cu = make(lengths, 12, 2, 128)
    p1 = A.cached_attn_plan(cu, cu, 600, 600, 12, 2, True, q.device)
    p2 = A.cached_attn_plan(cu, cu, 600, 600, 12, 2, True, q.device)
    assert p1 is p2
    assert A.cached_attn_plan(cu, cu, 600, 600, 12, 2, False, q.device) is not p1
    out1 = torch.ops.aten.clone(A.flash_attn_varlen_func(q, k, v, cu, cu, 300, 300, causal=True))
    # an in-place change of the offsets: a new plan, and the kernels follow the new sequences
    cu[1] = 150
    p3 = A.cached_attn_plan(cu, cu, 600, 600, 12, 2, True, q.device)
    assert p3 is not p1
    out2 = A.flash_attn_varlen_func(q, k, v, cu, cu, 300, 300, causal=True)
    assert torch.equal(out1[:100], out2[:100])  # the first 100 rows see the same keys
    assert not torch.equal(out1[100:150], out2[100:150])


def test_autograd_op_reuses_one_plan_for_all_layers():
    lengths = [300, 5, 700]
    q, k, v, do, cu = make(lengths, 12, 2, 128)
    xs = [t.clone().requires_grad_(True) for t in (q, k, v)]
    ys = [t.clone().requires_grad_(True) for t in (q, k, v)]
    o1 = A.flash_attn_varlen_func(*xs, cu, cu, 700, 700, causal=True)
    o2 = A.flash_attn_varlen_func(*ys, cu, cu, 700, 700, causal=True)
    plans = list(getattr(cu, "_siq_attn_plans").values())
    assert len(plans) == 1
    (o1 * do).sum().backward()
    (o2 * do).sum().backward()
    assert torch.equal(o1, o2)
    for a, b in zip(xs, ys):
        assert torch.equal(a.grad, b.grad)
    ref = legacy_fwd_bwd(q, k, v, do, cu, True)
    assert torch.equal(o1, ref[0]) and torch.equal(xs[0].grad, ref[2])
    assert torch.equal(xs[1].grad, ref[3]) and torch.equal(xs[2].grad, ref[4])


@pytest.mark.parametrize("idx", [2, 3, 5])
def test_no_overflow_on_baseline_workloads(idx):
    cfg = W.attn_config(idx)
    cu = cfg.cu_seqlens().to(DEV)
    plan = A.build_attn_plan(cu, cu, cfg.total, cfg.total, cfg.hq, cfg.hkv, cfg.causal)
    torch.cuda.synchronize()
    st = plan.status()
    assert st["magic"] == 0x51504C4E
    assert st["status_q"] == 0 and st["status_kv"] == 0


def test_mismatched_plan_writes_nothing_and_flags():
    """A plan built for hkv = 2 handed to a call with hkv = 4 (same sizes, so
    the plan buffer is large enough): the kernels compare the plan's header
    with their arguments, leave the outputs alone and set the mismatch bit."""
    lengths = [64, 200]
    q, k, v, do, cu = make(lengths, 12, 2, 128)
    plan = A.build_attn_plan(cu, cu, 264, 264, 12, 2, True)
    k4 = torch.randn(264, 4, 128, device=DEV).to(torch.bfloat16)
    v4 = torch.randn(264, 4, 128, device=DEV).to(torch.bfloat16)
    out = torch.full_like(q, 7.0)
    lse = torch.full((12, 264), 7.0, device=DEV)
    L = _lib.lib()
    st = _lib.int64_array([q.stride(0), q.stride(1), k4.stride(0), k4.stride(1), v4.stride(0), v4.stride(1),
                           out.stride(0), out.stride(1)])
    rc = L.siq_attn_varlen_fwd_plan(q.data_ptr(), k4.data_ptr(), v4.data_ptr(), out.data_ptr(), lse.data_ptr(), 2,
                                    264, 264, 12, 4, 128, st, 128**-0.5, 1, plan.buf.data_ptr(), plan.buf.numel(),
                                    torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    torch.cuda.synchronize()
    assert bool((out == 7.0).all()) and bool((lse == 7.0).all())
    assert plan.status()["status_use"] == 2
    # the Python op refuses such a plan up front
    with pytest.raises(ValueError, match="plan"):
        A.varlen_attn_fwd(q, k4, v4, cu, cu, 200, 200, 128**-0.5, True, plan=plan)


@pytest.mark.parametrize("deterministic", [True, False])
def test_backward_with_plan_of_other_causality_writes_nothing(deterministic):
    """A causal plan handed to a bidirectional backward through the C ABI, on
    config 2's sequences (heavy kv tiles are split, so the partial-sum kernel
    runs): every backward kernel -- dQ, dK/dV, the split-tile sum, the atomic
    mode's dq conversion -- compares the plan with the call, leaves dq / dk /
    dv at their fill value and flags the mismatch."""
    cfg = W.attn_config(2)
    lengths = cfg.lengths
    print(f"mismatched-causality backward deterministic={deterministic}", flush=True)
    q, k, v, do, cu = make(lengths, 12, 2, 128)
    total = q.shape[0]
    plan = A.build_attn_plan(cu, cu, total, total, 12, 2, True)
    out, lse = A.varlen_attn_fwd(q, k, v, cu, cu, 0, 0, 128**-0.5, True, plan=plan)
    dq, dk, dv = (torch.full_like(t, 3.0) for t in (q, k, v))
    L = _lib.lib()
    det = int(deterministic)
    ws = torch.empty(L.siq_attn_bwd_plan_workspace_bytes(plan.batch, total, total, 12, 2, 128, det),
                     dtype=torch.uint8, device=DEV)
    st = _lib.int64_array([q.stride(0), q.stride(1), k.stride(0), k.stride(1), v.stride(0), v.stride(1),
                           out.stride(0), out.stride(1), do.stride(0), do.stride(1), dq.stride(0), dq.stride(1),
                           dk.stride(0), dk.stride(1), dv.stride(0), dv.stride(1)])
    rc = L.siq_attn_varlen_bwd_plan(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), lse.data_ptr(),
                                    do.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), plan.batch, total,
                                    total, 12, 2, 128, st, 128**-0.5, 0, det, plan.buf.data_ptr(), plan.buf.numel(),
                                    ws.data_ptr(), ws.numel(), torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    torch.cuda.synchronize()
    for t in (dq, dk, dv):
        assert bool((t == 3.0).all())
    assert plan.status()["status_use"] == 2


def test_plan_of_other_offsets_with_equal_totals_is_refused():
    """Two packed batches with the same total and sequence count but other
    lengths: a plan built for one is refused for the other (the host compares
    the offsets), and accepted for tensors that hold its own offsets."""
    a, b = [100, 300, 200], [300, 100, 200]
    q, k, v, do, cu_a = make(a, 12, 2, 128)
    cu_b = make(b, 12, 2, 128)[4]
    plan = A.build_attn_plan(cu_a, cu_a, 600, 600, 12, 2, True)
    with pytest.raises(ValueError, match="cu_seqlens"):
        A.varlen_attn_fwd(q, k, v, cu_b, cu_b, 300, 300, 128**-0.5, True, plan=plan)
    out, lse = A.varlen_attn_fwd(q, k, v, cu_a, cu_a, 300, 300, 128**-0.5, True, plan=plan)
    with pytest.raises(ValueError, match="cu_seqlens"):
        A.varlen_attn_bwd(do, q, k, v, out, lse, cu_b, cu_b, 300, 300, 128**-0.5, True, plan=plan)
    # a copy of the same offsets (another tensor object, also on the CPU) is accepted
    ref = A.varlen_attn_fwd(q, k, v, cu_a.clone(), cu_a.cpu(), 300, 300, 128**-0.5, True, plan=plan)
    assert torch.equal(ref[0], out)
    # an in-place change of the tensor the plan was built from is seen
    cu_a[1] = 300
    cu_a[2] = 400
    with pytest.raises(ValueError, match="cu_seqlens"):
        A.varlen_attn_fwd(q, k, v, cu_a, cu_a, 300, 300, 128**-0.5, True, plan=plan)


def test_position_ids_offsets_computed_once():
    pos = torch.cat([torch.arange(n) for n in (5, 9, 2)]).reshape(1, -1).to(DEV)
    cu1, m1 = A._cu_from_position_ids(pos)
    cu2, m2 = A._cu_from_position_ids(pos)
    assert cu1 is cu2 and m1 == m2 == 9
    assert cu1.tolist() == [0, 5, 14, 16]
