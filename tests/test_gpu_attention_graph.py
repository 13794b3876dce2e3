"""The attention calls captured in a HIP graph, as bench.py times them.

One graph holds a plan build, the forward and the backward over that plan.
It is replayed several times, with the program's own eager work (other
attention calls, allocations, a synchronisation) between the replays, and
every replay must give bitwise the eager calls' outputs: O, LSE, dQ, dK, dV
for the deterministic backward; for the atomic-dQ backward dK and dV bitwise
and dQ within fp32 summation order (rel <= 1e-2).  The library records no
memset node: plans and workspaces are filled by its own kernels.
"""

import pytest
import torch

from siq_vl_amd import attention as A
from tests.test_gpu_attention import make, rel

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _eager(x, cu, mx, scale, causal, det):
    plan = A.build_attn_plan(cu, cu, x["q"].shape[0], x["k"].shape[0], x["q"].shape[1], x["k"].shape[1], causal, DEV)
    out, lse = A.varlen_attn_fwd(x["q"], x["k"], x["v"], cu, cu, mx, mx, scale, causal, plan=plan)
    dq, dk, dv = A.varlen_attn_bwd(x["do"], x["q"], x["k"], x["v"], out, lse, cu, cu, mx, mx, scale, causal,
                                   plan=plan, deterministic=det)
    return out, lse, dq, dk, dv


@pytest.mark.parametrize("d,causal,det", [(128, True, True), (64, False, True), (128, True, False)])
def test_graph_replays_match_the_eager_calls(d, causal, det):
    lengths = [300, 17, 1200, 64, 513, 1]
    hq, hkv = (12, 2) if d == 128 else (16, 16)
    q, k, v, do, cu = make(lengths, hq, hkv, d, seed=41)
    x = {name: t.to(DEV) for name, t in (("q", q), ("k", k), ("v", v), ("do", do))}
    cug = cu.to(DEV)
    mx = max(lengths)
    scale = d**-0.5
    print(f"attention graph d={d} causal={causal} deterministic={det}", flush=True)
    ref = _eager(x, cug, mx, scale, causal, det)
    torch.cuda.synchronize()

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        _eager(x, cug, mx, scale, causal, det)  # warm-up off the default stream before capture
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        got = _eager(x, cug, mx, scale, causal, det)

    other_q, other_k, other_v, other_do, other_cu = make([90, 410], hq, hkv, d, seed=42)
    for i in range(3):
        # eager work of the program between the replays
        y = {n: t.to(DEV) for n, t in (("q", other_q), ("k", other_k), ("v", other_v), ("do", other_do))}
        _eager(y, other_cu.to(DEV), 410, scale, causal, det)
        torch.cuda.synchronize()
        for t in got:
            t.fill_(float("nan"))  # a value the replay must overwrite
        graph.replay()
        torch.cuda.synchronize()
        names = ("out", "lse", "dq", "dk", "dv")
        for name, a, b in zip(names, got, ref):
            if name == "dq" and not det:
                assert rel(a.float().cpu().numpy(), b.float().cpu().numpy()) <= 1e-2, (i, name)
                assert bool(torch.isfinite(a).all()), (i, name)
            else:
                assert torch.equal(a, b), (i, name)
