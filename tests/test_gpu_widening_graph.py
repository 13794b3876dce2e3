"""The widening operators captured in HIP graphs, as bench.py times them.

Each raw call (RoPE forward and backward, projector forward and backward, the
splice in both launch paths, the embedding-table gradient) is captured once
and replayed three times, with eager calls of the same operator on other
inputs and a synchronisation between the replays; every replay must give
bitwise the eager call's outputs (all of these operators are deterministic).
Outputs are overwritten with a sentinel before each replay, so a replay that
skipped a write would show.
"""

import pytest
import torch

from siq_vl_amd import projector as PJ
from siq_vl_amd import rope as R
from siq_vl_amd import splice as SP

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _bf16(shape, g, scale=1.0):
    return (scale * torch.randn(shape, generator=g)).to(torch.bfloat16).to(DEV)


def _flat(outs):
    return [t for t in (outs if isinstance(outs, (tuple, list)) else (outs,)) if t is not None]


def _check_replays(fn, other_fn):
    ref = [t.clone() for t in _flat(fn())]
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        got = _flat(fn())
    assert len(got) == len(ref)
    for i in range(3):
        other_fn()
        torch.cuda.synchronize()
        for t in got:
            t.fill_(float("nan") if t.dtype.is_floating_point else -7)
        graph.replay()
        torch.cuda.synchronize()
        for j, (a, b) in enumerate(zip(got, ref)):
            assert torch.equal(a, b), (i, j)


def test_rope_forward_and_backward():
    g = torch.Generator().manual_seed(51)
    b, s, hq, hk, d = 1, 700, 12, 2, 128
    q, k = _bf16((b, s, hq, d), g), _bf16((b, s, hk, d), g)
    gq, gk = _bf16((b, s, hq, d), g), _bf16((b, s, hk, d), g)
    pos = torch.arange(s, dtype=torch.float32)
    inv = 1.0 / (10000.0 ** (torch.arange(0, d, 2, dtype=torch.float32) / d))
    emb = torch.cat([pos[:, None] * inv, pos[:, None] * inv], dim=-1)[None]
    cos, sin = emb.cos().to(torch.bfloat16).to(DEV), emb.sin().to(torch.bfloat16).to(DEV)
    q2, k2 = _bf16((b, s, hq, d), g), _bf16((b, s, hk, d), g)
    print("graph: rope", flush=True)
    _check_replays(lambda: R.rope_fwd(q, k, cos, sin), lambda: R.rope_fwd(q2, k2, cos, sin))
    _check_replays(lambda: R.rope_bwd(gq, gk, cos, sin), lambda: R.rope_bwd(q2, k2, cos, sin))


def test_projector_forward_and_backward():
    g = torch.Generator().manual_seed(52)
    batch, side, dv, r, n = 3, 16, 128, 2, 256
    x = _bf16((batch, side * side, dv), g)
    w = _bf16((n, dv * r * r), g, 0.05)
    dy = _bf16((batch, (side // r) ** 2, n), g)
    x2 = _bf16((batch, side * side, dv), g)
    print("graph: projector", flush=True)
    _check_replays(lambda: PJ.proj_fwd(x, w, r), lambda: PJ.proj_fwd(x2, w, r))
    _check_replays(lambda: PJ.proj_bwd(x, w, dy, r), lambda: PJ.proj_bwd(x2, w, dy, r))


@pytest.mark.parametrize("n", [5000, 40000])
def test_splice_and_table_gradient(n):
    # 5000 tokens: the one-kernel splice; 40000: the scan and the row gather
    g = torch.Generator().manual_seed(53)
    vocab, hidden, img = 4096, 256, 4000
    ids = torch.randint(0, vocab, (n,), generator=g)
    ids[ids == img] = 1
    ids[torch.randperm(n, generator=g)[: n // 4]] = img
    nv = int((ids == img).sum())
    ids = ids.to(DEV)
    weight = _bf16((vocab, hidden), g)
    vis = _bf16((nv, hidden), g)
    ids2 = torch.roll(ids, 1)
    gout = _bf16((n, hidden), g)
    print(f"graph: splice n={n}", flush=True)
    _check_replays(lambda: SP.splice_fwd(ids, weight, vis, img), lambda: SP.splice_fwd(ids2, weight, vis, img))
    _check_replays(lambda: SP.embedding_bwd(gout, ids, vocab, (img,)),
                   lambda: SP.embedding_bwd(gout, ids2, vocab, (img,)))
