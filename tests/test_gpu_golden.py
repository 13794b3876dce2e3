"""The HIP kernels against the committed golden fixtures (tests/golden/*.npz,
written by the fp64 oracle).  Tolerance: relative Frobenius error <= 2e-2;
counts and zero rows exact."""

from pathlib import Path

import numpy as np
import pytest
import torch

from siq_vl_amd import attention as A
from siq_vl_amd import cross_entropy as C

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
TOL = 2e-2
DEV = "cuda"


def rel(x, ref) -> float:
    x = np.asarray(x, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.linalg.norm(x - ref) / max(np.linalg.norm(ref), 1e-30))


def bf16(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16).to(DEV)


@pytest.mark.parametrize("name", ["attn_causal_gqa_d128", "attn_bidir_d64"])
def test_attention_golden(name):
    f = np.load(GOLDEN / f"{name}.npz", allow_pickle=False)
    print(f"golden {name}", flush=True)
    q, k, v, do = (bf16(f[n]) for n in ("q", "k", "v", "dout"))
    cu = torch.from_numpy(f["cu_seqlens"]).to(DEV)
    lens = np.diff(f["cu_seqlens"])
    mx = int(lens.max())
    scale, causal = float(f["scale"]), bool(f["causal"])
    out, lse = A.varlen_attn_fwd(q, k, v, cu, cu, mx, mx, scale, causal)
    dq, dk, dv = A.varlen_attn_bwd(do, q, k, v, out, lse, cu, cu, mx, mx, scale, causal)
    torch.cuda.synchronize()
    got = {"o": out, "lse": lse, "dq": dq, "dk": dk, "dv": dv}
    for key, t in got.items():
        r = rel(t.float().cpu().numpy(), f[key])
        assert r <= TOL, (key, r)


def test_cross_entropy_golden():
    f = np.load(GOLDEN / "ce_small.npz", allow_pickle=False)
    print("golden ce_small", flush=True)
    h, w = bf16(f["hidden"]), bf16(f["weight"])
    y = torch.from_numpy(f["labels"]).to(DEV)
    for chunk in (16, 8192):
        loss, count, bad, dh, dw = C.flce_fwd_bwd(h, w, y, -100, None, True, chunk)
        torch.cuda.synchronize()
        assert int(count) == int(f["count"]) and int(bad) == int(f["bad"])
        assert abs(float(loss) - float(f["loss"])) <= TOL * abs(float(f["loss"]))
        dh_np = dh.float().cpu().numpy()
        assert rel(dh_np, f["dh"]) <= TOL
        assert rel(dw.float().cpu().numpy(), f["dw"]) <= TOL
        zero_rows = np.all(f["dh"] == 0, axis=1)
        assert zero_rows.sum() > 0 and np.all(dh_np[zero_rows] == 0.0)
        # the frozen-lm_head call (no dW): the same loss and dH
        loss2, count2, _, dh2, dw2 = C.flce_fwd_bwd(h, w, y, -100, None, False, chunk)
        assert dw2 is None and int(count2) == int(f["count"])
        assert float(loss2) == float(loss) and torch.equal(dh2, dh)
