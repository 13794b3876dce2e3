"""Writes the golden fixtures of this directory (run from the repo root:
``python tests/golden/make_golden.py``).

The reference holds no golden vectors for this path (its arithmetic lives in
transformers / torch), so the fixtures are produced by the fp64 oracle
(``oracle/``), itself pinned by closed forms, brute force and library
cross-checks in ``tests/test_oracle_*.py``.  Inputs are stored as the exact
bf16 bit patterns the kernels consume (uint16); expected tensors as float16
(relative rounding 5e-4, far inside the 2e-2 parity bar), LSE and the loss
in float32 / float64.

Fixtures:
* ``attn_causal_gqa_d128.npz`` -- causal GQA (2 q / 1 kv heads, d 128), ragged
  lengths incl. a 1-token sequence and a tile-straddling one: O, LSE, dQ/dK/dV.
* ``attn_bidir_d64.npz`` -- bidirectional MHA (2 / 2 heads, d 64): same outputs.
* ``ce_small.npz`` -- linear CE (n 72, hdim 128, vocab 520 = 2 x 256 + 8), ignored rows and
  one out-of-range label: loss, count, bad, dH, dW (mean reduction).
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle import attention as oa  # noqa: E402
from oracle import cross_entropy as oc  # noqa: E402

ATTN_CASES = {
    "attn_causal_gqa_d128": dict(lengths=[1, 37, 130, 9], hq=2, hkv=1, d=128, causal=True, seed=7),
    "attn_bidir_d64": dict(lengths=[64, 3, 70], hq=2, hkv=2, d=64, causal=False, seed=8),
}
CE_CASE = dict(n=72, hdim=128, vocab=520, seed=9)


def bf16_bits(x: torch.Tensor) -> np.ndarray:
    return x.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def bits_to_f64(bits: np.ndarray) -> np.ndarray:
    return torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).to(torch.float64).numpy()


def attn_case(lengths, hq, hkv, d, causal, seed):
    g = torch.Generator().manual_seed(seed)
    t = sum(lengths)
    q, do = (torch.randn(t, hq, d, generator=g) for _ in range(2))
    k, v = (torch.randn(t, hkv, d, generator=g) for _ in range(2))
    bits = {n: bf16_bits(x) for n, x in (("q", q), ("k", k), ("v", v), ("dout", do))}
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    f = {n: bits_to_f64(b) for n, b in bits.items()}
    scale = d ** -0.5
    o, lse = oa.attention_fwd(f["q"], f["k"], f["v"], cu, cu, scale, causal)
    dq, dk, dv = oa.attention_bwd(f["dout"], f["q"], f["k"], f["v"], cu, cu, scale, causal)
    out = dict(bits, cu_seqlens=cu, scale=np.float64(scale), causal=np.bool_(causal))
    out["lse"] = lse.astype(np.float32)
    for n, x in (("o", o), ("dq", dq), ("dk", dk), ("dv", dv)):
        out[n] = x.astype(np.float16)
    return out


def ce_case(n, hdim, vocab, seed):
    g = torch.Generator().manual_seed(seed)
    h = torch.randn(n, hdim, generator=g)
    w = 0.05 * torch.randn(vocab, hdim, generator=g)
    y = torch.randint(0, vocab, (n,), generator=g)
    y[::5] = -100
    y[3] = vocab + 4  # out of range: counted as bad, treated as ignored
    hb, wb = bf16_bits(h), bf16_bits(w)
    r = oc.linear_ce(bits_to_f64(hb), bits_to_f64(wb), y.numpy())
    return dict(hidden=hb, weight=wb, labels=y.numpy().astype(np.int64), loss=np.float64(r["loss"]),
                count=np.int64(r["count"]), bad=np.int64(r["bad"]), lse=r["lse"].astype(np.float32),
                dh=r["dh"].astype(np.float16), dw=r["dw"].astype(np.float16))


def build_all() -> dict[str, dict[str, np.ndarray]]:
    out = {name: attn_case(**kw) for name, kw in ATTN_CASES.items()}
    out["ce_small"] = ce_case(**CE_CASE)
    return out


def main() -> None:
    for name, arrays in build_all().items():
        np.savez_compressed(HERE / f"{name}.npz", **arrays)
        print("wrote", name)


if __name__ == "__main__":
    main()
