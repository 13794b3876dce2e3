"""fp64 linear cross-entropy oracle (test infrastructure only; see package header).

Restates the reference's loss: logits = h W^T (transformers
models/qwen2/modeling_qwen2.py:465), ``logits.float()`` and
``F.cross_entropy(logits, shift_labels, ignore_index=-100)`` with
``reduction="mean"``, or ``"sum"`` divided by ``num_items_in_batch``
(transformers loss/loss_utils.py:32-71).  Labels outside [0, V) other than
ignore_index are an error in torch; here they are reported and treated as
ignored (mirroring the kernel's contract).

Closed form per row n with valid label y:
  lse_n = max_v z_nv + log sum_v exp(z_nv - max),  loss_n = lse_n - z_ny,
  dZ_n = (softmax(z_n) - onehot(y)) / den,  dH = dZ W,  dW = dZ^T H,
with den = #valid rows (mean) or the given divisor.  Ignored rows contribute
exactly zero.

Pinning (tests/test_oracle_ce.py): W = 0 gives loss = ln V exactly and dH = 0;
a dominant label logit gives loss ~ 0; all rows ignored gives NaN (mean) like
F.cross_entropy; ignored rows give dH rows of exactly 0; torch
F.cross_entropy + autograd in fp64 as a library cross-check; central finite
differences of loss w.r.t. h and W.
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


def _labels(y) -> np.ndarray:
    if hasattr(y, "detach"):
        y = y.detach().to("cpu").numpy()
    return np.asarray(y, dtype=np.int64)


def linear_ce(hidden, weight, labels, ignore_index: int = -100, divisor: float | None = None,
              need_dweight: bool = True, block: int = 256):
    """Returns dict(loss, count, bad, lse, dh, dw) in fp64 (dw None if not needed)."""
    h = _f64(hidden)
    w = _f64(weight)
    y = _labels(labels)
    n, _ = h.shape
    vocab = w.shape[0]
    in_range = (y >= 0) & (y < vocab)
    not_ignored = y != ignore_index
    valid = not_ignored & in_range
    count = int(valid.sum())
    bad = int((not_ignored & ~in_range).sum())
    den = float(count) if divisor is None else float(divisor)
    lse_all = np.zeros(n)
    loss_sum = 0.0
    dh = np.zeros_like(h)
    dw = np.zeros_like(w) if need_dweight else None
    for r0 in range(0, n, block):
        r1 = min(n, r0 + block)
        z = h[r0:r1] @ w.T
        m = z.max(axis=1, keepdims=True)
        lse = (m + np.log(np.exp(z - m).sum(axis=1, keepdims=True)))[:, 0]
        lse_all[r0:r1] = lse
        vb = valid[r0:r1]
        rows = np.nonzero(vb)[0]
        zy = z[rows, y[r0:r1][rows]]
        loss_sum += float((lse[rows] - zy).sum())
        p = np.exp(z - lse[:, None])
        p[rows, y[r0:r1][rows]] -= 1.0
        p[~vb] = 0.0
        if rows.size:
            with np.errstate(divide="ignore", invalid="ignore"):
                p[rows] = p[rows] / den
        dh[r0:r1] = p @ w
        if dw is not None:
            dw += p.T @ h[r0:r1]
    with np.errstate(divide="ignore", invalid="ignore"):
        loss = np.float64(loss_sum) / np.float64(den)
    return {"loss": float(loss), "count": count, "bad": bad, "lse": lse_all, "dh": dh, "dw": dw}
