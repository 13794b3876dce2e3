"""CPU oracle of the pixel-shuffle projector -- TEST INFRASTRUCTURE ONLY.

Restates SiQ_VLProjector (siq_vl/model/modeling.py:37-106) in numpy:

* ``pixel_shuffle`` follows ``_pixel_shuffle`` (:74-98): the same view /
  reshape / permute(0, 1, 3, 2, 4, 5) / reshape, including its two ValueError
  checks (perfect-square sequence, side divisible by the factor);
* ``projector_fwd`` is ``forward`` (:100-105): the shuffle, then the bias-free
  ``nn.Linear`` (:59), in float64;
* ``projector_bwd`` is its gradient: dX = unshuffle(dY W), dW = dY^T shuffle(X).

Parity pinning (tests/test_oracle_projector.py): the shuffle against an
independent index formula (token (ho, wo), feature (i r + j) dv + c reads patch
(ho r + i, wo r + j)), against torch's F.pixel_unshuffle after its channel
reorder, r = 1 as the identity, the shuffle as a bijection (same multiset of
values), unshuffle as its exact inverse; the backward through the adjoint
identity <P(x), g> = <x, P^T(g)> and torch autograd on the same math in
float64.
"""

from __future__ import annotations

import math

import numpy as np


def pixel_shuffle(x, factor: int) -> np.ndarray:
    """[B, L, D] -> [B, L / r^2, D r^2] (modeling.py:74-98)."""
    x = np.asarray(x)
    bsz, seq, dim = x.shape
    root = math.isqrt(seq)
    if root * root != seq:
        raise ValueError(f"Sequence length {seq} is not a perfect square")
    if root % factor != 0:
        raise ValueError(f"seq_root {root} is not divisible by scale factor {factor}")
    ho = root // factor
    x = x.reshape(bsz, root, root, dim)
    x = x.reshape(bsz, ho, factor, ho, factor, dim)
    x = np.transpose(x, (0, 1, 3, 2, 4, 5))
    return np.ascontiguousarray(x).reshape(bsz, ho * ho, dim * factor * factor)


def pixel_unshuffle(xs, factor: int, seq: int) -> np.ndarray:
    """Inverse of pixel_shuffle: [B, L / r^2, D r^2] -> [B, L, D]."""
    xs = np.asarray(xs)
    bsz, t, kdim = xs.shape
    dim = kdim // (factor * factor)
    root = math.isqrt(seq)
    ho = root // factor
    x = xs.reshape(bsz, ho, ho, factor, factor, dim)
    x = np.transpose(x, (0, 1, 3, 2, 4, 5))
    return np.ascontiguousarray(x).reshape(bsz, seq, dim)


def projector_fwd(x, weight, factor: int) -> np.ndarray:
    """y = pixel_shuffle(x) weight^T, float64."""
    xs = pixel_shuffle(np.asarray(x, dtype=np.float64), factor)
    return xs @ np.asarray(weight, dtype=np.float64).T


def projector_bwd(x, weight, dy, factor: int):
    """(dx, dweight) of projector_fwd for the upstream gradient dy [B, T, N], float64."""
    x = np.asarray(x, dtype=np.float64)
    w = np.asarray(weight, dtype=np.float64)
    dy = np.asarray(dy, dtype=np.float64)
    xs = pixel_shuffle(x, factor)
    dxs = dy @ w
    dx = pixel_unshuffle(dxs, factor, x.shape[1])
    dw = dy.reshape(-1, dy.shape[-1]).T @ xs.reshape(-1, xs.shape[-1])
    return dx, dw
