"""Pins the projector oracle (CPU, no GPU)."""

import numpy as np
import pytest
import torch

from oracle import projector as op


def rand(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape)


@pytest.mark.parametrize("side,r,d", [(4, 2, 3), (6, 3, 2), (8, 2, 5), (9, 3, 4)])
def test_shuffle_matches_index_formula(side, r, d):
    # token (ho, wo) of the side/r grid, feature (i r + j) d + c, reads patch (ho r + i, wo r + j)
    b = 2
    x = rand((b, side * side, d), side + r)
    xs = op.pixel_shuffle(x, r)
    wo = side // r
    assert xs.shape == (b, wo * wo, d * r * r)
    for bi in range(b):
        for ho in range(wo):
            for w_ in range(wo):
                for i in range(r):
                    for j in range(r):
                        for c in range(d):
                            assert xs[bi, ho * wo + w_, (i * r + j) * d + c] == x[bi, (ho * r + i) * side + w_ * r + j, c]


@pytest.mark.parametrize("r", [1, 2, 4])
def test_shuffle_vs_torch_pixel_unshuffle(r):
    # F.pixel_unshuffle on [B, C, H, W] gives channel c r^2 + i r + j at (ho, wo); the projector orders (i r + j) C + c
    b, side, d = 2, 8, 6
    x = rand((b, side * side, d), 7)
    t = torch.tensor(x).reshape(b, side, side, d).permute(0, 3, 1, 2)
    u = torch.nn.functional.pixel_unshuffle(t, r)               # [B, d r^2, H/r, W/r]
    u = u.reshape(b, d, r * r, side // r, side // r)            # channel = c r^2 + ij
    u = u.permute(0, 3, 4, 2, 1).reshape(b, (side // r) ** 2, r * r * d)
    assert np.array_equal(op.pixel_shuffle(x, r), u.numpy())


def test_identity_bijection_and_inverse():
    x = rand((3, 36, 4), 1)
    assert np.array_equal(op.pixel_shuffle(x, 1), x)
    xs = op.pixel_shuffle(x, 3)
    assert np.array_equal(np.sort(xs.ravel()), np.sort(x.ravel()))
    assert np.array_equal(op.pixel_unshuffle(xs, 3, 36), x)


def test_reference_errors():
    with pytest.raises(ValueError):
        op.pixel_shuffle(np.zeros((1, 15, 2)), 2)   # not a perfect square
    with pytest.raises(ValueError):
        op.pixel_shuffle(np.zeros((1, 36, 2)), 4)   # side 6 not divisible by 4


def test_backward_adjoint_and_torch_autograd():
    b, side, d, r, n = 2, 6, 4, 3, 5
    x = rand((b, side * side, d), 2)
    w = rand((n, d * r * r), 3)
    g = rand((b, (side // r) ** 2, n), 4)
    y = op.projector_fwd(x, w, r)
    dx, dw = op.projector_bwd(x, w, g, r)
    # the shuffle's transpose is the unshuffle
    gs = rand((b, (side // r) ** 2, d * r * r), 5)
    assert abs(np.sum(op.pixel_shuffle(x, r) * gs) - np.sum(x * op.pixel_unshuffle(gs, r, side * side))) < 1e-12
    # torch autograd of the same math (float64)
    xt = torch.tensor(x, requires_grad=True)
    wt = torch.tensor(w, requires_grad=True)
    xs = xt.reshape(b, side // r, r, side // r, r, d).permute(0, 1, 3, 2, 4, 5).reshape(b, (side // r) ** 2, -1)
    yt = torch.nn.functional.linear(xs, wt)
    yt.backward(torch.tensor(g))
    np.testing.assert_allclose(y, yt.detach().numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(dx, xt.grad.numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(dw, wt.grad.numpy(), rtol=1e-12, atol=1e-12)
