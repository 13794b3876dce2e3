"""Pins the fp64 linear cross-entropy oracle (CPU, no GPU)."""

import math

import numpy as np
import torch

from oracle import cross_entropy as oc


def make(n, h, v, seed, wscale=0.3):
    rng = np.random.default_rng(seed)
    hid = rng.standard_normal((n, h))
    w = wscale * rng.standard_normal((v, h))
    y = rng.integers(0, v, n)
    return hid, w, y


def test_zero_weight_gives_log_vocab_and_zero_dh():
    hid, w, y = make(6, 5, 11, 0)
    r = oc.linear_ce(hid, np.zeros_like(w), y)
    assert abs(r["loss"] - math.log(11)) < 1e-14
    assert np.max(np.abs(r["dh"])) == 0.0


def test_dominant_label_gives_near_zero_loss():
    hid = np.eye(4)
    w = 50.0 * np.eye(4)
    r = oc.linear_ce(hid, w, np.arange(4))
    assert r["loss"] < 1e-20 + 4 * math.exp(-50)


def test_ignored_rows_count_and_zero_gradient():
    hid, w, y = make(10, 4, 7, 1)
    y[[1, 4, 9]] = -100
    y[5] = 7  # out of range: reported, treated as ignored
    r = oc.linear_ce(hid, w, y)
    assert r["count"] == 6 and r["bad"] == 1
    assert np.all(r["dh"][[1, 4, 5, 9]] == 0.0)


def test_all_ignored_is_nan_mean():
    hid, w, y = make(3, 4, 5, 2)
    y[:] = -100
    r = oc.linear_ce(hid, w, y)
    assert math.isnan(r["loss"]) and r["count"] == 0 and np.all(r["dh"] == 0.0)


def test_matches_torch_cross_entropy_and_autograd():
    hid, w, y = make(20, 8, 13, 3)
    y[::3] = -100
    h_t = torch.tensor(hid, requires_grad=True)
    w_t = torch.tensor(w, requires_grad=True)
    y_t = torch.tensor(y)
    loss = torch.nn.functional.cross_entropy(h_t @ w_t.T, y_t, ignore_index=-100)
    loss.backward()
    r = oc.linear_ce(hid, w, y, block=7)
    assert abs(r["loss"] - loss.item()) < 1e-12
    np.testing.assert_allclose(r["dh"], h_t.grad.numpy(), rtol=1e-10, atol=1e-13)
    np.testing.assert_allclose(r["dw"], w_t.grad.numpy(), rtol=1e-10, atol=1e-13)


def test_sum_over_num_items_matches_torch():
    hid, w, y = make(15, 6, 9, 4)
    y[::4] = -100
    h_t = torch.tensor(hid, requires_grad=True)
    w_t = torch.tensor(w, requires_grad=True)
    loss = torch.nn.functional.cross_entropy(h_t @ w_t.T, torch.tensor(y), ignore_index=-100, reduction="sum") / 37.0
    loss.backward()
    r = oc.linear_ce(hid, w, y, divisor=37.0)
    assert abs(r["loss"] - loss.item()) < 1e-12
    np.testing.assert_allclose(r["dh"], h_t.grad.numpy(), rtol=1e-10, atol=1e-13)
    np.testing.assert_allclose(r["dw"], w_t.grad.numpy(), rtol=1e-10, atol=1e-13)


def test_finite_differences():
    hid, w, y = make(5, 3, 6, 5)
    y[2] = -100
    r = oc.linear_ce(hid, w, y)
    eps = 1e-6
    for arr, grad, idx in ((hid, r["dh"], (0, 1)), (hid, r["dh"], (4, 2)), (w, r["dw"], (3, 0)), (w, r["dw"], (5, 2))):
        p, m = arr.copy(), arr.copy()
        p[idx] += eps
        m[idx] -= eps
        if arr is hid:
            num = (oc.linear_ce(p, w, y)["loss"] - oc.linear_ce(m, w, y)["loss"]) / (2 * eps)
        else:
            num = (oc.linear_ce(hid, p, y)["loss"] - oc.linear_ce(hid, m, y)["loss"]) / (2 * eps)
        assert abs(num - grad[idx]) < 1e-7, (idx, num, grad[idx])


def test_row_blocking_does_not_change_result():
    hid, w, y = make(33, 4, 10, 6)
    a = oc.linear_ce(hid, w, y, block=1)
    b = oc.linear_ce(hid, w, y, block=64)
    assert abs(a["loss"] - b["loss"]) < 1e-13
    np.testing.assert_allclose(a["dw"], b["dw"], rtol=1e-12, atol=1e-14)
