"""Pins the splice oracle (CPU, no GPU)."""

import numpy as np
import pytest
import torch

from oracle import splice as osp

IMG = 7


def test_known_answer():
    ids = np.array([[1, IMG, IMG, 2], [IMG, 3, 0, IMG]])
    w = np.arange(10 * 2, dtype=np.float64).reshape(10, 2)
    vis = np.array([[100.0, 101.0], [102.0, 103.0], [104.0, 105.0], [106.0, 107.0]])
    out = osp.splice_fwd(ids, w, vis, IMG)
    expect = np.array([[[2, 3], [100, 101], [102, 103], [4, 5]], [[104, 105], [6, 7], [0, 1], [106, 107]]])
    assert np.array_equal(out, expect)
    g = np.ones((2, 4, 2))
    dw, dv = osp.splice_bwd(g, ids, IMG, 10)
    assert np.array_equal(dv, np.ones((4, 2)))
    assert dw[IMG].sum() == 0 and dw[1].tolist() == [1, 1] and dw[0].tolist() == [1, 1] and dw.sum() == 8


def test_count_check():
    with pytest.raises(ValueError, match="Shape Mismatch"):
        osp.splice_fwd(np.array([[IMG, 1]]), np.zeros((10, 2)), np.zeros((2, 2)), IMG)


@pytest.mark.parametrize("padding_idx", [None, 3])
def test_vs_torch_ops_and_autograd(padding_idx):
    # modeling.py:252-270 as torch runs it: embedding, nonzero, index assignment
    rng = np.random.default_rng(0)
    ids = rng.integers(0, 12, (3, 17))
    ids[0, 2:6] = IMG
    ids[2, 10:15] = IMG
    npos = int((ids == IMG).sum())
    w = rng.standard_normal((12, 5))
    vis = rng.standard_normal((npos, 5))
    g = rng.standard_normal((3, 17, 5))
    emb = torch.nn.Embedding(12, 5, padding_idx=padding_idx).double()
    with torch.no_grad():
        emb.weight.copy_(torch.tensor(w))
    vt = torch.tensor(vis, requires_grad=True)
    it = torch.tensor(ids)
    te = emb(it)
    positions = (it == IMG).nonzero(as_tuple=True)
    te[positions] = vt
    te.backward(torch.tensor(g))
    assert np.allclose(osp.splice_fwd(ids, w, vis, IMG), te.detach().numpy(), rtol=0, atol=0)
    dw, dv = osp.splice_bwd(g, ids, IMG, 12, padding_idx)
    np.testing.assert_allclose(dw, emb.weight.grad.numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(dv, vt.grad.numpy(), rtol=0, atol=0)


def test_gradient_conservation():
    rng = np.random.default_rng(1)
    ids = rng.integers(0, 9, (4, 11))
    ids[1, :3] = IMG
    g = rng.standard_normal((4, 11, 3))
    dw, dv = osp.splice_bwd(g, ids, IMG, 9)
    text = ids.reshape(-1) != IMG
    np.testing.assert_allclose(dw.sum(0), g.reshape(-1, 3)[text].sum(0), rtol=1e-12)
    np.testing.assert_allclose(dv.sum(0), g.reshape(-1, 3)[~text].sum(0), rtol=1e-12)
