"""Pins the RoPE oracle (CPU, no GPU).

Against torch's own bf16 ops and autograd -- the library the reference's
apply_rotary_pos_emb runs on -- bit for bit, and against closed forms that a
dropped term, a wrong sign or a swapped half would break.
"""

import numpy as np
import pytest
import torch

from oracle import rope as orope


def rotate_half_t(x):
    x1 = x[..., : x.shape[-1] // 2]
    x2 = x[..., x.shape[-1] // 2:]
    return torch.cat((-x2, x1), dim=-1)


def torch_rope(q, k, cos, sin, unsqueeze_dim=1):
    """transformers models/qwen2/modeling_qwen2.py:105-135, as torch runs it."""
    cos = cos.unsqueeze(unsqueeze_dim)
    sin = sin.unsqueeze(unsqueeze_dim)
    return (q * cos) + (rotate_half_t(q) * sin), (k * cos) + (rotate_half_t(k) * sin)


def make(b, s, hq, hkv, d, seed=0, positions=None):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, hq, s, d, generator=g).to(torch.bfloat16)
    k = torch.randn(b, hkv, s, d, generator=g).to(torch.bfloat16)
    pos = positions if positions is not None else torch.arange(s).repeat(b, 1)
    cos, sin = orope.qwen2_cos_sin(pos.numpy(), d)
    return q, k, torch.tensor(cos).to(torch.bfloat16), torch.tensor(sin).to(torch.bfloat16)


def f32(t):
    return t.float().numpy()


def test_round_bf16_matches_torch():
    x = np.random.default_rng(0).standard_normal(10000).astype(np.float32) * 37.0
    x = np.concatenate([x, np.float32([0.0, -0.0, 1.0 + 2**-8, 1.0 + 3 * 2**-8, 3.4e38])])
    ref = torch.tensor(x).to(torch.bfloat16).float().numpy()
    assert np.array_equal(orope.round_bf16(x).view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("d", [64, 128])
def test_forward_bitwise_vs_torch_bf16(d):
    q, k, cos, sin = make(2, 37, 4, 2, d)
    qe, ke = torch_rope(q, k, cos, sin)
    cq = f32(cos)[:, None]
    sq = f32(sin)[:, None]
    assert np.array_equal(orope.rope_fwd(f32(q), cq, sq), f32(qe))
    assert np.array_equal(orope.rope_fwd(f32(k), cq, sq), f32(ke))


@pytest.mark.parametrize("d", [64, 128])
def test_backward_bitwise_vs_torch_autograd(d):
    q, k, cos, sin = make(2, 29, 3, 1, d, seed=1)
    q.requires_grad_(True)
    k.requires_grad_(True)
    qe, ke = torch_rope(q, k, cos, sin)
    g = torch.Generator().manual_seed(5)
    gq = torch.randn(qe.shape, generator=g).to(torch.bfloat16)
    gk = torch.randn(ke.shape, generator=g).to(torch.bfloat16)
    torch.autograd.backward((qe, ke), (gq, gk))
    cq = f32(cos)[:, None]
    sq = f32(sin)[:, None]
    assert np.array_equal(orope.rope_bwd(f32(gq), cq, sq), f32(q.grad))
    assert np.array_equal(orope.rope_bwd(f32(gk), cq, sq), f32(k.grad))


def test_packed_positions_restart_per_sequence():
    # packed batch: position ids restart at each sequence start (the collator's contract)
    pos = torch.tensor([[0, 1, 2, 3, 0, 1, 0, 1, 2]])
    q, k, cos, sin = make(1, 9, 2, 1, 64, positions=pos)
    c = f32(cos)[0]
    assert np.array_equal(c[4], c[0]) and np.array_equal(c[6], c[0]) and np.array_equal(c[8], c[2])
    # position 0: cos = 1, sin = 0 -> the identity, bit for bit
    out = orope.rope_fwd(f32(q)[0, :, 4], c[4], f32(sin)[0, 4])
    assert np.array_equal(out, f32(q)[0, :, 4])


def test_identity_and_pure_rotation():
    rng = np.random.default_rng(2)
    x = orope.round_bf16(rng.standard_normal((5, 3, 64)))
    one, zero = np.ones(64, np.float32), np.zeros(64, np.float32)
    assert np.array_equal(orope.rope_fwd(x, one, zero), x)
    assert np.array_equal(orope.rope_fwd(x, zero, one), orope.rotate_half(x))
    assert np.array_equal(orope.rope_bwd(x, one, zero), x)
    # rotate_half twice is -identity, so the backward of the pure rotation is its inverse
    assert np.array_equal(orope.rope_bwd(orope.rope_fwd(x, zero, one), zero, one), x)


def test_rotation_preserves_pair_norms_and_adjoint():
    rng = np.random.default_rng(3)
    d = 128
    theta = rng.uniform(0, 2 * np.pi, d // 2)
    cos = np.concatenate([np.cos(theta), np.cos(theta)])
    sin = np.concatenate([np.sin(theta), np.sin(theta)])
    x = rng.standard_normal((7, d))
    y = orope.rope_fwd_f64(x, cos, sin)
    pair = lambda v: v[:, : d // 2] ** 2 + v[:, d // 2:] ** 2
    np.testing.assert_allclose(pair(y), pair(x), rtol=1e-12)
    g = rng.standard_normal((7, d))
    assert abs(np.sum(y * g) - np.sum(x * orope.rope_bwd_f64(g, cos, sin))) < 1e-10


def test_bf16_oracle_tracks_f64_map():
    q, k, cos, sin = make(1, 64, 2, 1, 128, seed=4)
    x = f32(q)
    c = f32(cos)[:, None]
    s = f32(sin)[:, None]
    ref = orope.rope_fwd_f64(x, c, s)
    err = np.abs(orope.rope_fwd(x, c, s) - ref)
    assert np.all(err <= 2 ** -7 * (np.abs(x) + np.abs(orope.rotate_half(x))) + 1e-30)
