"""Pins the fp64 varlen attention oracle (CPU, no GPU).

The reference ships no golden vectors for this path, so each property below
is chosen so that a plausible oracle mistake (wrong scale, missing mask,
cross-sequence leakage, wrong GQA head mapping, transposed operand, dropped
Delta term in the backward) fails at least one of them.
"""

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import cpu_path


def rand(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape)


def cu_of(lengths):
    cu = [0]
    for n in lengths:
        cu.append(cu[-1] + n)
    return cu


@pytest.mark.parametrize("causal", [True, False])
def test_zero_query_gives_mean_of_visible_values(causal):
    lengths = [5, 1, 9]
    cu = cu_of(lengths)
    t = cu[-1]
    q = np.zeros((t, 4, 8))
    k, v = rand((t, 2, 8), 1), rand((t, 2, 8), 2)
    out, lse = oa.attention_fwd(q, k, v, cu, cu, 0.3, causal)
    for b, n in enumerate(lengths):
        s = cu[b]
        for i in range(n):
            hi = i + 1 if causal else n
            for h in range(4):
                np.testing.assert_allclose(out[s + i, h], v[s:s + hi, h // 2].mean(0), rtol=1e-12, atol=1e-12)
                np.testing.assert_allclose(lse[h, s + i], np.log(hi), rtol=1e-12)


def test_single_token_sequences_return_their_value():
    cu = cu_of([1, 1, 1])
    q, k, v = rand((3, 2, 4), 3), rand((3, 1, 4), 4), rand((3, 1, 4), 5)
    out, lse = oa.attention_fwd(q, k, v, cu, cu, 0.5, True)
    for t in range(3):
        for h in range(2):
            np.testing.assert_allclose(out[t, h], v[t, 0], rtol=1e-12)
            np.testing.assert_allclose(lse[h, t], 0.5 * q[t, h] @ k[t, 0], rtol=1e-12)


def test_equal_keys_give_mean_value():
    lengths = [6]
    cu = cu_of(lengths)
    q, v = rand((6, 2, 4), 6), rand((6, 2, 4), 7)
    k = np.tile(rand((1, 2, 4), 8), (6, 1, 1))
    out, _ = oa.attention_fwd(q, k, v, cu, cu, 1.0, False)
    np.testing.assert_allclose(out, np.broadcast_to(v.mean(0, keepdims=True), out.shape), rtol=1e-12, atol=1e-12)


def test_no_leakage_and_permutation():
    lengths = [4, 7, 3]
    cu = cu_of(lengths)
    t = cu[-1]
    q, k, v = rand((t, 3, 8), 9), rand((t, 3, 8), 10), rand((t, 3, 8), 11)
    base, _ = oa.attention_fwd(q, k, v, cu, cu, 0.35, True)
    k2, v2 = k.copy(), v.copy()
    k2[4:11] += 5.0
    v2[4:11] *= -3.0
    pert, _ = oa.attention_fwd(q, k2, v2, cu, cu, 0.35, True)
    assert np.array_equal(base[:4], pert[:4]) and np.array_equal(base[11:], pert[11:])
    # reversing the sequence order permutes the output rows the same way
    order = [2, 1, 0]
    idx = np.concatenate([np.arange(cu[b], cu[b + 1]) for b in order])
    cu_r = cu_of([lengths[b] for b in order])
    outr, _ = oa.attention_fwd(q[idx], k[idx], v[idx], cu_r, cu_r, 0.35, True)
    np.testing.assert_allclose(outr, base[idx], rtol=1e-13, atol=1e-13)


def test_gqa_head_mapping():
    cu = cu_of([5])
    q = np.repeat(rand((5, 1, 8), 12), 6, axis=1)  # 6 identical q heads
    k, v = rand((5, 2, 8), 13), rand((5, 2, 8), 14)
    out, _ = oa.attention_fwd(q, k, v, cu, cu, 0.4, True)
    # heads 0-2 share kv head 0, heads 3-5 kv head 1
    np.testing.assert_allclose(out[:, 0], out[:, 2], rtol=1e-13)
    np.testing.assert_allclose(out[:, 3], out[:, 5], rtol=1e-13)
    assert not np.allclose(out[:, 0], out[:, 3])


@pytest.mark.parametrize("causal", [True, False])
def test_matches_torch_sdpa_block_diagonal(causal):
    lengths = [3, 17, 1, 30]
    cu = cu_of(lengths)
    t = cu[-1]
    g = torch.Generator().manual_seed(0)
    q = torch.randn(t, 6, 16, generator=g, dtype=torch.float64)
    k = torch.randn(t, 2, 16, generator=g, dtype=torch.float64)
    v = torch.randn(t, 2, 16, generator=g, dtype=torch.float64)
    ref = cpu_path.sdpa_attention(q, k, v, cu, 0.25, causal).numpy()
    out, _ = oa.attention_fwd(q, k, v, cu, cu, 0.25, causal)
    np.testing.assert_allclose(out, ref, rtol=1e-10, atol=1e-12)


def test_bottom_right_causal_alignment():
    # len_q = 2, len_k = 5: q row 0 sees k rows 0..3, q row 1 sees 0..4
    q, k, v = np.zeros((2, 1, 4)), rand((5, 1, 4), 15), rand((5, 1, 4), 16)
    out, lse = oa.attention_fwd(q, k, v, [0, 2], [0, 5], 1.0, True)
    np.testing.assert_allclose(out[0, 0], v[:4, 0].mean(0), rtol=1e-12)
    np.testing.assert_allclose(out[1, 0], v[:5, 0].mean(0), rtol=1e-12)
    np.testing.assert_allclose(lse[0], np.log([4, 5]), rtol=1e-12)


@pytest.mark.parametrize("causal", [True, False])
def test_backward_finite_differences(causal):
    lengths = [3, 5]
    cu = cu_of(lengths)
    t = cu[-1]
    q, k, v = rand((t, 2, 4), 20), rand((t, 1, 4), 21), rand((t, 1, 4), 22)
    do = rand((t, 2, 4), 23)
    scale = 0.7
    dq, dk, dv = oa.attention_bwd(do, q, k, v, cu, cu, scale, causal)

    def f(q_, k_, v_):
        return float((oa.attention_fwd(q_, k_, v_, cu, cu, scale, causal)[0] * do).sum())

    eps = 1e-6
    for name, x, grad in (("q", q, dq), ("k", k, dk), ("v", v, dv)):
        for idx in [(0, 0, 0), (2, 0, 3), (t - 1, x.shape[1] - 1, 1), (4, 0, 2)]:
            xp, xm = x.copy(), x.copy()
            xp[idx] += eps
            xm[idx] -= eps
            args_p = [xp if n == name else y for n, y in (("q", q), ("k", k), ("v", v))]
            args_m = [xm if n == name else y for n, y in (("q", q), ("k", k), ("v", v))]
            num = (f(*args_p) - f(*args_m)) / (2 * eps)
            assert abs(num - grad[idx]) <= 1e-6 * max(1.0, abs(num)), (name, idx, num, grad[idx])


def test_backward_matches_torch_autograd():
    lengths = [7, 12]
    cu = cu_of(lengths)
    t = cu[-1]
    g = torch.Generator().manual_seed(1)
    q = torch.randn(t, 4, 8, generator=g, dtype=torch.float64, requires_grad=True)
    k = torch.randn(t, 2, 8, generator=g, dtype=torch.float64, requires_grad=True)
    v = torch.randn(t, 2, 8, generator=g, dtype=torch.float64, requires_grad=True)
    do = torch.randn(t, 4, 8, generator=g, dtype=torch.float64)
    cpu_path.sdpa_attention(q, k, v, cu, 0.3, True).backward(do)
    dq, dk, dv = oa.attention_bwd(do, q.detach(), k.detach(), v.detach(), cu, cu, 0.3, True)
    np.testing.assert_allclose(dq, q.grad.numpy(), rtol=1e-9, atol=1e-11)
    np.testing.assert_allclose(dk, k.grad.numpy(), rtol=1e-9, atol=1e-11)
    np.testing.assert_allclose(dv, v.grad.numpy(), rtol=1e-9, atol=1e-11)


def test_backward_identities():
    lengths = [9]
    cu = cu_of(lengths)
    q, v, do = rand((9, 2, 4), 30), rand((9, 1, 4), 31), rand((9, 2, 4), 32)
    k = rand((9, 1, 4), 33)
    # every row of dS sums to zero
    sums = oa.attention_bwd_ds_rowsums(do, q, k, v, cu, cu, 0.5, True)
    assert np.max(np.abs(sums)) < 1e-12
    # equal keys: dQ = 0
    k_eq = np.tile(k[:1], (9, 1, 1))
    dq, _, _ = oa.attention_bwd(do, q, k_eq, v, cu, cu, 0.5, False)
    assert np.max(np.abs(dq)) < 1e-12
    # shifting every key by the same vector leaves O, dQ and dV unchanged
    shift = rand((1, 1, 4), 34)
    o1, _ = oa.attention_fwd(q, k, v, cu, cu, 0.5, True)
    o2, _ = oa.attention_fwd(q, k + shift, v, cu, cu, 0.5, True)
    np.testing.assert_allclose(o1, o2, rtol=1e-10, atol=1e-12)
    g1 = oa.attention_bwd(do, q, k, v, cu, cu, 0.5, True)
    g2 = oa.attention_bwd(do, q, k + shift, v, cu, cu, 0.5, True)
    np.testing.assert_allclose(g1[0], g2[0], rtol=1e-9, atol=1e-11)
    np.testing.assert_allclose(g1[2], g2[2], rtol=1e-9, atol=1e-11)


@pytest.mark.parametrize("causal", [True, False])
def test_backward_stored_output_row_term(causal):
    lengths = [11, 5]
    cu = cu_of(lengths)
    t = cu[-1]
    q, k, v, do = rand((t, 4, 8), 40), rand((t, 2, 8), 41), rand((t, 2, 8), 42), rand((t, 4, 8), 43)
    o, _ = oa.attention_fwd(q, k, v, cu, cu, 0.4, causal)
    exact = oa.attention_bwd(do, q, k, v, cu, cu, 0.4, causal)
    # the exact output gives the exact row term: rowsum(dO o O) = rowsum(P o dP)
    stored = oa.attention_bwd(do, q, k, v, cu, cu, 0.4, causal, out=o)
    for a, b in zip(exact, stored):
        np.testing.assert_allclose(b, a, rtol=1e-10, atol=1e-12)
    # a changed output shifts D_i by e_i = rowsum(dO_i o (O'_i - O_i)): dV stays,
    # dQ_i moves by -scale e_i sum_j P_ij K_j (P K is attention with V = K)
    o2 = o + 0.1 * rand(o.shape, 44)
    moved = oa.attention_bwd(do, q, k, v, cu, cu, 0.4, causal, out=o2)
    np.testing.assert_allclose(moved[2], exact[2], rtol=1e-12, atol=1e-12)
    pk, _ = oa.attention_fwd(q, k, k, cu, cu, 0.4, causal)
    e = (do * (o2 - o)).sum(-1, keepdims=True)
    np.testing.assert_allclose(moved[0] - exact[0], -0.4 * e * pk, rtol=1e-9, atol=1e-11)
