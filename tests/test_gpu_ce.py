"""GPU parity of the fused linear cross-entropy (through the C ABI).

Small shapes against the fp64 CPU oracle; the full BASELINE shape against an
fp32 torch reference computed in row chunks on the GPU.  Tolerance: relative
Frobenius error <= 2e-2 for loss, dhidden, dweight; the valid-row count and the
zero rows of ignored labels are exact.
"""

import numpy as np
import pytest
import torch

from oracle import cross_entropy as oc
from siq_vl_amd import cross_entropy as C
from siq_vl_amd import workloads as W

pytestmark = pytest.mark.gpu

TOL = 2e-2
DEV = "cuda"


def rel(x, ref) -> float:
    x = np.asarray(x, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.linalg.norm(x - ref) / max(np.linalg.norm(ref), 1e-30))


def make(n, hdim, vocab, seed=0, ignore_frac=0.3, wscale=0.05):
    g = torch.Generator().manual_seed(seed)
    h = torch.randn(n, hdim, generator=g).to(torch.bfloat16)
    w = (wscale * torch.randn(vocab, hdim, generator=g)).to(torch.bfloat16)
    y = torch.randint(0, vocab, (n,), generator=g)
    y[torch.rand(n, generator=g) < ignore_frac] = -100
    return h, w, y


def run(h, w, y, chunk, divisor=None, need_dw=True):
    div = None if divisor is None else torch.tensor(float(divisor), device=DEV)
    loss, count, bad, dh, dw = C.flce_fwd_bwd(h.to(DEV), w.to(DEV), y.to(DEV), -100, div, need_dw, chunk)
    torch.cuda.synchronize()
    return (float(loss), int(count), int(bad), dh.float().cpu().numpy(),
            None if dw is None else dw.float().cpu().numpy())


@pytest.mark.parametrize("chunk", [128, 4096])
def test_small_vs_oracle(chunk):
    h, w, y = make(300, 256, 1000, seed=1)
    y[5] = 1000  # out of range: counted as bad, treated as ignored
    print(f"flce small chunk={chunk}", flush=True)
    loss, count, bad, dh, dw = run(h, w, y, chunk)
    ref = oc.linear_ce(h, w, y)
    assert count == ref["count"] and bad == ref["bad"] == 1
    assert abs(loss - ref["loss"]) <= TOL * abs(ref["loss"])
    assert rel(dh, ref["dh"]) <= TOL
    assert rel(dw, ref["dw"]) <= TOL
    ignored = (y == -100) | (y >= 1000)
    assert np.all(dh[ignored.numpy()] == 0.0)


@pytest.mark.parametrize("hdim,vocab", [(896, 2000), (320, 1000)])
def test_hidden_sizes_off_the_tile_grid(hdim, vocab):
    """hdim 896 (Qwen2.5-0.5B: three whole 256-wide tiles of the gradient
    GEMMs and a half one) and 320 (one whole tile and a quarter), with a
    vocabulary that ends inside a tile, over three chunks."""
    h, w, y = make(300, hdim, vocab, seed=31)
    print(f"flce hdim={hdim} V={vocab}", flush=True)
    loss, count, bad, dh, dw = run(h, w, y, 128)
    ref = oc.linear_ce(h, w, y)
    assert count == ref["count"] and bad == 0
    assert abs(loss - ref["loss"]) <= TOL * abs(ref["loss"])
    assert rel(dh, ref["dh"]) <= TOL and rel(dw, ref["dw"]) <= TOL
    assert np.all(dh[(y == -100).numpy()] == 0.0)


def test_sum_reduction_with_divisor():
    h, w, y = make(200, 128, 520, seed=2)
    loss, count, _, dh, dw = run(h, w, y, 64, divisor=517.0)
    ref = oc.linear_ce(h, w, y, divisor=517.0)
    assert count == ref["count"]
    assert abs(loss - ref["loss"]) <= TOL * abs(ref["loss"])
    assert rel(dh, ref["dh"]) <= TOL and rel(dw, ref["dw"]) <= TOL


def test_all_ignored_gives_nan_and_zero_grads():
    h, w, y = make(64, 64, 256, seed=3)
    y[:] = -100
    loss, count, bad, dh, dw = run(h, w, y, 4096)
    assert count == 0 and bad == 0 and np.isnan(loss)
    assert np.all(dh == 0.0) and np.all(dw == 0.0)


def test_no_ignored_rows_several_chunks():
    h, w, y = make(600, 256, 1000, seed=8, ignore_frac=0.0)
    loss, count, bad, dh, dw = run(h, w, y, 256)
    ref = oc.linear_ce(h, w, y)
    assert count == ref["count"] == 600 and bad == 0
    assert abs(loss - ref["loss"]) <= TOL * abs(ref["loss"])
    assert rel(dh, ref["dh"]) <= TOL and rel(dw, ref["dw"]) <= TOL


@pytest.mark.parametrize("chunk", [4096, 512])
def test_ignored_rows_cost_nothing_but_a_zero_row(chunk):
    """Rows whose label is ignored are compacted away before the GEMMs: the batch
    gives bitwise the loss, dW and valid-row dH of the valid rows alone."""
    g = torch.Generator().manual_seed(9)
    h = torch.randn(2048, 512, generator=g).to(torch.bfloat16)
    w = (0.05 * torch.randn(4096, 512, generator=g)).to(torch.bfloat16)
    y = W.span_masked_labels(2048, 4096, 0.3, g)
    valid = (y != -100).numpy()
    print(f"flce compaction chunk={chunk} valid={int(valid.sum())}", flush=True)
    full = run(h, w, y, chunk)
    sub = run(h[valid], w, y[valid], chunk)
    assert full[1] == sub[1] == int(valid.sum())
    assert full[0] == sub[0]
    assert np.array_equal(full[3][valid], sub[3]) and np.all(full[3][~valid] == 0.0)
    if chunk >= 2048:  # one chunk either way: the same rows in the same k-steps
        assert np.array_equal(full[4], sub[4])
    else:
        assert rel(full[4], sub[4]) <= 1e-2


def test_qwen_vocab_vs_oracle():
    h, w, y = make(256, 1536, W.QWEN_VOCAB, seed=4, wscale=0.02)
    print("flce qwen vocab n=256", flush=True)
    loss, count, _, dh, dw = run(h, w, y, 4096)
    ref = oc.linear_ce(h, w, y, block=64)
    assert count == ref["count"]
    assert abs(loss - ref["loss"]) <= TOL * abs(ref["loss"])
    assert rel(dh, ref["dh"]) <= TOL and rel(dw, ref["dw"]) <= TOL


def test_vocab_past_one_factor_segment_vs_oracle():
    """V = 270000: 1055 vocab tiles, more than the row pass keeps factors for
    at once (1024), so it streams each row in two segments; the last tile
    holds 176 columns.  Two chunks, so dW is also summed over chunks."""
    h, w, y = make(96, 64, 270000, seed=9, wscale=0.05)
    y[7] = 269999  # the last column of the partial last tile
    y[8] = 262143  # the last column of the first segment
    y[9] = 262144  # the first column of the second segment
    print("flce vocab 270000 n=96 chunk=64", flush=True)
    loss, count, _, dh, dw = run(h, w, y, 64)
    ref = oc.linear_ce(h, w, y, block=32)
    assert count == ref["count"]
    assert abs(loss - ref["loss"]) <= TOL * abs(ref["loss"])
    assert rel(dh, ref["dh"]) <= TOL and rel(dw, ref["dw"]) <= TOL
    # the labelled columns' dW rows are dominated by the -g term: check them alone too
    for v in (269999, 262143, 262144):
        assert rel(dw[v], ref["dw"][v]) <= TOL, v


def test_large_logits_keep_relative_precision():
    # logits of magnitude ~30: the exp-normalised chunk buffer keeps precision
    h, w, y = make(128, 256, 2048, seed=6, wscale=2.0)
    loss, _, _, dh, dw = run(h, w, y, 4096)
    ref = oc.linear_ce(h, w, y)
    assert abs(loss - ref["loss"]) <= TOL * abs(ref["loss"])
    assert rel(dh, ref["dh"]) <= TOL and rel(dw, ref["dw"]) <= TOL


@pytest.mark.parametrize("n,hdim,vocab,chunk", [(300, 256, 1000, 128), (300, 256, 1000, 4096),
                                                (256, 1536, W.QWEN_VOCAB, 4096)])
def test_dh_only_vs_oracle(n, hdim, vocab, chunk):
    """The call of a frozen lm_head (dweight = NULL: the reference's stage 1,
    siq_vl/model/modeling.py:329-330, and stage 2's LoRA, which leaves lm_head
    out of its targets, :377-386): loss and dH against the oracle, ignored
    rows exactly zero, and bitwise the loss and dH of the call that also
    forms dW."""
    h, w, y = make(n, hdim, vocab, seed=21, wscale=0.05 if vocab < 4096 else 0.02)
    y[5] = vocab + 1  # out of range: counted as bad, treated as ignored
    print(f"flce dH only n={n} V={vocab} chunk={chunk}", flush=True)
    loss, count, bad, dh, dw = run(h, w, y, chunk, need_dw=False)
    assert dw is None
    ref = oc.linear_ce(h, w, y, block=64)
    assert count == ref["count"] and bad == ref["bad"] == 1
    assert abs(loss - ref["loss"]) <= TOL * abs(ref["loss"])
    assert rel(dh, ref["dh"]) <= TOL
    ignored = ((y == -100) | (y >= vocab)).numpy()
    assert np.all(dh[ignored] == 0.0)
    both = run(h, w, y, chunk, need_dw=True)
    assert both[0] == loss and np.array_equal(both[3], dh)


def test_frozen_lm_head_autograd_takes_the_dh_only_call():
    """hidden requires grad, the weight does not: the autograd op forms no dW
    and hidden's gradient is the raw dH-only call's, scaled."""
    h, w, y = make(200, 128, 768, seed=22)
    hg = h.to(DEV).requires_grad_(True)
    wd = w.to(DEV)
    loss = C.fused_linear_cross_entropy(hg, wd, y.to(DEV), chunk_tokens=64)
    (2.0 * loss).backward()
    assert wd.grad is None
    _, _, _, dh, dw = run(h, w, y, 64, need_dw=False)
    assert dw is None
    assert np.array_equal(hg.grad.float().cpu().numpy(), (torch.from_numpy(dh) * 2.0).to(torch.bfloat16).float().numpy())


def test_autograd_matches_raw_and_scales():
    h, w, y = make(96, 128, 512, seed=8)
    hg = h.to(DEV).requires_grad_(True)
    wg = w.to(DEV).requires_grad_(True)
    loss = C.fused_linear_cross_entropy(hg, wg, y.to(DEV), chunk_tokens=64)
    (3.0 * loss).backward()
    _, _, _, dh, dw = run(h, w, y, 64)
    assert np.allclose(hg.grad.float().cpu().numpy(), 3.0 * dh, rtol=1e-2, atol=1e-6)
    assert np.allclose(wg.grad.float().cpu().numpy(), 3.0 * dw, rtol=1e-2, atol=1e-6)


@pytest.mark.slow
def test_full_size_vs_torch_fp32():
    """Config 4 at full size, both the training call (dH and dW) and the
    frozen-lm_head call (dH only), against one fp32 torch reference."""
    cfg = W.CONFIG4
    print(f"flce full size n={cfg.n} hdim={cfg.hdim} V={cfg.vocab}", flush=True)
    x = W.ce_inputs(cfg, device=DEV)
    loss, count, bad, dh, dw = C.flce_fwd_bwd(x["hidden"], x["weight"], x["labels"])
    loss_h, count_h, bad_h, dh_h, dw_h = C.flce_fwd_bwd(x["hidden"], x["weight"], x["labels"], need_dweight=False)
    assert dw_h is None and int(count_h) == int(count) and int(bad_h) == int(bad)
    assert float(loss_h) == float(loss) and torch.equal(dh_h, dh)
    del dh_h
    hf = x["hidden"].float()
    wf = x["weight"].float()
    y = x["labels"]
    valid = y != -100
    cnt = int(valid.sum())
    assert int(count) == cnt and int(bad) == 0
    ref_loss = torch.zeros((), device=DEV, dtype=torch.float64)
    ref_dh = torch.empty_like(hf)
    ref_dw = torch.zeros_like(wf)
    for r0 in range(0, cfg.n, 2048):
        z = hf[r0:r0 + 2048] @ wf.t()
        yb = y[r0:r0 + 2048]
        ref_loss += torch.nn.functional.cross_entropy(z, yb, ignore_index=-100, reduction="sum").double()
        p = torch.softmax(z, -1)
        vb = yb != -100
        idx = torch.nonzero(vb).reshape(-1)
        p[idx, yb[idx]] -= 1.0
        p[~vb] = 0.0
        p /= cnt
        ref_dh[r0:r0 + 2048] = p @ wf
        ref_dw += p.t() @ hf[r0:r0 + 2048]
        del z, p
    ref_loss = float(ref_loss / cnt)
    r_loss = abs(float(loss) - ref_loss) / abs(ref_loss)
    r_dh = float((dh.float() - ref_dh).norm() / ref_dh.norm())
    r_dw = float((dw.float() - ref_dw).norm() / ref_dw.norm())
    print(f"  loss {float(loss):.6f} ref {ref_loss:.6f} rel {r_loss:.2e}; dh rel {r_dh:.2e}; dw rel {r_dw:.2e}",
          flush=True)
    assert r_loss <= TOL and r_dh <= TOL and r_dw <= TOL
    assert bool((dh[~valid] == 0).all())
