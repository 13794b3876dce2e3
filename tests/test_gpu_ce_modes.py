"""GPU checks of the fused CE's other call modes (through the C ABI):

* the loss-only entry point (evaluation under torch.no_grad, as the
  reference's eval_loss pass, scripts/train.py:693-699) gives bitwise the loss,
  count and bad-label count of the training entry point;
* the default chunk (bounded softmax numerators) over several chunks, with
  the valid rows ending in the first, second or third chunk (the dW
  accumulation mode is chosen on the device);
* the autograd op's backward leaves its saved gradients untouched, so a
  second backward through a retained graph is correct;
* labels outside [0, vocab) that are not ignore_index raise, as
  F.cross_entropy does.
"""

import numpy as np
import pytest
import torch

from oracle import cross_entropy as oc
from siq_vl_amd import cross_entropy as C

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


@pytest.mark.parametrize("n,hdim,vocab,div", [(300, 256, 1000, None), (700, 128, 2048, 650.0), (0, 128, 512, None),
                                               (256, 1536, 151936, None)])
def test_loss_only_is_bitwise_the_training_loss(n, hdim, vocab, div):
    h, w, y = make(n, hdim, vocab, seed=11, wscale=0.02)
    if n > 5:
        y[5] = vocab + 3  # a bad label: counted by both
    print(f"flce loss-only n={n} V={vocab}", flush=True)
    d = None if div is None else torch.tensor(div, device=DEV)
    hd, wd, yd = h.to(DEV), w.to(DEV), y.to(DEV)
    l1, c1, b1, _, _ = C.flce_fwd_bwd(hd, wd, yd, -100, d, True, 256)
    l2, c2, b2 = C.flce_loss(hd, wd, yd, -100, d)
    torch.cuda.synchronize()
    assert int(c1) == int(c2) and int(b1) == int(b2)
    assert np.array_equal(l1.cpu().numpy(), l2.cpu().numpy(), equal_nan=True)
    if n:
        ref = oc.linear_ce(h, w, y, divisor=div, block=64)
        assert abs(float(l2) - ref["loss"]) <= TOL * abs(ref["loss"])


def test_no_grad_takes_the_loss_only_path():
    h, w, y = make(200, 128, 512, seed=12)
    hg, wg = h.to(DEV).requires_grad_(True), w.to(DEV).requires_grad_(True)
    with torch.no_grad():
        ev = C.fused_linear_cross_entropy(hg, wg, y.to(DEV))
    assert ev.grad_fn is None
    tr = C.fused_linear_cross_entropy(hg, wg, y.to(DEV))
    assert tr.grad_fn is not None
    assert float(ev) == float(tr.detach())
    # nothing requires grad: also loss only
    frozen = C.fused_linear_cross_entropy(h.to(DEV), w.to(DEV), y.to(DEV))
    assert frozen.grad_fn is None and float(frozen) == float(ev)


@pytest.mark.parametrize("valid_rows", [100, 300, 650, 0])
def test_chunked_dw_accumulation_modes(valid_rows):
    """chunk 256 over 800 rows: the valid rows end in chunk 0, 1 or 2 (or there
    are none), so the dW kernel stores bf16 at once, or starts / continues /
    finishes the fp32 sum, as decided on the device."""
    n, hdim, vocab = 800, 128, 1024
    h, w, y = make(n, hdim, vocab, seed=13, ignore_frac=0.0)
    y[valid_rows:] = -100
    print(f"flce chunked valid={valid_rows}", flush=True)
    loss, count, _, dh, dw = C.flce_fwd_bwd(h.to(DEV), w.to(DEV), y.to(DEV), -100, None, True, 256)
    torch.cuda.synchronize()
    assert int(count) == valid_rows
    if valid_rows == 0:
        assert np.isnan(float(loss)) and bool((dw == 0).all()) and bool((dh == 0).all())
        return
    ref = oc.linear_ce(h, w, y)
    assert abs(float(loss) - ref["loss"]) <= TOL * abs(ref["loss"])
    assert rel(dh.float().cpu().numpy(), ref["dh"]) <= TOL
    assert rel(dw.float().cpu().numpy(), ref["dw"]) <= TOL
    # one chunk of the same valid rows gives the same result up to the fp32 summation order
    _, _, _, _, dw1 = C.flce_fwd_bwd(h.to(DEV), w.to(DEV), y.to(DEV), -100, None, True, 4096)
    assert rel(dw.float().cpu().numpy(), dw1.float().cpu().numpy()) <= 1e-2


def test_default_chunk_spans_several_chunks_at_qwen_vocab():
    # 7000 valid rows > the default 6912-row chunk: two chunks at the default bound
    n, hdim, vocab = 7200, 256, 151936
    h, w, y = make(n, hdim, vocab, seed=14, ignore_frac=0.0, wscale=0.02)
    y[7000:] = -100
    print("flce default chunk, 7000 valid rows at V=151936", flush=True)
    hd, wd, yd = h.to(DEV), w.to(DEV), y.to(DEV)
    loss, count, _, dh, dw = C.flce_fwd_bwd(hd, wd, yd)
    big = C.flce_fwd_bwd(hd, wd, yd, chunk_tokens=8192)
    torch.cuda.synchronize()
    assert int(count) == 7000
    assert float(loss) == float(big[0])  # the loss does not depend on the chunking
    assert torch.equal(dh, big[3])      # nor does dH (each row lies in one chunk either way)
    assert rel(dw.float().cpu().numpy(), big[4].float().cpu().numpy()) <= 1e-2


def test_second_backward_through_retained_graph():
    h, w, y = make(96, 128, 512, seed=15)
    hg, wg = h.to(DEV).requires_grad_(True), w.to(DEV).requires_grad_(True)
    loss = C.fused_linear_cross_entropy(hg, wg, y.to(DEV))
    g1 = torch.autograd.grad(3.0 * loss, [hg, wg], retain_graph=True)
    g2 = torch.autograd.grad(5.0 * loss, [hg, wg], retain_graph=True)
    g3 = torch.autograd.grad(loss, [hg, wg])
    _, _, _, dh, dw = C.flce_fwd_bwd(h.to(DEV), w.to(DEV), y.to(DEV), -100, None, True, None)
    for scale, (gh, gw) in ((3.0, g1), (5.0, g2), (1.0, g3)):
        assert torch.equal(gh, (dh.float() * scale).to(torch.bfloat16))
        assert torch.equal(gw, (dw.float() * scale).to(torch.bfloat16))


def test_out_of_range_label_raises():
    h, w, y = make(64, 128, 256, seed=16)
    y[3] = 256  # vocab is 256: out of range
    hg, wg = h.to(DEV).requires_grad_(True), w.to(DEV)
    with pytest.raises(C.LabelError, match="outside"):
        C.fused_linear_cross_entropy(hg, wg, y.to(DEV), validate="sync")
    # lazy (default): no host sync in the call; raised once the count has landed
    C.check_pending_labels(block=True)  # nothing pending from before
    loss = C.fused_linear_cross_entropy(hg, wg, y.to(DEV))
    assert loss.grad_fn is not None
    with pytest.raises(C.LabelError):
        C.check_pending_labels(block=True)
    C.check_pending_labels(block=True)  # reported once
    with torch.no_grad():
        C.fused_linear_cross_entropy(hg, wg, y.to(DEV))
    with pytest.raises(C.LabelError):
        C.check_pending_labels(block=True)
    # negative labels other than ignore_index too; validate=False never checks
    y2 = y.clone()
    y2[3] = -5
    C.fused_linear_cross_entropy(hg, wg, y2.to(DEV), validate=False)
    C.check_pending_labels(block=True)
    with pytest.raises(C.LabelError):
        C.fused_linear_cross_entropy(hg, wg, y2.to(DEV), validate="sync")


def test_capture_in_a_hip_graph_with_a_lazy_check_pending():
    """The raw training call and the autograd op captured in a HIP graph while
    an earlier call's lazy label check is still pending: inside the capture
    no event is queried and no count is copied, and every replay (with eager
    work and synchronisation between them) gives the eager call's loss, dH and
    dW bit for bit."""
    h, w, y = make(300, 256, 1000, seed=3)
    print("flce graph capture n=300 V=1000", flush=True)
    hd, wd, yd = h.to(DEV), w.to(DEV), y.to(DEV)
    loss_e, _, _, dh_e, dw_e = C.flce_fwd_bwd(hd, wd, yd, -100, None, True, 256)
    hg, wg = hd.clone().requires_grad_(True), wd.clone().requires_grad_(True)
    op_e = C.fused_linear_cross_entropy(hg, wg, yd)  # leaves a lazy check pending
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up off the capture, as graphs want
        C.flce_fwd_bwd(hd, wd, yd, -100, None, True, 256)
        C.fused_linear_cross_entropy(hg, wg, yd)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        loss_g, _, _, dh_g, dw_g = C.flce_fwd_bwd(hd, wd, yd, -100, None, True, 256)
        op_g = C.fused_linear_cross_entropy(hg, wg, yd)
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(loss_g, loss_e) and torch.equal(dh_g, dh_e) and torch.equal(dw_g, dw_e)
        assert torch.equal(op_g.detach(), op_e.detach())
        (hd.float() * 2.0).sum().item()  # eager work between the replays
    C.check_pending_labels(block=True)
