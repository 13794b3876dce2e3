"""GPU parity of the vision-token splice, and a tiny SiQ-VL-shaped model end to end.

Bar: the splice only copies rows, so its output and the vision-row gradient
are bitwise those of the reference's torch ops (embedding, nonzero, index
assignment, autograd), for bf16 and fp32 tables; the embedding table's
gradient is one rounding of the exact per-id sum, deterministic, and bitwise
torch's own where torch takes its sorted path.  End to end, a
small model assembled like SiQ_VLForCausalLM (SigLIP tower -> pixel-shuffle
projector -> splice -> Qwen2 decoder with labels) gives bitwise the stock
logits and gradients with the splice alone patched (the embedding table's
within 1e-2: torch sums a short batch in another order, rounding to bf16 in
between); with every fused operator
of this package on (bf16) its loss stays within 2e-2 and every parameter
gradient within 5e-2 of the stock fp32 model's.
"""

import types

import numpy as np
import pytest
import torch

from oracle import splice as osp
from siq_vl_amd import splice as S

pytestmark = pytest.mark.gpu

DEV = "cuda"
IMG = 250
TOL = 2e-2


def bits(t):
    return t.detach().contiguous().view(torch.int16).cpu()


def make(b, s, vocab, hidden, n_img_rows, seed=0, padding_idx=None, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    ids = torch.randint(0, vocab, (b, s), generator=g)
    ids[ids == IMG] = 1
    flat = ids.view(-1)
    pos = torch.randperm(flat.numel(), generator=g)[:n_img_rows]
    flat[pos] = IMG
    if padding_idx is not None:
        flat[torch.randperm(flat.numel(), generator=g)[:5]] = padding_idx  # some padding tokens too
        flat[pos] = IMG
    emb = torch.nn.Embedding(vocab, hidden, padding_idx=padding_idx)
    with torch.no_grad():
        emb.weight.copy_(torch.randn(vocab, hidden, generator=g))
    vis = torch.randn(n_img_rows, hidden, generator=g)
    return ids.to(DEV), emb.to(DEV).to(dtype), vis.to(torch.bfloat16).to(DEV)


def reference(ids, emb, vis):
    """modeling.py:252-270 as torch runs it."""
    te = emb(ids)
    positions = (ids == IMG).nonzero(as_tuple=True)
    te[positions] = vis.to(dtype=te.dtype)
    return te


def table_grad_oracle(g, ids, vocab, padding_idx):
    """fp64 per-id sum (the oracle's splice_bwd) of the upstream gradient."""
    dw, _ = osp.splice_bwd(g.double().cpu().numpy(), ids.cpu().numpy(), IMG, vocab, padding_idx)
    return dw


@pytest.mark.parametrize("shape", [(1, 1, 0), (2, 37, 9), (3, 300, 256), (1, 4096, 1024), (2, 9000, 512)])
@pytest.mark.parametrize("padding_idx", [None, 0])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_forward_backward(shape, padding_idx, dtype):
    """Forward and the vision rows' gradient bitwise torch's ops (the splice
    copies rows); the table's gradient within one rounding of the fp64 per-id
    sum, deterministic, and bitwise torch's own embedding backward where torch
    takes its sorted path (more than 3072 tokens), whose summation order the
    kernel follows."""
    b, s, nimg = shape
    print(f"splice {shape} padding_idx={padding_idx} dtype={dtype}", flush=True)
    big = s >= 4096
    vocab, hidden = (151936, 1536) if big else (256, 128)
    ids, emb, vis = make(b, s, vocab, hidden, nimg, padding_idx=padding_idx, dtype=dtype)
    g = torch.randn(b, s, hidden, generator=torch.Generator().manual_seed(1)).to(dtype).to(DEV)
    v1 = vis.clone().requires_grad_()
    w1 = emb.weight.detach().clone().requires_grad_()
    out = S.splice_vision_tokens(ids, w1, v1, IMG, padding_idx, validate="sync")
    out.backward(g)
    emb.zero_grad(set_to_none=True)
    v2 = vis.clone().requires_grad_()
    ref = reference(ids, emb, v2)
    ref.backward(g)
    torch.cuda.synchronize()
    assert out.dtype == dtype
    assert torch.equal(out, ref)
    assert torch.equal(v1.grad, v2.grad)
    # the table's gradient: one rounding of the exact per-id sum (fp32 accumulation of at most a few thousand
    # rows stays far inside half a bf16 ulp; for fp32 tables the bound is the fp32 sum's own error)
    exact = torch.from_numpy(table_grad_oracle(g.reshape(-1, hidden), ids.reshape(-1), vocab, padding_idx))
    got = w1.grad.double().cpu()
    if dtype == torch.bfloat16:
        assert torch.equal(w1.grad.cpu(), exact.to(torch.bfloat16)) or \
            bool(((got - exact).abs() <= 2.0**-8 * exact.abs() + 1e-30).all())
    else:
        assert bool(((got - exact).abs() <= 1e-5 * exact.abs().clamp_min(1.0)).all())
    again = S.embedding_bwd(g.reshape(-1, hidden).contiguous(), ids.reshape(-1), vocab, (IMG, padding_idx))
    assert torch.equal(again, w1.grad)  # deterministic
    same_as_torch = torch.equal(w1.grad, emb.weight.grad)
    print(f"  table gradient bitwise torch's: {same_as_torch}", flush=True)
    if b * s > 3072:
        assert same_as_torch
    if s <= 300 and dtype == torch.bfloat16:
        ow = osp.splice_fwd(ids.cpu().numpy(), emb.weight.float().detach().cpu().numpy(),
                            vis.float().cpu().numpy(), IMG)
        assert np.array_equal(out.float().detach().cpu().numpy(), ow)


@pytest.mark.parametrize("n", [1, 100, 20000, 32768, 32769, 40000])
@pytest.mark.parametrize("vis_rows", ["fewer", "equal", "more"])
def test_raw_outputs_both_launch_paths(n, vis_rows):
    """The raw call's three outputs against numpy: up to 32768 tokens one
    kernel counts the image tokens per workgroup, above that a one-workgroup
    scan runs first.  Rows of image tokens past the vision rows and of ids
    outside [0, vocab) are zero; image_pos holds each vision row's token and
    -1 for rows no token took; counts = (image tokens, bad ids)."""
    print(f"splice raw n={n} vision rows {vis_rows}", flush=True)
    g = torch.Generator().manual_seed(n)
    vocab, hidden = 256, 64
    ids = torch.randint(0, vocab, (n,), generator=g)
    ids[ids == IMG] = 1
    n_img = n // 5
    ids[torch.randperm(n, generator=g)[:n_img]] = IMG
    if n > 1:
        ids[torch.randperm(n, generator=g)[:3]] = torch.tensor([-4, vocab, vocab + 77])[: min(3, n)]
    found = int((ids == IMG).sum())
    nv = {"fewer": max(found - 7, 0), "equal": found, "more": found + 11}[vis_rows]
    weight = torch.randn(vocab, hidden, generator=g).to(torch.bfloat16)
    vis = torch.randn(nv, hidden, generator=g).to(torch.bfloat16)
    out, image_pos, counts = S.splice_fwd(ids.to(DEV), weight.to(DEV), vis.to(DEV), IMG)
    torch.cuda.synchronize()
    idn = ids.numpy()
    want = np.zeros((n, hidden), np.float32)
    ok = (idn >= 0) & (idn < vocab) & (idn != IMG)
    want[ok] = weight.float().numpy()[idn[ok]]
    pos = np.nonzero(idn == IMG)[0]
    k = min(len(pos), nv)
    want[pos[:k]] = vis.float().numpy()[:k]
    want_pos = np.full(nv, -1, np.int64)
    want_pos[:k] = pos[:k]
    assert np.array_equal(out.float().cpu().numpy(), want)
    assert np.array_equal(image_pos.cpu().numpy().astype(np.int64), want_pos)
    assert counts.cpu().tolist() == [found, int(((idn < 0) | (idn >= vocab)).sum())]


def test_count_mismatch_and_bad_ids():
    ids, emb, vis = make(2, 50, 256, 64, 10)
    with pytest.raises(ValueError, match="Shape Mismatch"):
        S.splice_vision_tokens(ids, emb.weight, vis[:9], IMG, validate="sync")
    bad = ids.clone()
    bad[0, 3] = 300
    with pytest.raises(IndexError):
        S.splice_vision_tokens(bad, emb.weight, vis, IMG, validate="sync")


def test_lazy_checks_raise_later_and_never_read_garbage():
    """The default validation: the call returns at once; the error comes at the
    next call or check_pending_splices().  Meanwhile a backward through a call
    with fewer placeholders than vision rows gathers zero rows for the missing
    ones (image_pos holds -1 there), never memory past the gradient."""
    S.check_pending_splices(block=True)
    ids, emb, vis = make(2, 50, 256, 64, 10)
    v = torch.cat([vis, vis[:3]]).requires_grad_()  # 13 vision rows, 10 placeholders
    out = S.splice_vision_tokens(ids, emb.weight, v, IMG)
    out.float().sum().backward()
    torch.cuda.synchronize()
    assert bool((v.grad[10:] == 0).all()) and bool((v.grad[:10] == 1).all())
    with pytest.raises(ValueError, match="Shape Mismatch"):
        S.check_pending_splices(block=True)
    S.check_pending_splices(block=True)  # reported once
    bad = ids.clone()
    bad[1, 7] = -4
    S.splice_vision_tokens(bad, emb.weight, vis, IMG)
    with pytest.raises(IndexError):
        S.splice_vision_tokens(ids, emb.weight, vis, IMG)  # raised at the next call
    S.check_pending_splices(block=True)


# ----------------------------------------------------------------- end to end
transformers = pytest.importorskip("transformers")


class Projector(torch.nn.Module):
    """SiQ_VLProjector's structure (modeling.py:37-106)."""

    def __init__(self, dv, n, r):
        super().__init__()
        self.vision_pixel_shuffle_factor = r
        self.mlp = torch.nn.Linear(dv * r * r, n, bias=False)

    def forward(self, x):
        b, seq, d = x.shape
        side, r = int(seq**0.5), self.vision_pixel_shuffle_factor
        xs = x.view(b, side, side, d).reshape(b, side // r, r, side // r, r, d).permute(0, 1, 3, 2, 4, 5).contiguous()
        return self.mlp(xs.reshape(b, (side // r) ** 2, d * r * r))


class TinyVLM(torch.nn.Module):
    """SiQ_VLForCausalLM's structure (modeling.py:200-288) at toy sizes."""

    def __init__(self, attn="eager"):
        super().__init__()
        vcfg = transformers.SiglipVisionConfig(hidden_size=128, intermediate_size=256, num_hidden_layers=1,
                                               num_attention_heads=2, image_size=32, patch_size=4)
        self.vision_model = transformers.SiglipVisionModel._from_config(vcfg, attn_implementation=attn)
        self.projector = Projector(128, 128, 2)
        tcfg = transformers.Qwen2Config(vocab_size=256, hidden_size=128, intermediate_size=256, num_hidden_layers=2,
                                        num_attention_heads=2, num_key_value_heads=1, max_position_embeddings=512,
                                        use_cache=False)
        self.text_model = transformers.Qwen2ForCausalLM._from_config(tcfg, attn_implementation=attn)
        self.config = types.SimpleNamespace(image_token_index=IMG)

    def forward(self, input_ids=None, pixel_values=None, labels=None, **kwargs):
        vf = self.vision_model(pixel_values).last_hidden_state
        vte = self.projector(vf)
        flat = vte.view(-1, vte.size(-1))
        te = self.text_model.get_input_embeddings()(input_ids)
        positions = (input_ids == IMG).nonzero(as_tuple=True)
        if positions[0].numel() != flat.shape[0]:
            raise ValueError("Shape Mismatch!")
        te[positions] = flat.to(dtype=te.dtype)
        return self.text_model(inputs_embeds=te, labels=labels, **kwargs)


def vlm_batch(n_images=2, seq=120):
    g = torch.Generator().manual_seed(5)
    pix = torch.randn(n_images, 3, 32, 32, generator=g)
    ids = torch.randint(0, 240, (1, seq), generator=g)
    ids[0, 10:10 + 16 * n_images] = IMG  # 16 tokens per 8 x 8-patch image after the shuffle
    labels = ids.clone()
    labels[0, :10 + 16 * n_images] = -100
    return ids.to(DEV), pix.to(DEV), labels.to(DEV)


def grads(model):
    return {n: p.grad.detach().clone() for n, p in model.named_parameters() if p.grad is not None}


def test_tiny_vlm_splice_only():
    print("tiny VLM, splice only", flush=True)
    torch.manual_seed(0)
    model = TinyVLM().to(DEV).to(torch.bfloat16)
    ids, pix, labels = vlm_batch()
    out_ref = model(input_ids=ids, pixel_values=pix.to(torch.bfloat16), labels=labels)
    out_ref.loss.backward()
    g_ref = grads(model)
    model.zero_grad(set_to_none=True)
    S.enable_fused_splice(model)
    out = model(input_ids=ids, pixel_values=pix.to(torch.bfloat16), labels=labels)
    out.loss.backward()
    g = grads(model)
    assert torch.equal(bits(out.logits), bits(out_ref.logits))
    table = "text_model.model.embed_tokens.weight"
    for n in g_ref:
        if n == table:
            # 120 tokens: torch's short-batch embedding backward rounds its running sum to bf16 per batch of 64
            # tokens, the kernel once per id (exactly torch's sorted path, checked bitwise above), so where an
            # id's rows nearly cancel the two differ by the intermediate roundings
            r = float((g[n].double() - g_ref[n].double()).norm() / g_ref[n].double().norm())
            assert r <= 1e-2, (n, r)
        else:
            assert torch.equal(bits(g[n]), bits(g_ref[n])), n


def test_tiny_vlm_all_fused_vs_fp32():
    from siq_vl_amd import attention, projector, rope, text_model

    print("tiny VLM, every fused operator", flush=True)
    attention.register()
    torch.manual_seed(0)
    ref = TinyVLM().to(DEV).float()
    torch.manual_seed(0)
    ours = TinyVLM(attn="siq_varlen").to(DEV)
    ours.load_state_dict(ref.state_dict())
    ours = ours.to(torch.bfloat16)
    ids, pix, labels = vlm_batch()
    out_ref = ref(input_ids=ids, pixel_values=pix, labels=labels)
    out_ref.loss.backward()
    g_ref = grads(ref)
    S.enable_fused_splice(ours)
    projector.enable_fused_projector(ours)
    text_model.enable_fused_cross_entropy(ours.text_model)
    rope.enable_fused_rope()
    try:
        out = ours(input_ids=ids, pixel_values=pix.to(torch.bfloat16), labels=labels)
        out.loss.backward()
    finally:
        rope.disable_fused_rope()
    g = grads(ours)
    rl = abs(float(out.loss) - float(out_ref.loss)) / abs(float(out_ref.loss))
    print(f"  loss {float(out.loss):.5f} ref {float(out_ref.loss):.5f} rel {rl:.2e}", flush=True)
    assert rl <= TOL
    # relative to each parameter's gradient norm, floored at 1e-3 of the largest one: some gradients vanish
    # analytically (a key bias only shifts each query's scores uniformly, which softmax ignores), so the fp32
    # reference holds only roundoff there
    gmax = max(float(gr.norm()) for gr in g_ref.values())
    worst = 0.0
    for n, gr in g_ref.items():
        r = float((g[n].float() - gr).norm() / max(float(gr.norm()), 1e-3 * gmax))
        worst = max(worst, r)
        assert r <= 5e-2, (n, r)
    print(f"  worst parameter-gradient relative error {worst:.2e}", flush=True)
