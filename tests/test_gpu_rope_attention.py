"""GPU checks of the rotary embedding fused into the attention kernels
(siq_attn_rope_fwd_plan / siq_attn_rope_bwd_plan, through the C ABI, and the
rotation + attention autograd op built on them).

Bar: bitwise.  The fused path must reproduce, bit for bit, the unfused
pipeline the reference runs -- apply_rotary_pos_emb on q and k
(transformers models/qwen2/modeling_qwen2.py:105-135, here the bitwise RoPE
kernels) then attention forward, and in the backward attention then the
rotation's backward: out, lse, the rotated q, dq (of the q before rotation),
dk (of k before rotation, via the k-only pass) and dv.  Also checked: a tiny
bf16 Qwen2 on the siq_varlen backend gives the same logits and parameter
gradients with enable_fused_rope_attention as with the unfused RoPE, on the
cu_seq_lens, position_ids and padding-mask routes.
"""

import pytest
import torch

from oracle import rope as orope
from siq_vl_amd import attention as A
from siq_vl_amd import rope as R

pytestmark = pytest.mark.gpu

DEV = "cuda"


def bits(t):
    return t.detach().contiguous().view(torch.int16).cpu()


def same(a, b):
    return torch.equal(bits(a), bits(b))


def make(lengths, hq, hkv, d, seed=0):
    g = torch.Generator().manual_seed(seed)
    t = sum(lengths)
    mk = lambda h: torch.randn(t, h, d, generator=g).to(torch.bfloat16).to(DEV)
    pos = torch.cat([torch.arange(n) for n in lengths])
    cos, sin = orope.qwen2_cos_sin(pos.numpy()[None], d)
    cos = torch.tensor(cos[0]).to(torch.bfloat16).to(DEV)
    sin = torch.tensor(sin[0]).to(torch.bfloat16).to(DEV)
    cu = [0]
    for n in lengths:
        cu.append(cu[-1] + n)
    return mk(hq), mk(hkv), mk(hkv), mk(hq), cos, sin, torch.tensor(cu, dtype=torch.int32, device=DEV)


@pytest.mark.parametrize("lengths,hq,hkv,d,causal", [
    ([1, 17, 130, 257, 64, 600, 2], 12, 2, 128, True),
    ([300, 5, 1000], 14, 2, 64, True),
    ([200, 333], 8, 8, 128, False),
    ([81] * 7 + [640], 12, 2, 128, True),
])
def test_fused_is_bitwise_the_unfused_pipeline(lengths, hq, hkv, d, causal):
    print(f"rope+attention lengths={lengths[:6]} hq={hq} hkv={hkv} d={d} causal={causal}", flush=True)
    q, k, v, do, cos, sin, cu = make(lengths, hq, hkv, d)
    scale = d**-0.5
    # unfused: RoPE of q and k, attention, attention backward, RoPE backward
    qe_ref, ke_ref = R.rope_fwd(q[None], k[None], cos[None], sin[None])
    qe_ref, ke_ref = qe_ref[0], ke_ref[0]
    out_ref, lse_ref = A.varlen_attn_fwd(qe_ref, ke_ref, v, cu, cu, 0, 0, scale, causal)
    dqe, dke, dv_ref = A.varlen_attn_bwd(do, qe_ref, ke_ref, v, out_ref, lse_ref, cu, cu, 0, 0, scale, causal)
    dq_ref, dk_ref = R.rope_bwd(dqe[None], dke[None], cos[None], sin[None])
    # fused: k-only rotation, attention with q rotated in the kernels
    ke = R.rotate_k(k[None], cos[None], sin[None])[0]
    out, lse, qe = A.varlen_attn_rope_fwd(q, ke, v, cos, sin, cu, cu, 0, 0, scale, causal)
    dq, dke2, dv = A.varlen_attn_rope_bwd(do, qe, ke, v, out, lse, cos, sin, cu, cu, 0, 0, scale, causal)
    dk = R._k_only("siq_rope_bwd", dke2[None], cos[None], sin[None])[0]
    torch.cuda.synchronize()
    assert same(ke, ke_ref) and same(qe, qe_ref)
    assert same(out, out_ref) and torch.equal(lse, lse_ref)
    assert same(dq, dq_ref[0]) and same(dk, dk_ref[0]) and same(dv, dv_ref)


def test_autograd_op_matches_unfused_autograd():
    q, k, v, do, cos, sin, cu = make([40, 300, 7], 12, 2, 128, seed=3)
    xq, xk, xv = (t.clone().requires_grad_(True) for t in (q, k, v))
    out = A.flash_attn_varlen_rope_func(xq, xk, xv, cos, sin, cu, cu, 300, 300, causal=True)
    out.backward(do)
    yq, yk, yv = (t.clone().requires_grad_(True) for t in (q, k, v))
    qe, ke2 = R.apply_rotary_pos_emb(yq[None], yk[None], cos[None], sin[None], unsqueeze_dim=2)
    out2 = A.flash_attn_varlen_func(qe[0], ke2[0], yv, cu, cu, 300, 300, causal=True)
    out2.backward(do)
    assert same(out, out2)
    for a, b in ((xq, yq), (xk, yk), (xv, yv)):
        assert same(a.grad, b.grad)


transformers = pytest.importorskip("transformers")


def _qwen(head_dim, seed=0):
    A.register()
    heads = 4
    cfg = transformers.Qwen2Config(vocab_size=512, hidden_size=heads * head_dim, intermediate_size=512,
                                   num_hidden_layers=2, num_attention_heads=heads, num_key_value_heads=2,
                                   max_position_embeddings=4096, use_cache=False)
    torch.manual_seed(seed)
    return transformers.Qwen2ForCausalLM._from_config(cfg, attn_implementation="siq_varlen").to(DEV).to(
        torch.bfloat16)


@pytest.mark.parametrize("route", ["cu_seq_lens", "position_ids", "mask"])
@pytest.mark.parametrize("head_dim", [128, 64])
def test_dropin_qwen2_bitwise(route, head_dim):
    print(f"rope+attention drop-in route={route} d={head_dim}", flush=True)
    lengths = [37, 130, 1, 64, 90]
    g = torch.Generator().manual_seed(1)
    ids = [torch.randint(0, 512, (n,), generator=g) for n in lengths]
    if route == "mask":
        s = max(lengths)
        input_ids = torch.zeros(len(lengths), s, dtype=torch.int64)
        mask = torch.zeros(len(lengths), s, dtype=torch.int64)
        for i, r in enumerate(ids):
            input_ids[i, :len(r)] = r
            mask[i, :len(r)] = 1
        kwargs = {"input_ids": input_ids.to(DEV), "attention_mask": mask.to(DEV)}
    else:
        flat = torch.cat(ids)[None]
        pos = torch.cat([torch.arange(n) for n in lengths])[None]
        kwargs = {"input_ids": flat.to(DEV), "position_ids": pos.to(DEV)}
        if route == "cu_seq_lens":
            cu = torch.tensor([0] + list(torch.tensor(lengths).cumsum(0).tolist()), dtype=torch.int32, device=DEV)
            kwargs.update(cu_seq_lens_q=cu, cu_seq_lens_k=cu, max_length_q=max(lengths), max_length_k=max(lengths))
    model = _qwen(head_dim)

    def run():
        model.zero_grad(set_to_none=True)
        logits = model(**kwargs).logits
        logits.float().square().mean().backward()
        return logits.detach(), {n: p.grad.detach().clone() for n, p in model.named_parameters()}

    R.enable_fused_rope()
    try:
        ref_logits, ref_grads = run()
        assert R.enable_fused_rope_attention(model) == 2
        logits, grads = run()
    finally:
        R.disable_fused_rope()
    if route == "mask":  # padded positions carry no defined output; compare the real tokens
        keep = kwargs["attention_mask"].bool()
        logits, ref_logits = logits[keep], ref_logits[keep]
    assert same(logits, ref_logits)
    for n in ref_grads:
        # the embedding gradient is an atomic scatter-add: not bitwise repeatable on its own
        if "embed_tokens" not in n:
            assert same(grads[n], ref_grads[n]), n


@pytest.mark.parametrize("route", ["cu_seq_lens", "position_ids"])
def test_dropin_qwen2_autocast_over_fp32_weights_bitwise(route):
    """The reference's bf16=True training: fp32 master weights, bf16 autocast
    (scripts/train.py:712), so the rotary embedding hands fp32 cos / sin to
    bf16 q / k and the rotation runs in fp32.  With the rotation fused into
    the attention (fp32 rotation rounded once to bf16, as the attention's cast
    rounds it) the logits and every parameter gradient are bitwise those of
    siq_varlen alone with the stock rotation."""
    print(f"rope+attention drop-in under autocast route={route}", flush=True)
    lengths = [37, 130, 1, 64, 90]
    g = torch.Generator().manual_seed(3)
    ids = [torch.randint(0, 512, (n,), generator=g) for n in lengths]
    flat = torch.cat(ids)[None]
    pos = torch.cat([torch.arange(n) for n in lengths])[None]
    kwargs = {"input_ids": flat.to(DEV), "position_ids": pos.to(DEV)}
    if route == "cu_seq_lens":
        cu = torch.tensor([0] + list(torch.tensor(lengths).cumsum(0).tolist()), dtype=torch.int32, device=DEV)
        kwargs.update(cu_seq_lens_q=cu, cu_seq_lens_k=cu, max_length_q=max(lengths), max_length_k=max(lengths))
    model = _qwen(128).float()

    def run():
        model.zero_grad(set_to_none=True)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            logits = model(**kwargs).logits
        logits.float().square().mean().backward()
        return logits.detach(), {n: p.grad.detach().clone() for n, p in model.named_parameters()}

    ref_logits, ref_grads = run()
    assert R.enable_fused_rope_attention(model) == 2
    logits, grads = run()
    assert logits.dtype == torch.bfloat16
    assert same(logits, ref_logits)
    for n in ref_grads:
        if "embed_tokens" not in n:  # the embedding gradient is an atomic scatter-add
            assert same(grads[n], ref_grads[n]), n


def test_dropin_falls_back_where_it_cannot_fuse():
    # fp32 activations: the stock forward (with the stock rotation) runs unchanged
    model = _qwen(64).float()
    R.enable_fused_rope_attention(model)
    ids = torch.randint(0, 512, (1, 50), device=DEV)
    logits = model(input_ids=ids).logits
    assert logits.dtype == torch.float32 and torch.isfinite(logits).all()
