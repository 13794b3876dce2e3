"""GPU parity of the fused RoPE (through the C ABI).

Bar: bitwise.  The kernel repeats the bf16 roundings of the reference's torch
ops, so its outputs must equal, bit for bit, (a) the CPU oracle
(oracle/rope.py, itself pinned to torch's bf16 ops and autograd) and (b) the
reference formula run by torch on the GPU on the same inputs -- forward and
backward, for the layouts the reference produces ([B, H, S, D] transposed
views), for [B, S, H, D] inputs, strided and broadcast cos / sin, packed
position ids, empty inputs and the config-2 shape.
"""

import numpy as np
import pytest
import torch

from oracle import rope as orope
from siq_vl_amd import rope as R

pytestmark = pytest.mark.gpu

DEV = "cuda"


def rotate_half_t(x):
    x1 = x[..., : x.shape[-1] // 2]
    x2 = x[..., x.shape[-1] // 2:]
    return torch.cat((-x2, x1), dim=-1)


def torch_rope(q, k, cos, sin, unsqueeze_dim=1):
    """transformers models/qwen2/modeling_qwen2.py:105-135 as the reference runs it."""
    cos = cos.unsqueeze(unsqueeze_dim)
    sin = sin.unsqueeze(unsqueeze_dim)
    return (q * cos) + (rotate_half_t(q) * sin), (k * cos) + (rotate_half_t(k) * sin)


def projected(b, s, h, d, g):
    """q / k as Qwen2Attention hands them over: a [B, S, H*D] projection viewed as [B, H, S, D]."""
    return torch.randn(b, s, h * d, generator=g).to(torch.bfloat16).to(DEV).view(b, s, h, d).transpose(1, 2)


def make(b, s, hq, hkv, d, seed=0, positions=None):
    g = torch.Generator().manual_seed(seed)
    q = projected(b, s, hq, d, g)
    k = projected(b, s, hkv, d, g)
    pos = positions if positions is not None else torch.arange(s).repeat(b, 1)
    cos, sin = orope.qwen2_cos_sin(pos.numpy(), d)
    return q, k, torch.tensor(cos).to(torch.bfloat16).to(DEV), torch.tensor(sin).to(torch.bfloat16).to(DEV)


def bits(t):
    return t.detach().contiguous().view(torch.int16).cpu()


def same(a, b):
    return torch.equal(bits(a), bits(b))


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("shape", [(1, 1, 1, 1), (2, 37, 4, 2), (3, 130, 12, 2)])
def test_forward_bitwise(d, shape):
    b, s, hq, hkv = shape
    print(f"rope fwd d={d} shape={shape}", flush=True)
    q, k, cos, sin = make(b, s, hq, hkv, d)
    qe, ke = R.apply_rotary_pos_emb(q, k, cos, sin)
    torch.cuda.synchronize()
    rq, rk = torch_rope(q, k, cos, sin)
    assert qe.shape == q.shape and ke.shape == k.shape
    assert same(qe, rq) and same(ke, rk)
    c = cos.float().cpu().numpy()[:, None]
    sn = sin.float().cpu().numpy()[:, None]
    assert np.array_equal(orope.rope_fwd(q.float().cpu().numpy(), c, sn), qe.float().cpu().numpy())
    assert np.array_equal(orope.rope_fwd(k.float().cpu().numpy(), c, sn), ke.float().cpu().numpy())


@pytest.mark.parametrize("d", [64, 128])
def test_backward_bitwise(d):
    print(f"rope bwd d={d}", flush=True)
    q, k, cos, sin = make(2, 53, 6, 2, d, seed=1)
    g = torch.Generator().manual_seed(2)
    gq = torch.randn(q.shape, generator=g).to(torch.bfloat16).to(DEV)
    gk = torch.randn(k.shape, generator=g).to(torch.bfloat16).to(DEV)
    q1, k1 = q.detach().clone().requires_grad_(), k.detach().clone().requires_grad_()
    qe, ke = R.apply_rotary_pos_emb(q1, k1, cos, sin)
    torch.autograd.backward((qe, ke), (gq, gk))
    q2, k2 = q.detach().clone().requires_grad_(), k.detach().clone().requires_grad_()
    rq, rk = torch_rope(q2, k2, cos, sin)
    torch.autograd.backward((rq, rk), (gq, gk))
    assert same(q1.grad, q2.grad) and same(k1.grad, k2.grad)
    c = cos.float().cpu().numpy()[:, None]
    sn = sin.float().cpu().numpy()[:, None]
    assert np.array_equal(orope.rope_bwd(gq.float().cpu().numpy(), c, sn), q1.grad.float().cpu().numpy())


def test_bshd_layout_strided_and_broadcast_cos():
    print("rope layouts", flush=True)
    g = torch.Generator().manual_seed(3)
    b, s, hq, hkv, d = 2, 40, 4, 2, 128
    # [B, S, H, D] inputs (unsqueeze_dim=2) carved out of wider buffers: non-contiguous rows
    qbuf = torch.randn(b, s, hq + 2, d, generator=g).to(torch.bfloat16).to(DEV)
    kbuf = torch.randn(b, s, hkv + 1, d, generator=g).to(torch.bfloat16).to(DEV)
    q, k = qbuf[:, :, 1:hq + 1], kbuf[:, :, :hkv]
    cos1, sin1 = orope.qwen2_cos_sin(np.arange(s)[None], d)
    cos = torch.tensor(cos1).to(torch.bfloat16).to(DEV)  # [1, S, D]: shared by the batch
    sin = torch.tensor(sin1).to(torch.bfloat16).to(DEV)
    qe, ke = R.apply_rotary_pos_emb(q, k, cos, sin, unsqueeze_dim=2)
    rq, rk = torch_rope(q, k, cos, sin, unsqueeze_dim=2)
    assert same(qe, rq) and same(ke, rk)


def test_packed_positions():
    print("rope packed positions", flush=True)
    lens = [81, 600, 7, 1, 311]
    pos = torch.cat([torch.arange(n) for n in lens])[None]
    q, k, cos, sin = make(1, int(pos.shape[1]), 12, 2, 128, seed=4, positions=pos)
    qe, ke = R.apply_rotary_pos_emb(q, k, cos, sin)
    rq, rk = torch_rope(q, k, cos, sin)
    assert same(qe, rq) and same(ke, rk)
    # every sequence start (position 0) is left unchanged
    starts = np.cumsum([0] + lens[:-1])
    assert same(qe[:, :, starts], q[:, :, starts])


def test_empty():
    q, k, cos, sin = make(2, 0, 4, 2, 64)
    qe, ke = R.apply_rotary_pos_emb(q, k, cos, sin)
    assert qe.shape == q.shape and ke.shape == k.shape


def test_rejects_fp32_without_original():
    q, k, cos, sin = make(1, 8, 2, 1, 64)
    R.disable_fused_rope()
    with pytest.raises(ValueError):
        R.apply_rotary_pos_emb(q.float(), k.float(), cos.float(), sin.float())


@pytest.mark.slow
def test_config2_shape_bitwise():
    # Qwen2.5-1.5B heads at the bench's packed shape: 16384 tokens, 12 q / 2 kv heads, d 128
    print("rope config-2 shape", flush=True)
    from siq_vl_amd import workloads as W

    cfg = W.attn_config(2)
    cu = cfg.cu_seqlens().tolist()
    pos = torch.cat([torch.arange(cu[i + 1] - cu[i]) for i in range(len(cu) - 1)])[None]
    q, k, cos, sin = make(1, cfg.total, 12, 2, 128, seed=5, positions=pos)
    q.requires_grad_(True)
    k.requires_grad_(True)
    qe, ke = R.apply_rotary_pos_emb(q, k, cos, sin)
    rq, rk = torch_rope(q.detach(), k.detach(), cos, sin)
    assert same(qe, rq) and same(ke, rk)
    g = torch.Generator().manual_seed(6)
    gq = torch.randn(q.shape, generator=g).to(torch.bfloat16).to(DEV)
    gk = torch.randn(k.shape, generator=g).to(torch.bfloat16).to(DEV)
    torch.autograd.backward((qe, ke), (gq, gk))
    c = cos.float().cpu().numpy()[:, None]
    sn = sin.float().cpu().numpy()[:, None]
    assert np.array_equal(orope.rope_bwd(gk.float().cpu().numpy(), c, sn), k.grad.float().cpu().numpy())


def test_dropin_qwen2_bitwise():
    """enable_fused_rope() leaves a bf16 Qwen2's logits and gradients bit-identical."""
    transformers = pytest.importorskip("transformers")
    print("rope drop-in qwen2", flush=True)
    cfg = transformers.Qwen2Config(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                                   num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=1024,
                                   use_cache=False)
    torch.manual_seed(0)
    model = transformers.Qwen2ForCausalLM._from_config(cfg, attn_implementation="eager").to(DEV).to(torch.bfloat16)
    ids = torch.randint(0, 512, (2, 70), generator=torch.Generator().manual_seed(1)).to(DEV)

    def run():
        model.zero_grad(set_to_none=True)
        logits = model(input_ids=ids).logits
        logits.float().square().mean().backward()
        return logits.detach(), {n: p.grad.detach().clone() for n, p in model.named_parameters()}

    R.disable_fused_rope()
    ref_logits, ref_grads = run()
    R.enable_fused_rope()
    try:
        from transformers.models.qwen2 import modeling_qwen2 as m

        assert m.apply_rotary_pos_emb is R.apply_rotary_pos_emb
        logits, grads = run()
    finally:
        R.disable_fused_rope()
    assert same(logits, ref_logits)
    for n in ref_grads:
        # the embedding gradient is an atomic scatter-add: not bitwise repeatable on its own
        if "embed_tokens" not in n:
            assert same(grads[n], ref_grads[n]), n


@pytest.mark.parametrize("d", [16, 48, 80])
def test_other_head_dims_bitwise(d):
    # chunk counts that are not powers of two (and leave block threads idle)
    print(f"rope d={d}", flush=True)
    q, k, cos, sin = make(2, 45, 5, 3, d, seed=7)
    qe, ke = R.apply_rotary_pos_emb(q, k, cos, sin)
    rq, rk = torch_rope(q, k, cos, sin)
    assert same(qe, rq) and same(ke, rk)


def test_in_place_through_the_abi():
    print("rope in place", flush=True)
    q, k, cos, sin = make(2, 33, 4, 2, 128, seed=8)
    rq, rk = torch_rope(q, k, cos, sin)
    bq = R._bshd(q, 1).contiguous()
    bk = R._bshd(k, 1).contiguous()
    R._launch("siq_rope_fwd", bq, bk, cos, sin, bq, bk)  # outputs are the inputs
    assert same(bq, R._bshd(rq, 1)) and same(bk, R._bshd(rk, 1))


def fp32_cos_sin(b, s, d, theta=1000000.0):
    """cos / sin as Qwen2RotaryEmbedding returns them for fp32 hidden states
    (bf16 autocast over fp32 master weights): fp32, not rounded to bf16."""
    pos = torch.arange(s, dtype=torch.float32).repeat(b, 1)
    inv = 1.0 / (theta ** (torch.arange(0, d, 2, dtype=torch.float32) / d))
    emb = torch.cat([pos[..., None] * inv, pos[..., None] * inv], dim=-1)
    return emb.cos().to(DEV), emb.sin().to(DEV)


@pytest.mark.parametrize("d", [64, 128])
def test_fp32_cos_sin_is_the_promoted_rotation_rounded_once(d):
    """bf16 q / k with fp32 cos / sin (the reference's bf16=True training):
    torch promotes q * cos + rotate_half(q) * sin to fp32 and the attention
    casts the result to bf16.  siq_rope_fwd_ex writes that bf16 value, bitwise
    (checked against torch on the GPU and against fp32 torch on the CPU), and
    siq_rope_bwd_ex is the autograd of the promoted ops and the cast, bitwise."""
    b, s, hq, hkv = 2, 45, 6, 2
    print(f"rope fp32 cos/sin d={d}", flush=True)
    g = torch.Generator().manual_seed(5)
    q, k = projected(b, s, hq, d, g), projected(b, s, hkv, d, g)
    cos, sin = fp32_cos_sin(b, s, d)
    qe, ke = R.rope_fwd(q.transpose(1, 2), k.transpose(1, 2), cos, sin)
    rq, rk = torch_rope(q, k, cos, sin)
    assert rq.dtype == torch.float32
    assert same(qe.transpose(1, 2), rq.to(torch.bfloat16)) and same(ke.transpose(1, 2), rk.to(torch.bfloat16))
    cq, ck = torch_rope(q.cpu(), k.cpu(), cos.cpu(), sin.cpu())
    assert same(qe.transpose(1, 2), cq.to(torch.bfloat16)) and same(ke.transpose(1, 2), ck.to(torch.bfloat16))
    # backward through the promoted ops and the cast
    gq = torch.randn(b, hq, s, d, generator=g).to(torch.bfloat16).to(DEV)
    gk = torch.randn(b, hkv, s, d, generator=g).to(torch.bfloat16).to(DEV)
    xq, xk = q.detach().clone().requires_grad_(), k.detach().clone().requires_grad_()
    oq, ok = torch_rope(xq, xk, cos, sin)
    torch.autograd.backward([oq.to(torch.bfloat16), ok.to(torch.bfloat16)], [gq, gk])
    dq, dk = R.rope_bwd(gq.transpose(1, 2), gk.transpose(1, 2), cos, sin)
    assert same(dq.transpose(1, 2), xq.grad) and same(dk.transpose(1, 2), xk.grad)
