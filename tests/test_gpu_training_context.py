"""The drop-ins in the reference's training context, on the GPU.

The reference trains with ``gradient_checkpointing=True`` and ``bf16=True``
(scripts/train.py:712-714): ``Trainer`` runs the forward under bf16 autocast
over fp32 master weights, and every decoder layer's forward -- attention
included -- runs a second time inside the backward.  Stage 1 freezes the text
model (siq_vl/model/modeling.py:329-330), so the fused CE runs with a frozen
``lm_head`` (no dW).

Checked here, against the stock fp32 model run per sequence without
checkpointing:

* a tiny Qwen2 with ``siq_varlen`` attention, the fused CE and the fused
  RoPE attention, under ``gradient_checkpointing_enable()`` (re-entrant and
  not) and bf16 autocast, on a packed batch (cu_seq_lens kwargs or restarting
  position_ids): loss and every parameter gradient within 2e-2 (relative to
  the gradient's norm, floored at 1e-3 of the largest one: some gradients
  vanish analytically and hold only roundoff in the reference);
* the plan cache under checkpointing: the recomputed forwards reuse the
  batch's one plan;
* stages 1 and 2 on a tiny SiQ-VL-shaped model (frozen tower; text model
  frozen or trained, trainable projector; every fused operator on): the loss
  and every trained parameter's gradient within 2e-2.
"""

import numpy as np
import pytest
import torch

from siq_vl_amd import attention as A
from siq_vl_amd import rope as R
from siq_vl_amd.collator import pack_rows
from siq_vl_amd.text_model import enable_fused_cross_entropy

pytestmark = pytest.mark.gpu

transformers = pytest.importorskip("transformers")
TOL = 2e-2
DEV = "cuda"
LENGTHS = [37, 130, 1, 64, 90, 211]


def rel(x, ref) -> float:
    x = x.detach().double().cpu()
    ref = ref.detach().double().cpu()
    return float(torch.linalg.norm(x - ref) / max(float(torch.linalg.norm(ref)), 1e-30))


def grad_errors(model, ref_grads):
    gmax = max(float(g.norm()) for g in ref_grads.values())
    errs = {}
    for n, p in model.named_parameters():
        if n in ref_grads:
            assert p.grad is not None, n
            errs[n] = float((p.grad.double() - ref_grads[n].double()).norm() /
                            max(float(ref_grads[n].norm()), 1e-3 * gmax))
    return errs


def tiny_qwen(head_dim: int, attn: str, seed: int):
    cfg = transformers.Qwen2Config(vocab_size=1024, hidden_size=4 * head_dim, intermediate_size=512,
                                   num_hidden_layers=3, num_attention_heads=4, num_key_value_heads=2,
                                   max_position_embeddings=4096, use_cache=False)
    torch.manual_seed(seed)
    return transformers.Qwen2ForCausalLM._from_config(cfg, attn_implementation=attn).to(DEV).float()


def sequences(seed: int):
    g = torch.Generator().manual_seed(seed)
    seqs = [torch.randint(0, 1024, (n,), generator=g) for n in LENGTHS]
    labs = []
    for s in seqs:
        lab = s.clone()
        lab[torch.rand(s.numel(), generator=g) < 0.3] = -100
        labs.append(lab)
    return seqs, labs


def stock_per_sequence(ref, seqs, labs):
    """Stock fp32 model, eager attention, one sequence at a time: the summed
    per-sequence loss sums over the total count (what the packed batch's mean
    equals, since the separator stops the shift at each boundary)."""
    count = sum(int((lab[1:] != -100).sum()) for lab in labs)
    ref.zero_grad(set_to_none=True)
    total = 0.0
    for s, lab in zip(seqs, labs):
        out = ref(input_ids=s[None].to(DEV), labels=lab[None].to(DEV), num_items_in_batch=count)
        out.loss.backward()
        total += float(out.loss)
    return total, {n: p.grad.detach().clone() for n, p in ref.named_parameters() if p.grad is not None}


@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("route", ["cu_seq_lens", "position_ids"])
@pytest.mark.parametrize("reentrant", [True, False])
def test_checkpointed_autocast_training_step(head_dim, route, reentrant):
    print(f"training context head_dim={head_dim} route={route} reentrant={reentrant}", flush=True)
    A.register()
    ref = tiny_qwen(head_dim, "eager", seed=3)
    ours = tiny_qwen(head_dim, "siq_varlen", seed=3)
    ours.load_state_dict(ref.state_dict())
    enable_fused_cross_entropy(ours, chunk_tokens=128)
    assert R.enable_fused_rope_attention(ours) == 3
    ours.gradient_checkpointing_enable(gradient_checkpointing_kwargs={"use_reentrant": reentrant})
    ours.train()
    ref.train()
    seqs, labs = sequences(11)
    ref_loss, ref_grads = stock_per_sequence(ref, seqs, labs)

    packed = pack_rows(seqs, labs)
    batch = {"input_ids": packed["input_ids"].to(DEV), "labels": packed["labels"].to(DEV),
             "position_ids": packed["position_ids"].to(DEV)}
    if route == "cu_seq_lens":
        for key in ("cu_seq_lens_q", "cu_seq_lens_k"):
            batch[key] = packed[key].to(DEV)
        batch["max_length_q"] = packed["max_length_q"]
        batch["max_length_k"] = packed["max_length_k"]
    R.enable_fused_rope()
    try:
        with torch.autocast("cuda", dtype=torch.bfloat16):
            out = ours(**batch)
        assert out.logits is None
        out.loss.backward()
    finally:
        R.disable_fused_rope()
    torch.cuda.synchronize()
    rl = abs(float(out.loss) - ref_loss) / abs(ref_loss)
    errs = grad_errors(ours, ref_grads)
    worst = max(errs, key=errs.get)
    print(f"  loss {float(out.loss):.5f} ref {ref_loss:.5f} rel {rl:.2e}; worst grad {worst} {errs[worst]:.2e}",
          flush=True)
    assert np.isfinite(float(out.loss)) and rl <= TOL
    for n, r in errs.items():
        assert r <= TOL, (n, r)
    if route == "cu_seq_lens":
        # the three layers' forwards, their recomputation inside the backward and the backwards share one plan
        plans = getattr(batch["cu_seq_lens_q"], "_siq_attn_plans")
        assert len(plans) == 1


@pytest.mark.parametrize("stage", [1, 2])
def test_vlm_stage_training_step(stage):
    """Stage 1 (siq_vl/model/modeling.py:322-330): tower and text model frozen,
    the projector trains.  Stage 2 without LoRA (:369-370): the text model
    trains too, so the fp32 embedding table's gradient comes from the HIP
    kernel.  Every fused operator on, bf16 autocast over fp32 weights,
    checkpointing on the text model.  In stage 1 the fused CE takes the
    frozen-lm_head call (no dW) and the projector's gradient flows back through
    the decoder, the splice and the projector's own kernels."""
    from siq_vl_amd import projector, splice
    from tests.test_gpu_splice import TinyVLM, vlm_batch

    print(f"training context: stage {stage}", flush=True)
    A.register()
    torch.manual_seed(0)
    ref = TinyVLM().to(DEV).float()
    torch.manual_seed(0)
    ours = TinyVLM(attn="siq_varlen").to(DEV).float()
    ours.load_state_dict(ref.state_dict())
    for m in (ref, ours):
        for p in m.vision_model.parameters():
            p.requires_grad_(False)
        for p in m.text_model.parameters():
            p.requires_grad_(stage == 2)
    ids, pix, labels = vlm_batch()
    out_ref = ref(input_ids=ids, pixel_values=pix, labels=labels)
    out_ref.loss.backward()
    g_ref = {n: p.grad.detach().clone() for n, p in ref.named_parameters() if p.grad is not None}

    splice.enable_fused_splice(ours)
    projector.enable_fused_projector(ours)
    enable_fused_cross_entropy(ours.text_model, chunk_tokens=64)
    ours.text_model.gradient_checkpointing_enable()
    # transformers 5 also hooks the embedding output to require grad; 4.57, the reference's pin, does that only
    # under PEFT, and the stock splice's in-place assignment fails on such an output
    ours.text_model.disable_input_require_grads()
    ours.train()
    R.enable_fused_rope()
    try:
        with torch.autocast("cuda", dtype=torch.bfloat16):
            out = ours(input_ids=ids, pixel_values=pix, labels=labels)
        out.loss.backward()
    finally:
        R.disable_fused_rope()
    splice.check_pending_splices(block=True)
    torch.cuda.synchronize()
    if stage == 1:
        assert ours.text_model.lm_head.weight.grad is None
        assert set(g_ref) == {"projector.mlp.weight"}
    else:
        assert ours.text_model.model.embed_tokens.weight.grad is not None
    rl = abs(float(out.loss) - float(out_ref.loss)) / abs(float(out_ref.loss))
    errs = grad_errors(ours, g_ref)
    worst = max(errs, key=errs.get)
    print(f"  loss rel {rl:.2e}; worst grad {worst} {errs[worst]:.2e}", flush=True)
    assert rl <= TOL
    for n, r in errs.items():
        assert r <= TOL, (n, r)
