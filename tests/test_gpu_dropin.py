"""End-to-end drop-in checks on a tiny random-init Qwen2 (the reference's text
model family, transformers models/qwen2/modeling_qwen2.py), on the GPU:

* ``attn_implementation="siq_varlen"`` on a packed batch (cu_seq_lens kwargs,
  restarting position_ids, or a padded batch with a 2-D mask) gives the
  logits and parameter gradients of the stock eager model run on each
  sequence separately;
* ``enable_fused_cross_entropy`` gives the stock loss and gradients (mean and
  sum / num_items_in_batch) without materialising logits, and keeps the
  logits path when no labels are given.

Reference models run in fp32 (eager attention, fp32 softmax). Tolerance:
relative Frobenius error <= 2e-2 on logits, losses and gradients.
"""

import copy

import numpy as np
import pytest
import torch

from siq_vl_amd import attention as A
from siq_vl_amd.collator import pack_rows
from siq_vl_amd.text_model import enable_fused_cross_entropy

pytestmark = pytest.mark.gpu

transformers = pytest.importorskip("transformers")
TOL = 2e-2
DEV = "cuda"
LENGTHS = [37, 130, 1, 64, 90]


def rel(x, ref) -> float:
    x = x.detach().double().cpu()
    ref = ref.detach().double().cpu()
    return float(torch.linalg.norm(x - ref) / max(float(torch.linalg.norm(ref)), 1e-30))


def tiny_config(head_dim: int):
    heads = 4
    return transformers.Qwen2Config(vocab_size=1024, hidden_size=heads * head_dim, intermediate_size=512,
                                    num_hidden_layers=2, num_attention_heads=heads, num_key_value_heads=2,
                                    max_position_embeddings=4096, use_cache=False)


def model_pair(head_dim: int, seed: int = 0):
    A.register()
    cfg = tiny_config(head_dim)
    torch.manual_seed(seed)
    ref = transformers.Qwen2ForCausalLM._from_config(cfg, attn_implementation="eager").to(DEV).float()
    ours = transformers.Qwen2ForCausalLM._from_config(cfg, attn_implementation="siq_varlen").to(DEV).float()
    ours.load_state_dict(ref.state_dict())
    return ref, ours


def rows(seed: int = 1):
    g = torch.Generator().manual_seed(seed)
    return [torch.randint(0, 1024, (n,), generator=g) for n in LENGTHS]


def per_sequence_reference(ref, seqs, probe):
    """Logits of each sequence on its own, concatenated, and the grads of <logits, probe>."""
    ref.zero_grad(set_to_none=True)
    outs = [ref(input_ids=s[None].to(DEV)).logits[0] for s in seqs]
    logits = torch.cat(outs)
    (logits * probe).sum().backward()
    return logits.detach(), {n: p.grad.detach().clone() for n, p in ref.named_parameters() if p.grad is not None}


def check_grads(model, ref_grads):
    worst = 0.0
    for n, p in model.named_parameters():
        if n in ref_grads:
            assert p.grad is not None, n
            r = rel(p.grad, ref_grads[n])
            worst = max(worst, r)
            assert r <= TOL, (n, r)
    return worst


@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("route", ["cu_seq_lens", "position_ids"])
def test_siq_varlen_packed_matches_per_sequence_eager(head_dim, route):
    print(f"dropin attention head_dim={head_dim} route={route}", flush=True)
    ref, ours = model_pair(head_dim)
    seqs = rows()
    packed = pack_rows(seqs)
    total = sum(LENGTHS)
    probe = torch.randn(total, 1024, generator=torch.Generator().manual_seed(3)).to(DEV)
    ref_logits, ref_grads = per_sequence_reference(ref, seqs, probe)

    kwargs = {"input_ids": packed["input_ids"].to(DEV), "position_ids": packed["position_ids"].to(DEV)}
    if route == "cu_seq_lens":
        for key in ("cu_seq_lens_q", "cu_seq_lens_k"):
            kwargs[key] = packed[key].to(DEV)
        kwargs["max_length_q"] = packed["max_length_q"]
        kwargs["max_length_k"] = packed["max_length_k"]
    kwargs["questions"] = ["ignored raw-data kwarg"]  # the reference collator's extra keys
    logits = ours(**kwargs).logits[0]
    assert rel(logits, ref_logits) <= TOL
    (logits * probe).sum().backward()
    check_grads(ours, ref_grads)


def test_siq_varlen_padded_batch_with_mask():
    print("dropin attention padded+mask", flush=True)
    ref, ours = model_pair(64)
    seqs = rows(2)
    seq = max(LENGTHS)
    ids = torch.zeros(len(seqs), seq, dtype=torch.int64)
    mask = torch.zeros(len(seqs), seq, dtype=torch.int64)
    for i, s in enumerate(seqs):
        ids[i, :s.numel()] = s
        mask[i, :s.numel()] = 1
    probe = torch.randn(sum(LENGTHS), 1024, generator=torch.Generator().manual_seed(4)).to(DEV)
    ref_logits, ref_grads = per_sequence_reference(ref, seqs, probe)
    out = ours(input_ids=ids.to(DEV), attention_mask=mask.to(DEV)).logits
    keep = mask.reshape(-1).bool().to(DEV)
    logits = out.reshape(-1, out.shape[-1])[keep]
    assert rel(logits, ref_logits) <= TOL
    (logits * probe).sum().backward()
    check_grads(ours, ref_grads)


def _labels_for(seqs, seed=5):
    g = torch.Generator().manual_seed(seed)
    labs = []
    for s in seqs:
        lab = s.clone()
        lab[torch.rand(s.numel(), generator=g) < 0.3] = -100
        labs.append(lab)
    return labs


@pytest.mark.parametrize("use_num_items", [False, True])
def test_fused_cross_entropy_matches_stock_loss(use_num_items):
    print(f"dropin fused CE num_items={use_num_items}", flush=True)
    ref, _ = model_pair(64)
    fused = copy.deepcopy(ref)
    enable_fused_cross_entropy(fused, chunk_tokens=128)
    g = torch.Generator().manual_seed(6)
    ids = torch.randint(0, 1024, (3, 96), generator=g).to(DEV)
    labels = ids.clone()
    labels[torch.rand(3, 96, generator=g).to(DEV) < 0.3] = -100
    extra = {}
    if use_num_items:
        extra["num_items_in_batch"] = torch.tensor(200, device=DEV)
    ref.zero_grad(set_to_none=True)
    out_ref = ref(input_ids=ids, labels=labels, **extra)
    out_ref.loss.backward()
    out = fused(input_ids=ids, labels=labels, **extra)
    assert out.logits is None
    assert rel(out.loss, out_ref.loss) <= TOL, (float(out.loss), float(out_ref.loss))
    out.loss.backward()
    ref_grads = {n: p.grad for n, p in ref.named_parameters() if p.grad is not None}
    check_grads(fused, ref_grads)
    # no labels: the logits path is untouched
    with torch.no_grad():
        assert torch.equal(fused(input_ids=ids).logits, ref(input_ids=ids).logits)


def test_packed_training_step_end_to_end():
    """Collator -> siq_varlen attention -> fused CE: the loss and grads of the
    stock model run per sequence (same targets: the separator stops the shift
    at each boundary)."""
    print("dropin packed training step", flush=True)
    ref, ours = model_pair(64, seed=11)
    enable_fused_cross_entropy(ours, chunk_tokens=64)
    seqs = rows(7)
    labs = _labels_for(seqs)
    packed = pack_rows(seqs, labs)
    # reference: per-sequence stock losses summed, divided by the total count
    count = sum(int((lab[1:] != -100).sum()) for lab in labs)
    ref.zero_grad(set_to_none=True)
    total = 0.0
    for s, lab in zip(seqs, labs):
        out = ref(input_ids=s[None].to(DEV), labels=lab[None].to(DEV), num_items_in_batch=count)
        out.loss.backward()
        total += float(out.loss)
    batch = {k: (v.to(DEV) if torch.is_tensor(v) else v) for k, v in packed.items()}
    out = ours(**batch)
    # ours is the mean over valid targets, which equals the summed per-sequence sums / count
    assert np.isfinite(float(out.loss))
    assert abs(float(out.loss) - total) <= TOL * abs(total), (float(out.loss), total)
    out.loss.backward()
    check_grads(ours, {n: p.grad for n, p in ref.named_parameters() if p.grad is not None})
