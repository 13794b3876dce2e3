"""Host-side logic of the Python mirror (CPU): argument checks, feature
rejection, cu_seqlens handling, FLOP counts and the seeded workloads."""

import math

import pytest
import torch

from siq_vl_amd import attention, cross_entropy, workloads


def test_validate_cu_seqlens_accepts_good_offsets():
    attention.validate_cu_seqlens(torch.tensor([0, 3, 3, 10], dtype=torch.int32), 10)
    attention.validate_cu_seqlens(torch.tensor([0], dtype=torch.int32), 0)


@pytest.mark.parametrize("cu,total,msg", [
    (torch.tensor([0, 3, 10], dtype=torch.int64), 10, "int32"),
    (torch.tensor([[0, 3]], dtype=torch.int32), 3, "1-D"),
    (torch.tensor([1, 3, 10], dtype=torch.int32), 10, r"\[0\]"),
    (torch.tensor([0, 5, 3, 10], dtype=torch.int32), 10, "non-decreasing"),
    (torch.tensor([0, 3, 9], dtype=torch.int32), 10, "must equal"),
])
def test_validate_cu_seqlens_rejects(cu, total, msg):
    with pytest.raises(ValueError, match=msg):
        attention.validate_cu_seqlens(cu, total)


def test_cpu_tensors_are_rejected_not_computed():
    q = torch.zeros(8, 2, 64, dtype=torch.bfloat16)
    cu = torch.tensor([0, 8], dtype=torch.int32)
    with pytest.raises(ValueError, match="GPU"):
        attention.varlen_attn_fwd(q, q[:, :1], q[:, :1], cu, cu, 8, 8, 0.125, True)
    with pytest.raises(ValueError, match="bfloat16"):
        attention.varlen_attn_fwd(q.float(), q, q, cu, cu, 8, 8, 0.125, True)
    with pytest.raises(ValueError, match="GPU"):
        cross_entropy.flce_fwd_bwd(torch.zeros(4, 64, dtype=torch.bfloat16), torch.zeros(8, 64, dtype=torch.bfloat16),
                                   torch.zeros(4, dtype=torch.int64))


@pytest.mark.parametrize("kw,msg", [
    (dict(dropout_p=0.1), "dropout"),
    (dict(window_size=(16, 0)), "sliding"),
    (dict(softcap=30.0), "softcap"),
    (dict(alibi_slopes=torch.ones(2)), "ALiBi"),
    (dict(return_attn_probs=True), "probabilities"),
])
def test_flash_attn_varlen_func_rejects_unsupported_features(kw, msg):
    q = torch.zeros(4, 2, 64, dtype=torch.bfloat16)
    cu = torch.tensor([0, 4], dtype=torch.int32)
    with pytest.raises(ValueError, match=msg):
        attention.flash_attn_varlen_func(q, q, q, cu, cu, 4, 4, **kw)


def test_attention_interface_rejects_dropout_and_window():
    q = torch.zeros(1, 2, 4, 64, dtype=torch.bfloat16)
    mod = torch.nn.Module()
    with pytest.raises(ValueError, match="dropout"):
        attention.siq_varlen_attention_forward(mod, q, q, q, None, dropout=0.1)
    with pytest.raises(ValueError, match="sliding"):
        attention.siq_varlen_attention_forward(mod, q, q, q, None, sliding_window=128)


def test_cu_from_position_ids():
    pos = torch.tensor([[0, 1, 2, 0, 1, 0, 1, 2, 3]])
    cu, mx = attention._cu_from_position_ids(pos)
    assert cu.tolist() == [0, 3, 5, 9] and cu.dtype == torch.int32 and mx == 4


def test_register_adds_backend():
    transformers = pytest.importorskip("transformers")
    name = attention.register()
    assert name in transformers.AttentionInterface._global_mapping
    from transformers.masking_utils import ALL_MASK_ATTENTION_FUNCTIONS

    assert name in ALL_MASK_ATTENTION_FUNCTIONS._global_mapping


def test_attention_flops_closed_form():
    cu = torch.tensor([0, 3, 7], dtype=torch.int32)
    # causal pairs 6 + 10 = 16; bidirectional 9 + 16 = 25
    assert attention.attention_flops(cu, 12, 128, True) == 12 * 128 * 16 * 12
    assert attention.attention_flops(cu, 12, 128, False, backward=False) == 4 * 128 * 25 * 12
    assert cross_entropy.ce_flops(16384, 1536, 151936) == pytest.approx(2.294e13, rel=1e-3)


def test_shift_labels_pads_with_ignore():
    lab = torch.tensor([[5, 6, 7]])
    assert cross_entropy.shift_labels(lab).tolist() == [[6, 7, -100]]


@pytest.mark.parametrize("idx,total,nseq,maxlen", [(1, 4096, 8, None), (2, 16384, 32, None), (3, 16384, 16, 1024),
                                                   (5, 32768, None, 16384)])
def test_workload_configs(idx, total, nseq, maxlen):
    cfg = workloads.attn_config(idx)
    lens = cfg.lengths
    assert sum(lens) == total == cfg.total
    assert all(n >= 1 for n in lens)
    if nseq is not None:
        assert len(lens) == nseq
    if maxlen is not None:
        assert max(lens) == maxlen
    cu = cfg.cu_seqlens()
    assert cu.dtype == torch.int32 and cu[0] == 0 and int(cu[-1]) == total
    assert workloads.attn_config(idx).lengths == lens  # seeded, reproducible


def test_config2_and_5_shapes():
    c2 = workloads.attn_config(2)
    assert all(16 <= n <= 4096 for n in c2.lengths)
    c5 = workloads.attn_config(5)
    assert c5.lengths[0] == 16384 and c5.lengths[1] == 8192
    assert all(81 <= n <= 600 for n in c5.lengths[2:-1])


def test_span_masked_labels_fraction_and_range():
    g = torch.Generator().manual_seed(0)
    lab = workloads.span_masked_labels(16384, 151936, 0.3, g)
    masked = (lab == -100).float().mean().item()
    assert abs(masked - 0.3) < 0.05
    valid = lab[lab != -100]
    assert valid.min() >= 0 and valid.max() < 151936
    assert math.isclose(workloads.CONFIG4.flops(), 6.0 * 16384 * 1536 * 151936)


def test_plan_describes_only_its_own_offsets():
    """The host check behind an explicit ``plan=``: a plan accepts its own
    offset copies, the unchanged tensors it was built from and equal values,
    and refuses other offsets with the same totals and sequence count, or its
    source tensor after an in-place change (CPU tensors stand in for the
    device copies; the comparison is the same)."""
    import weakref

    src = torch.tensor([0, 100, 400, 600], dtype=torch.int32)
    own = src.clone()
    plan = attention.AttnPlan(None, 3, 600, 600, 12, 2, True, own, own,
                              ((weakref.ref(src), src._version), (weakref.ref(src), src._version)))
    assert plan.describes(own, own)
    assert plan.describes(src, src)
    assert plan.describes(src.clone(), torch.tensor([0, 100, 400, 600], dtype=torch.int64))
    assert not plan.describes(torch.tensor([0, 300, 400, 600], dtype=torch.int32), own)
    assert not plan.describes(own, torch.tensor([0, 600], dtype=torch.int32))
    src[1] = 300
    assert not plan.describes(src, src)
    src[1] = 100  # same values again (a newer version): compared, and accepted
    assert plan.describes(src, src)


def test_fused_ce_patches_the_model_inside_a_peft_wrapper():
    """Stage 2 with LoRA wraps the text model (siq_vl/model/modeling.py:388);
    PEFT's wrapper forwards to the wrapped model's ``forward`` attribute, which
    is what gets patched.  peft is not installed here: a stand-in with PEFT's
    ``get_base_model()`` and forwarding shape plays the wrapper."""
    transformers = pytest.importorskip("transformers")
    from siq_vl_amd.text_model import enable_fused_cross_entropy, fused_causal_lm_forward

    cfg = transformers.Qwen2Config(vocab_size=64, hidden_size=32, intermediate_size=64, num_hidden_layers=1,
                                   num_attention_heads=2, num_key_value_heads=1, use_cache=False)
    inner = transformers.Qwen2ForCausalLM(cfg)

    class Wrapper(torch.nn.Module):
        def __init__(self, m):
            super().__init__()
            self.base_model = torch.nn.Module()
            self.base_model.model = m

        def get_base_model(self):
            return self.base_model.model

        def forward(self, *args, **kwargs):
            return self.base_model.model.forward(*args, **kwargs)

    class VLM(torch.nn.Module):
        def __init__(self, m):
            super().__init__()
            self.text_model = Wrapper(m)

    vlm = VLM(inner)
    patched = enable_fused_cross_entropy(vlm, chunk_tokens=256)
    assert patched is inner
    assert inner.forward.__func__ is fused_causal_lm_forward
    # no labels: the logits path, reached through the wrapper
    out = vlm.text_model(input_ids=torch.randint(0, 64, (1, 5)))
    assert out.logits.shape == (1, 5, 64)
