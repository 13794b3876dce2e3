"""Fused lm_head cross-entropy for SiQ-VL's text model.

``model.loss_function`` (transformers modeling_utils.py:4654-4672) only ever
sees materialised logits, so the fused loss has to replace the forward of the
causal-LM head itself.  ``fused_causal_lm_forward`` has exactly the signature
of ``Qwen2ForCausalLM.forward`` (transformers models/qwen2/modeling_qwen2.py:
423-477), which the reference's ``SiQ_VLTextModel`` inherits
(siq_vl/model/modeling.py:139-153):

* with ``labels``: the decoder runs as usual, then the last hidden states go
  straight into ``fused_linear_cross_entropy`` with the labels shifted as
  ``ForCausalLMLoss`` shifts them (loss/loss_utils.py:63-64, or the given
  ``shift_labels``) and ``num_items_in_batch`` honoured; ``logits`` is None;
* without ``labels`` (``generate``): the original logits path;
* with ``labels`` but no gradient (evaluation under ``torch.no_grad``): the
  loss-only kernel, no logits and no gradient work.

``enable_fused_cross_entropy(model)`` installs it on a model instance (the
``SiQ_VLTextModel`` inside ``SiQ_VLForCausalLM``, or any Qwen2-style causal LM).
"""

from __future__ import annotations

import types
from typing import Any

import torch

from .cross_entropy import IGNORE_INDEX, fused_linear_cross_entropy, shift_labels


def fused_causal_lm_forward(self, input_ids=None, attention_mask=None, position_ids=None, past_key_values=None,
                            inputs_embeds=None, labels=None, use_cache=None, logits_to_keep=0, **kwargs: Any):
    from transformers.modeling_outputs import CausalLMOutputWithPast

    outputs = self.model(
        input_ids=input_ids,
        attention_mask=attention_mask,
        position_ids=position_ids,
        past_key_values=past_key_values,
        inputs_embeds=inputs_embeds,
        use_cache=use_cache,
        **kwargs,
    )
    # the same positions the stock forward turns into logits (all of them for logits_to_keep=0)
    slice_indices = slice(-logits_to_keep, None) if isinstance(logits_to_keep, int) else logits_to_keep
    hidden = outputs.last_hidden_state[:, slice_indices, :]
    if labels is None:
        logits = self.lm_head(hidden)
        return CausalLMOutputWithPast(loss=None, logits=logits, past_key_values=outputs.past_key_values,
                                      hidden_states=outputs.hidden_states, attentions=outputs.attentions)
    targets = kwargs.get("shift_labels")
    if targets is None:
        targets = shift_labels(labels, IGNORE_INDEX)
    loss = fused_linear_cross_entropy(
        hidden.reshape(-1, hidden.shape[-1]),
        self.lm_head.weight,
        targets.reshape(-1).to(hidden.device),
        ignore_index=IGNORE_INDEX,
        num_items_in_batch=kwargs.get("num_items_in_batch"),
        chunk_tokens=getattr(self, "siq_ce_chunk_tokens", None),
    )
    return CausalLMOutputWithPast(loss=loss, logits=None, past_key_values=outputs.past_key_values,
                                  hidden_states=outputs.hidden_states, attentions=outputs.attentions)


def enable_fused_cross_entropy(model: torch.nn.Module, chunk_tokens: int | None = None) -> torch.nn.Module:
    """Routes ``model``'s loss through the fused kernel (in place); returns the
    module whose forward was replaced.  For ``SiQ_VLForCausalLM`` the text
    model (``model.text_model``) is patched, and when that is a PEFT wrapper
    (``get_base_model()``), the causal LM inside it.  ``chunk_tokens`` None
    keeps the default bound on the logits chunk."""
    target = getattr(model, "text_model", model)
    # The reference's stage 2 with LoRA replaces text_model by a PEFT wrapper
    # (siq_vl/model/modeling.py:388).  The wrapper's forward ends in the
    # wrapped model's own ``forward`` attribute, so that model is patched.
    get_base_model = getattr(target, "get_base_model", None)
    if callable(get_base_model):
        target = get_base_model()
    if not hasattr(target, "lm_head") or not hasattr(target, "model"):
        raise TypeError("expected a causal LM with .model (decoder) and .lm_head")
    target.siq_ce_chunk_tokens = None if chunk_tokens is None else int(chunk_tokens)
    target.forward = types.MethodType(fused_causal_lm_forward, target)
    return target


__all__ = ["enable_fused_cross_entropy", "fused_causal_lm_forward"]
