"""Vision-token splice fused with the embedding gather on MI355X: host side.

Replaces, in ``SiQ_VLForCausalLM.forward`` (siq_vl/model/modeling.py:252-270),
the text-embedding lookup, the ``nonzero()`` of the ``<|image_pad|>``
positions, the count check and the index assignment of the flattened vision
rows by one ``siq_splice_fwd`` call: every output row is written once, from
the vision rows (image tokens, in row-major order) or from the embedding
table.

* ``splice_vision_tokens(input_ids, embed_weight, vision_flat,
  image_token_index, padding_idx=None)`` -- the autograd op.  It raises the
  reference's ``ValueError`` when the placeholder count differs from the
  number of vision rows (reading one device scalar, as the reference's
  ``nonzero()`` does).  Backward: the vision rows' gradient is a gather of the
  upstream gradient at the image positions (``siq_gather_rows``); the
  embedding table's gradient is torch's own embedding backward with the image
  token as padding index, which skips exactly the rows the reference's index
  assignment overwrote (and zeroed in its backward).
* ``fused_vlm_forward`` -- ``SiQ_VLForCausalLM.forward`` (:200-288) with the
  splice above; ``enable_fused_splice(model)`` installs it on the model.
"""

from __future__ import annotations

import types
from typing import Any

import torch

from . import _lib


def _check_ids(ids: torch.Tensor, weight: torch.Tensor, vision: torch.Tensor) -> None:
    if ids.dtype != torch.int64:
        raise ValueError(f"input_ids must be int64, got {ids.dtype}")
    for name, t in (("input_ids", ids), ("embed_weight", weight), ("vision_flat", vision)):
        if t.device.type != "cuda":
            raise ValueError(f"{name} must live on the GPU, got {t.device}")
    if weight.dtype != torch.bfloat16:
        raise ValueError(f"embed_weight must be bfloat16, got {weight.dtype}")
    if vision.dim() != 2 or vision.shape[1] != weight.shape[1]:
        raise ValueError(f"vision_flat must be [n, {weight.shape[1]}], got {tuple(vision.shape)}")


def splice_fwd(ids: torch.Tensor, weight: torch.Tensor, vision: torch.Tensor, image_token_index: int):
    """Raw forward on flat ids [n]; returns ``(out [n, H], image_pos [n_vision] int32, counts [2] int64)``."""
    n, (vocab, hidden) = ids.numel(), weight.shape
    nv = vision.shape[0]
    out = torch.empty(n, hidden, dtype=torch.bfloat16, device=ids.device)
    image_pos = torch.empty(max(nv, 1), dtype=torch.int32, device=ids.device)
    counts = torch.empty(2, dtype=torch.int64, device=ids.device)
    ws = torch.empty(int(_lib.lib().siq_splice_workspace_bytes(n)), dtype=torch.uint8, device=ids.device)
    stream = torch.cuda.current_stream(ids.device).cuda_stream
    rc = _lib.lib().siq_splice_fwd(ids.data_ptr(), n, weight.data_ptr(), vocab, hidden,
                                   vision.data_ptr() if nv else None, nv, int(image_token_index), out.data_ptr(),
                                   image_pos.data_ptr(), counts.data_ptr(), ws.data_ptr(), ws.numel(), stream)
    _lib.check(rc, "siq_splice_fwd")
    return out, image_pos[:nv], counts


def gather_rows(src: torch.Tensor, rows: torch.Tensor) -> torch.Tensor:
    """``src[rows]`` for bf16 rows and int32 row indices."""
    n, hidden = rows.numel(), src.shape[1]
    dst = torch.empty(n, hidden, dtype=src.dtype, device=src.device)
    if n:
        rc = _lib.lib().siq_gather_rows(src.data_ptr(), rows.data_ptr(), n, hidden, dst.data_ptr(),
                                        torch.cuda.current_stream(src.device).cuda_stream)
        _lib.check(rc, "siq_gather_rows")
    return dst


class _Splice(torch.autograd.Function):
    @staticmethod
    def forward(ctx, input_ids, weight, vision, image_token_index, padding_idx):
        ids = input_ids.reshape(-1).contiguous()
        vis = vision.to(weight.dtype).contiguous()
        _check_ids(ids, weight, vis)
        out, image_pos, counts = splice_fwd(ids, weight.contiguous(), vis, image_token_index)
        found, bad = (int(c) for c in counts.tolist())
        if bad:
            raise IndexError(f"index out of range in self: {bad} input_ids outside [0, {weight.shape[0]})")
        if found != vis.shape[0]:
            raise ValueError(
                f"Shape Mismatch! \n"
                f"Text has {found} image placeholders.\n"
                f"Vision Encoder produced {vis.shape[0]} tokens.\n"
                f"Check Processor logic regarding 'tokens_per_tile' calculation."
            )
        ctx.save_for_backward(ids, image_pos)
        ctx.vocab = weight.shape[0]
        ctx.image_token_index = int(image_token_index)
        ctx.padding_idx = padding_idx
        ctx.vision_dtype = vision.dtype
        return out.view(*input_ids.shape, weight.shape[1])

    @staticmethod
    def backward(ctx, grad):
        ids, image_pos = ctx.saved_tensors
        g = grad.reshape(-1, grad.shape[-1]).to(torch.bfloat16).contiguous()
        d_weight = d_vision = None
        if ctx.needs_input_grad[2]:
            d_vision = gather_rows(g, image_pos).to(ctx.vision_dtype)
        if ctx.needs_input_grad[1]:
            # the image rows were overwritten in the forward, so they send nothing to the table: the image token as
            # padding index skips them (and the model's own padding index, if any, is folded into it)
            skip = ctx.image_token_index
            idx = ids
            if ctx.padding_idx is not None and ctx.padding_idx >= 0:
                idx = torch.where(ids == ctx.padding_idx, torch.full_like(ids, skip), ids)
            d_weight = torch.ops.aten.embedding_dense_backward(g, idx, ctx.vocab, skip, False)
        return None, d_weight, d_vision, None, None


def splice_vision_tokens(input_ids: torch.Tensor, embed_weight: torch.Tensor, vision_flat: torch.Tensor,
                         image_token_index: int, padding_idx: int | None = None) -> torch.Tensor:
    """``embedding(input_ids)`` with the image-token rows replaced, in order, by ``vision_flat``."""
    return _Splice.apply(input_ids, embed_weight, vision_flat, int(image_token_index), padding_idx)


def fused_vlm_forward(self, input_ids=None, pixel_values=None, num_image_tokens=None, attention_mask=None,
                      position_ids=None, past_key_values=None, inputs_embeds=None, labels=None, use_cache=None,
                      cache_position=None, logits_to_keep=0, **kwargs: Any):
    """``SiQ_VLForCausalLM.forward`` (modeling.py:200-288) with the fused splice."""
    del num_image_tokens, logits_to_keep
    if past_key_values is None and pixel_values is not None:
        vision_features = self.vision_model(pixel_values).last_hidden_state
        vision_token_embeddings = self.projector(vision_features)
        vision_flat = vision_token_embeddings.view(-1, vision_token_embeddings.size(-1))
        embed = self.text_model.get_input_embeddings()
        if embed.weight.dtype == torch.bfloat16 and embed.weight.is_cuda:
            inputs_embeds = splice_vision_tokens(input_ids, embed.weight, vision_flat, self.config.image_token_index,
                                                 embed.padding_idx)
        else:  # the reference's own ops (fp32 / CPU evaluation)
            token_embeddings = embed(input_ids)
            positions = (input_ids == self.config.image_token_index).nonzero(as_tuple=True)
            if positions[0].numel() != vision_flat.shape[0]:
                raise ValueError(
                    f"Shape Mismatch! \n"
                    f"Text has {positions[0].numel()} image placeholders.\n"
                    f"Vision Encoder produced {vision_flat.shape[0]} tokens.\n"
                    f"Check Processor logic regarding 'tokens_per_tile' calculation."
                )
            token_embeddings[positions] = vision_flat.to(dtype=token_embeddings.dtype)
            inputs_embeds = token_embeddings
        input_ids = None
    return self.text_model(input_ids=input_ids, attention_mask=attention_mask, position_ids=position_ids,
                           past_key_values=past_key_values, inputs_embeds=inputs_embeds, labels=labels,
                           use_cache=use_cache, cache_position=cache_position, **kwargs)


def enable_fused_splice(model: torch.nn.Module) -> torch.nn.Module:
    """Installs ``fused_vlm_forward`` on a SiQ-VL model (``vision_model``, ``projector``,
    ``text_model`` and ``config.image_token_index``)."""
    for attr in ("vision_model", "projector", "text_model"):
        if not hasattr(model, attr):
            raise ValueError(f"not a SiQ-VL model: no '{attr}'")
    if not hasattr(model.config, "image_token_index"):
        raise ValueError("not a SiQ-VL model: config has no image_token_index")
    model.forward = types.MethodType(fused_vlm_forward, model)
    return model


def splice_bytes(n_tokens: int, hidden: int) -> int:
    """Algorithmic HBM bytes of the forward: one row read and one written per token, plus the ids."""
    return n_tokens * (2 * hidden * 2 + 8)
