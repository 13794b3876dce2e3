"""Vision-token splice fused with the embedding gather on MI355X: host side.

Replaces, in ``SiQ_VLForCausalLM.forward`` (siq_vl/model/modeling.py:252-270),
the text-embedding lookup, the ``nonzero()`` of the ``<|image_pad|>``
positions, the count check and the index assignment of the flattened vision
rows by one ``siq_splice_fwd`` call: every output row is written once, from
the vision rows (image tokens, in row-major order) or from the embedding
table.

* ``splice_vision_tokens(input_ids, embed_weight, vision_flat,
  image_token_index, padding_idx=None, validate="lazy")`` -- the autograd op,
  for bf16 tables and for the fp32 tables of the reference's fp32 master
  weights (the kernels copy rows, whatever their element type).  It raises the
  reference's ``ValueError`` when the placeholder count differs from the
  number of vision rows, and ``IndexError`` for ids outside the table: by
  default once the device's counts have reached the host (at the next call or
  ``check_pending_splices()``), so that no call stalls the host.  Backward:
  the vision rows' gradient is a gather of the upstream gradient at the image
  positions (``siq_gather_rows``); the embedding table's gradient is
  ``siq_embedding_bwd``, a deterministic per-id sum that skips exactly the
  rows the reference's index assignment overwrote (and zeroed in its
  backward) and the padding index.
* ``fused_vlm_forward`` -- ``SiQ_VLForCausalLM.forward`` (:200-288) with the
  splice above; ``enable_fused_splice(model)`` installs it on the model.
"""

from __future__ import annotations

import types
from typing import Any

import torch

from . import _lib
from ._deferred import DeferredChecks


SUPPORTED_DTYPES = (torch.bfloat16, torch.float32)
_DTYPE_TAG = {torch.bfloat16: 0, torch.float32: 1}  # SIQ_DTYPE_BF16 / SIQ_DTYPE_FP32


def _check_ids(ids: torch.Tensor, weight: torch.Tensor, vision: torch.Tensor) -> None:
    if ids.dtype != torch.int64:
        raise ValueError(f"input_ids must be int64, got {ids.dtype}")
    for name, t in (("input_ids", ids), ("embed_weight", weight), ("vision_flat", vision)):
        if t.device.type != "cuda":
            raise ValueError(f"{name} must live on the GPU, got {t.device}")
    if weight.dtype not in SUPPORTED_DTYPES:
        raise ValueError(f"embed_weight must be bfloat16 or float32, got {weight.dtype}")
    if weight.shape[1] % 8:
        raise ValueError(f"the hidden size ({weight.shape[1]}) must be a multiple of 8")
    if vision.dim() != 2 or vision.shape[1] != weight.shape[1]:
        raise ValueError(f"vision_flat must be [n, {weight.shape[1]}], got {tuple(vision.shape)}")


def _rows16(t: torch.Tensor) -> torch.Tensor:
    """The bf16 view of a contiguous bf16 / fp32 matrix's rows: the splice and
    the row gather copy 16-byte chunks, whatever the element type."""
    return t if t.dtype == torch.bfloat16 else t.view(torch.bfloat16)


def splice_fwd(ids: torch.Tensor, weight: torch.Tensor, vision: torch.Tensor, image_token_index: int):
    """Raw forward on flat ids [n] (weight and vision of one dtype, bf16 or
    fp32); returns ``(out [n, H], image_pos [n_vision] int32, counts [2] int64)``."""
    n, (vocab, hidden) = ids.numel(), weight.shape
    nv = vision.shape[0]
    out = torch.empty(n, hidden, dtype=weight.dtype, device=ids.device)
    # one allocation for the counts, the image positions and the workspace (16-byte aligned pieces)
    ws_bytes = int(_lib.lib().siq_splice_workspace_bytes(n))
    pos_bytes = (4 * max(nv, 1) + 15) // 16 * 16
    buf = torch.empty(16 + pos_bytes + ws_bytes, dtype=torch.uint8, device=ids.device)
    counts = buf[:16].view(torch.int64)
    image_pos = buf[16:16 + pos_bytes].view(torch.int32)
    ws = buf[16 + pos_bytes:]
    stream = torch.cuda.current_stream(ids.device).cuda_stream
    w16, v16, o16 = _rows16(weight), _rows16(vision), _rows16(out)
    rc = _lib.lib().siq_splice_fwd(ids.data_ptr(), n, w16.data_ptr(), vocab, w16.shape[1],
                                   v16.data_ptr() if nv else None, nv, int(image_token_index), o16.data_ptr(),
                                   image_pos.data_ptr(), counts.data_ptr(), ws.data_ptr(), ws.numel(), stream)
    _lib.check(rc, "siq_splice_fwd")
    return out, image_pos[:nv], counts


def gather_rows(src: torch.Tensor, rows: torch.Tensor) -> torch.Tensor:
    """``src[rows]`` for contiguous bf16 / fp32 rows and int32 row indices
    (a negative index gives a zero row)."""
    n = rows.numel()
    dst = torch.empty(n, src.shape[1], dtype=src.dtype, device=src.device)
    if n:
        s16, d16 = _rows16(src), _rows16(dst)
        rc = _lib.lib().siq_gather_rows(s16.data_ptr(), rows.data_ptr(), n, s16.shape[1], d16.data_ptr(),
                                        torch.cuda.current_stream(src.device).cuda_stream)
        _lib.check(rc, "siq_gather_rows")
    return dst


def embedding_bwd(grad: torch.Tensor, ids: torch.Tensor, vocab: int, skip_ids=()) -> torch.Tensor:
    """The embedding table's gradient (``siq_embedding_bwd``): ``grad [n, H]``
    (bf16 or fp32, contiguous) summed per id of ``ids [n]`` into ``[vocab, H]``
    of the same dtype; ids in ``skip_ids`` (at most two; the image token and
    the padding index) and ids outside [0, vocab) send nothing."""
    skip = [int(x) for x in skip_ids if x is not None and int(x) >= 0]
    if len(skip) > 2:
        raise ValueError("at most two skipped ids")
    skip += [-1] * (2 - len(skip))
    n, hidden = grad.shape
    if grad.dtype not in _DTYPE_TAG:
        raise ValueError(f"grad must be bfloat16 or float32, got {grad.dtype}")
    dw = torch.empty(vocab, hidden, dtype=grad.dtype, device=grad.device)
    L = _lib.lib()
    ws = torch.empty(max(int(L.siq_embedding_bwd_workspace_bytes(n, vocab)), 16), dtype=torch.uint8,
                     device=grad.device)
    rc = L.siq_embedding_bwd(grad.data_ptr(), ids.data_ptr(), n, vocab, hidden, _DTYPE_TAG[grad.dtype], skip[0],
                             skip[1], dw.data_ptr(), ws.data_ptr(), ws.numel(),
                             torch.cuda.current_stream(grad.device).cuda_stream)
    _lib.check(rc, "siq_embedding_bwd")
    return dw


def _shape_mismatch(found: int, n_vision: int) -> ValueError:
    return ValueError(
        f"Shape Mismatch! \n"
        f"Text has {found} image placeholders.\n"
        f"Vision Encoder produced {n_vision} tokens.\n"
        f"Check Processor logic regarding 'tokens_per_tile' calculation."
    )


# The placeholder count and the out-of-range ids are counted on the device.
# validate="lazy" (the default) judges them once their copy to the host has
# landed -- at the next splice call or check_pending_splices() -- so that no
# call stalls the host (the rows the counts would condemn are written as
# zeros meanwhile, and their backward reads nothing); "sync" judges them at
# once (one device-to-host read, as the reference's nonzero() makes).
_SPLICE_CHECKS = DeferredChecks()


def _judge(vocab: int, n_vision: int):
    def judge(vals):
        found, bad = int(vals[0]), int(vals[1])
        if bad:
            raise IndexError(f"index out of range in self: {bad} input_ids outside [0, {vocab})")
        if found != n_vision:
            raise _shape_mismatch(found, n_vision)

    return judge


def check_pending_splices(block: bool = False) -> None:
    """Raises the error of an earlier lazily validated splice call whose counts
    have landed (all of them when ``block``): the reference's ValueError for a
    placeholder count that differs from the vision rows, IndexError for ids
    outside the table."""
    _SPLICE_CHECKS.check(block)


class _Splice(torch.autograd.Function):
    @staticmethod
    def forward(ctx, input_ids, weight, vision, image_token_index, padding_idx, validate):
        ids = input_ids.reshape(-1).contiguous()
        weight = weight.contiguous()
        vis = vision.to(weight.dtype).contiguous()
        _check_ids(ids, weight, vis)
        out, image_pos, counts = splice_fwd(ids, weight, vis, image_token_index)
        judge = _judge(weight.shape[0], vis.shape[0])
        if validate == "sync":
            judge(counts.tolist())
        elif validate:
            _SPLICE_CHECKS.add(counts, judge)
        ctx.save_for_backward(ids, image_pos)
        ctx.vocab = weight.shape[0]
        ctx.image_token_index = int(image_token_index)
        ctx.padding_idx = padding_idx
        ctx.vision_dtype = vision.dtype
        return out.view(*input_ids.shape, weight.shape[1])

    @staticmethod
    def backward(ctx, grad):
        ids, image_pos = ctx.saved_tensors
        g = grad.reshape(-1, grad.shape[-1]).contiguous()
        d_weight = d_vision = None
        if ctx.needs_input_grad[2]:
            d_vision = gather_rows(g, image_pos).to(ctx.vision_dtype)
        if ctx.needs_input_grad[1]:
            # the image rows were overwritten in the forward, so they send nothing to the table; neither does the
            # table's padding index
            d_weight = embedding_bwd(g, ids, ctx.vocab, (ctx.image_token_index, ctx.padding_idx))
        return None, d_weight, d_vision, None, None, None


def splice_vision_tokens(input_ids: torch.Tensor, embed_weight: torch.Tensor, vision_flat: torch.Tensor,
                         image_token_index: int, padding_idx: int | None = None, validate="lazy") -> torch.Tensor:
    """``embedding(input_ids)`` with the image-token rows replaced, in order, by
    ``vision_flat`` (cast to the table's dtype, bf16 or fp32).  ``validate``:
    "lazy" (default), "sync" or False (see ``check_pending_splices``)."""
    return _Splice.apply(input_ids, embed_weight, vision_flat, int(image_token_index), padding_idx, validate)


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
        w = embed.weight
        if w.is_cuda and w.dtype in SUPPORTED_DTYPES and w.shape[1] % 8 == 0:
            inputs_embeds = splice_vision_tokens(input_ids, w, vision_flat, self.config.image_token_index,
                                                 embed.padding_idx)
        else:  # the reference's own ops (CPU evaluation, other dtypes)
            token_embeddings = embed(input_ids)
            positions = (input_ids == self.config.image_token_index).nonzero(as_tuple=True)
            if positions[0].numel() != vision_flat.shape[0]:
                raise _shape_mismatch(positions[0].numel(), vision_flat.shape[0])
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
