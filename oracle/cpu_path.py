"""The reference path's CPU arithmetic, restated with the same library calls
(test infrastructure and timed CPU baseline only; see package header).

The reference never packs: its collator pads (siq_vl/collator.py:28-34) and
transformers' ``sdpa_attention_forward`` (integrations/sdpa_attention.py:
79-166) expands K/V to all q heads with ``repeat_kv`` (:15-24, :97-102) when a
mask is present and calls ``F.scaled_dot_product_attention`` with the boolean
mask (:154-163).  Packed into one row, the mask is block-diagonal (causal
within each block), as ``create_causal_mask`` builds from packed position ids
(masking_utils.py:728-757).  The loss is ``F.linear`` -> ``.float()`` ->
``F.cross_entropy(ignore_index=-100)`` (loss/loss_utils.py:32-71).  All in
fp32 with autograd for the backward.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def block_diagonal_mask(cu_seqlens: list[int], causal: bool) -> torch.Tensor:
    """Boolean [T, T]: True where query i may attend key j (same sequence, and
    j <= i when causal)."""
    total = cu_seqlens[-1]
    seq = torch.empty(total, dtype=torch.int64)
    for b in range(len(cu_seqlens) - 1):
        seq[cu_seqlens[b]:cu_seqlens[b + 1]] = b
    mask = seq[:, None] == seq[None, :]
    if causal:
        mask &= torch.ones(total, total, dtype=torch.bool).tril()
    return mask


def repeat_kv(x: torch.Tensor, n_rep: int) -> torch.Tensor:
    """[B, Hkv, S, D] -> [B, Hkv * n_rep, S, D] (transformers modeling_qwen2.py:138-147)."""
    if n_rep == 1:
        return x
    b, h, s, d = x.shape
    return x[:, :, None].expand(b, h, n_rep, s, d).reshape(b, h * n_rep, s, d)


def sdpa_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cu_seqlens: list[int], scale: float,
                   causal: bool) -> torch.Tensor:
    """q [T, Hq, D], k/v [T, Hkv, D] (fp32, CPU) -> out [T, Hq, D] via SDPA with
    a block-diagonal boolean mask, one packed row, as the reference computes it."""
    hq, hkv = q.shape[1], k.shape[1]
    qb = q.transpose(0, 1)[None]
    kb = repeat_kv(k.transpose(0, 1)[None], hq // hkv)
    vb = repeat_kv(v.transpose(0, 1)[None], hq // hkv)
    mask = block_diagonal_mask(cu_seqlens, causal)
    out = F.scaled_dot_product_attention(qb, kb, vb, attn_mask=mask, dropout_p=0.0, scale=scale)
    return out[0].transpose(0, 1).contiguous()


def cross_entropy(hidden: torch.Tensor, weight: torch.Tensor, labels: torch.Tensor, ignore_index: int = -100,
                  num_items_in_batch=None) -> torch.Tensor:
    logits = F.linear(hidden, weight).float()
    if num_items_in_batch is None:
        return F.cross_entropy(logits, labels, ignore_index=ignore_index, reduction="mean")
    return F.cross_entropy(logits, labels, ignore_index=ignore_index, reduction="sum") / num_items_in_batch
