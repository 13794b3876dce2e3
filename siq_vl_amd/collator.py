"""Packing collator and label masking for the varlen hot path.

The reference collator (siq_vl/collator.py:11-45) pads every batch to its
longest row and the processor masks labels (siq_vl/model/processing.py:
450-479).  ``SiQ_VLPackingCollator`` keeps the reference's
``__call__(features) -> dict`` signature and processor call, then flattens the
padded rows into one packed row the way transformers' packing contract does
(DataCollatorWithFlattening, data/data_collator.py:1424-1500):

* ``input_ids`` / ``labels`` / ``position_ids``: ``[1, T]`` int64, rows
  concatenated without padding, positions restarting at 0 per row;
* each row's first label becomes the separator (-100), so the causal-LM left
  shift never predicts across a row boundary;
* ``cu_seq_lens_q == cu_seq_lens_k``: int32 ``[B + 1]`` offsets, and
  ``max_length_q == max_length_k`` as Python ints (no device sync later);
* everything else the processor returned (``pixel_values``,
  ``num_image_tokens``) passes through; ``attention_mask`` is dropped (a
  packed row has no padding).

These are the kwargs the ``siq_varlen`` attention backend reads.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any

import torch

IGNORE_INDEX = -100
# Qwen2 tokenizer ids used by the reference (siq_vl/model/configuration.py:129,
# README.md:184); parameters everywhere below, never hard-wired.
QWEN_IM_START = 151644
QWEN_IM_END = 151645
QWEN_IMAGE_PAD = 151655


def assistant_label_mask(input_ids: torch.Tensor, im_start_id: int, assistant_id: int, im_end_id: int,
                         image_pad_id: int, has_answer: list[bool] | None = None,
                         ignore_index: int = IGNORE_INDEX) -> torch.Tensor:
    """Labels of a padded ``[B, S]`` batch, exactly as the reference's processor
    builds them (siq_vl/model/processing.py:450-479): everything ``ignore_index``
    except the first assistant turn, which starts 3 tokens after
    ``<|im_start|> assistant`` and ends before the next ``<|im_end|>`` (or at
    the row end); image-pad tokens are never labels; rows without an answer
    stay fully masked."""
    if input_ids.dim() != 2:
        raise ValueError("input_ids must be [batch, seq]")
    bsz, seq = input_ids.shape
    labels = torch.full_like(input_ids, ignore_index)
    if has_answer is None:
        has_answer = [True] * bsz
    pos = torch.arange(seq, device=input_ids.device)
    for i in range(bsz):
        if not has_answer[i]:
            continue
        row = input_ids[i]
        hit = (row[:-1] == im_start_id) & (row[1:] == assistant_id)
        idx = torch.nonzero(hit, as_tuple=False)
        if idx.numel():
            start = int(idx[0, 0]) + 3
            ends = torch.nonzero((row == im_end_id) & (pos >= start), as_tuple=False)
            end = int(ends[0, 0]) if ends.numel() else seq
            if end > start:
                labels[i, start:end] = row[start:end]
        labels[i, row == image_pad_id] = ignore_index
    return labels


def pack_rows(rows: list[torch.Tensor], labels: list[torch.Tensor] | None = None,
              separator: int = IGNORE_INDEX) -> dict[str, Any]:
    """Flattens token rows (1-D int tensors, no padding) into one packed row
    with the DataCollatorWithFlattening contract."""
    if not rows:
        raise ValueError("pack_rows needs at least one row")
    ids = torch.cat([r.reshape(-1).to(torch.int64) for r in rows])
    lens = [int(r.numel()) for r in rows]
    lab_rows = []
    for i, r in enumerate(rows):
        src = (labels[i] if labels is not None else r).reshape(-1).to(torch.int64)
        if src.numel() != r.numel():
            raise ValueError(f"row {i}: labels and input_ids lengths differ")
        lab = src.clone()
        if lab.numel():
            lab[0] = separator
        lab_rows.append(lab)
    lab = torch.cat(lab_rows)
    pos = torch.cat([torch.arange(n, dtype=torch.int64) for n in lens])
    cu = torch.zeros(len(rows) + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.tensor(lens, dtype=torch.int64), 0).to(torch.int32)
    max_len = max(lens)
    return {
        "input_ids": ids[None],
        "labels": lab[None],
        "position_ids": pos[None],
        "cu_seq_lens_q": cu,
        "cu_seq_lens_k": cu.clone(),
        "max_length_q": max_len,
        "max_length_k": max_len,
    }


@dataclass
class SiQ_VLPackingCollator:
    """Drop-in sibling of ``SiQ_VLDataCollator`` (siq_vl/collator.py:6-45) that
    emits packed (cu_seqlens) batches."""

    processor: Any
    max_length: int | None = None
    return_raw_data: bool = False

    def __call__(self, features: list[dict[str, Any] | None]) -> dict[str, Any]:
        features = [f for f in features if f is not None]
        if len(features) == 0:
            raise ValueError("Collator received empty features list!")
        images = [f["image"] for f in features]
        questions = [f["question"] for f in features]
        answers = [f["answer"] for f in features]
        batch = list(zip(images, questions, answers, strict=False))
        processed = self.processor(
            batch=batch,
            return_tensors="pt",
            truncation=self.max_length is not None,
            max_length=self.max_length,
            padding="longest",
        )
        result = dict(processed)
        packed = pack_padded(result)
        if self.return_raw_data:
            packed["questions"] = questions
            packed["answers"] = answers
            packed["images"] = images
        return packed


def pack_padded(batch: dict[str, Any]) -> dict[str, Any]:
    """Packs a padded processor output (``input_ids`` / ``attention_mask`` /
    optional ``labels`` ``[B, S]``) and carries every other key through."""
    ids = batch["input_ids"]
    mask = batch.get("attention_mask")
    if mask is None:
        mask = torch.ones_like(ids)
    labels = batch.get("labels")
    rows, lab_rows = [], []
    for i in range(ids.shape[0]):
        keep = mask[i].to(torch.bool)
        rows.append(ids[i][keep])
        if labels is not None:
            lab_rows.append(labels[i][keep])
    out = pack_rows(rows, lab_rows if labels is not None else None)
    if labels is None:
        out.pop("labels")
    for key, val in batch.items():
        if key not in ("input_ids", "attention_mask", "labels"):
            out[key] = val
    return out


__all__ = [
    "IGNORE_INDEX",
    "SiQ_VLPackingCollator",
    "assistant_label_mask",
    "pack_padded",
    "pack_rows",
]
