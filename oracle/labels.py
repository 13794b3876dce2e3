"""Pure-Python restatement of the label bits of the path (test infrastructure only).

* ``assistant_labels``: the reference's supervised label mask,
  siq_vl/model/processing.py:450-479.  For each row with an answer: all
  positions -100, then the first ``<|im_start|>`` immediately followed by the
  ``assistant`` token opens the span at j + 3 (after im_start, assistant,
  newline) up to the next ``<|im_end|>`` (exclusive) or the row end; only the
  first assistant turn is unmasked; finally every ``<|image_pad|>`` is forced
  back to -100.  Rows without an answer stay fully masked.
* ``flatten``: the packing contract of DataCollatorWithFlattening
  (transformers data/data_collator.py:1424-1500): concatenate the rows, label
  each row's first token with the separator (``[sep] + labels[1:]``),
  position ids restart at 0, ``cu_seq_lens_q == cu_seq_lens_k`` are the
  running offsets and ``max_length_q == max_length_k`` the longest row.
* ``shift``: ForCausalLMLoss's left shift (transformers
  loss/loss_utils.py:63-64): append ignore_index, drop the first label.

Pinning (tests/test_labels.py): hand-worked known answers on synthetic id
rows (answer span, missing im_end, image pads inside the answer, second
assistant turn left masked, no-answer rows), and the property that after
flattening and shifting no label ever points across a sequence boundary.
"""

from __future__ import annotations

IGNORE = -100


def assistant_labels(rows: list[list[int]], has_answer: list[bool], im_start: int, assistant: int, im_end: int,
                     image_pad: int, ignore: int = IGNORE) -> list[list[int]]:
    out = []
    for ids, ans in zip(rows, has_answer):
        lab = [ignore] * len(ids)
        if ans:
            for j in range(len(ids)):
                if ids[j] == im_start and j + 1 < len(ids) and ids[j + 1] == assistant:
                    start = j + 3
                    end = len(ids)
                    for t in range(start, len(ids)):
                        if ids[t] == im_end:
                            end = t
                            break
                    for t in range(start, end):
                        lab[t] = ids[t]
                    break
            for t in range(len(ids)):
                if ids[t] == image_pad:
                    lab[t] = ignore
        out.append(lab)
    return out


def flatten(rows: list[list[int]], labels: list[list[int]] | None = None, separator: int = IGNORE) -> dict:
    input_ids: list[int] = []
    out_labels: list[int] = []
    position_ids: list[int] = []
    cu = [0]
    max_len = 0
    for i, ids in enumerate(rows):
        input_ids += list(ids)
        src = labels[i] if labels is not None else ids
        out_labels += [separator] + list(src[1:])
        position_ids += list(range(len(ids)))
        cu.append(cu[-1] + len(ids))
        max_len = max(max_len, len(ids))
    return {
        "input_ids": input_ids,
        "labels": out_labels,
        "position_ids": position_ids,
        "cu_seq_lens_q": cu,
        "cu_seq_lens_k": list(cu),
        "max_length_q": max_len,
        "max_length_k": max_len,
    }


def shift(labels: list[int], ignore: int = IGNORE) -> list[int]:
    padded = list(labels) + [ignore]
    return padded[1:]
