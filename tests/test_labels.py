"""Label masking, packing and shift: the integer bits of the path (CPU).

The oracle (oracle/labels.py) is pinned by hand-worked known answers on
synthetic id rows; the product code (siq_vl_amd/collator.py,
siq_vl_amd/cross_entropy.shift_labels) must then agree with it bit for bit.
Token ids are parameters (Qwen's values are the defaults, tokenizer-free).
"""

import random

import pytest
import torch

from oracle import labels as ol
from siq_vl_amd import collator
from siq_vl_amd.cross_entropy import shift_labels

S, A, E, P = 151644, 77091, 151645, 151655  # im_start, assistant, im_end, image_pad
NL = 198
I = -100


# --------------------------------------------------------------------------- oracle KATs
def test_oracle_answer_span():
    row = [S, 8948, NL, 5, 6, E, NL, S, A, NL, 11, 12, 13, E, NL]
    want = [I] * 10 + [11, 12, 13] + [I, I]
    assert ol.assistant_labels([row], [True], S, A, E, P) == [want]


def test_oracle_missing_im_end_runs_to_row_end():
    row = [S, A, NL, 21, 22, 23]
    assert ol.assistant_labels([row], [True], S, A, E, P) == [[I, I, I, 21, 22, 23]]


def test_oracle_image_pad_inside_answer_is_masked():
    row = [S, A, NL, 31, P, P, 32, E]
    assert ol.assistant_labels([row], [True], S, A, E, P) == [[I, I, I, 31, I, I, 32, I]]


def test_oracle_only_first_assistant_turn():
    row = [S, A, NL, 41, E, S, A, NL, 42, E]
    assert ol.assistant_labels([row], [True], S, A, E, P) == [[I, I, I, 41, I, I, I, I, I, I]]


def test_oracle_no_answer_row_and_no_assistant():
    rows = [[S, A, NL, 7, E], [S, 8948, NL, 7, E]]
    out = ol.assistant_labels(rows, [False, True], S, A, E, P)
    assert out == [[I] * 5, [I] * 5]


def test_oracle_assistant_at_row_end_has_empty_span():
    row = [1, 2, S, A]
    assert ol.assistant_labels([row], [True], S, A, E, P) == [[I] * 4]


def test_oracle_flatten_known_answer():
    out = ol.flatten([[1, 2, 3], [4, 5]], [[9, 8, 7], [6, 5]])
    assert out["input_ids"] == [1, 2, 3, 4, 5]
    assert out["labels"] == [I, 8, 7, I, 5]
    assert out["position_ids"] == [0, 1, 2, 0, 1]
    assert out["cu_seq_lens_q"] == [0, 3, 5] and out["cu_seq_lens_k"] == [0, 3, 5]
    assert out["max_length_q"] == 3 and out["max_length_k"] == 3


def test_oracle_shift_known_answer():
    assert ol.shift([I, 8, 7, I, 5]) == [8, 7, I, 5, I]


# --------------------------------------------------------------------------- product vs oracle
def random_rows(seed, n_rows=6, ids=(S, A, E, P, NL)):
    rng = random.Random(seed)
    rows = []
    for _ in range(n_rows):
        n = rng.randint(1, 40)
        row = [rng.choice(list(ids) + [rng.randint(0, 1000) for _ in range(5)]) for _ in range(n)]
        if rng.random() < 0.7 and n > 6:  # plant a real assistant turn
            j = rng.randint(0, n - 4)
            row[j], row[j + 1], row[j + 2] = S, A, NL
        rows.append(row)
    return rows


@pytest.mark.parametrize("seed", range(8))
def test_assistant_label_mask_matches_oracle(seed):
    rows = random_rows(seed)
    has = [random.Random(seed + 100 + i).random() < 0.85 for i in range(len(rows))]
    pad_id = 0
    seq = max(len(r) for r in rows)
    padded = torch.tensor([r + [pad_id] * (seq - len(r)) for r in rows], dtype=torch.int64)
    got = collator.assistant_label_mask(padded, S, A, E, P, has_answer=has)
    # the oracle sees the padded rows too (the processor masks after padding)
    want = ol.assistant_labels([r + [pad_id] * (seq - len(r)) for r in rows], has, S, A, E, P)
    assert got.tolist() == want


def test_assistant_label_mask_other_token_ids():
    s2, a2, e2, p2 = 10, 11, 12, 13
    row = torch.tensor([[s2, a2, 99, 1, p2, 2, e2, 3]])
    assert collator.assistant_label_mask(row, s2, a2, e2, p2).tolist() == [[I, I, I, 1, I, 2, I, I]]


@pytest.mark.parametrize("seed", range(6))
def test_pack_rows_matches_oracle_flatten(seed):
    rows = random_rows(seed, n_rows=1 + seed)
    labs = ol.assistant_labels(rows, [True] * len(rows), S, A, E, P)
    got = collator.pack_rows([torch.tensor(r) for r in rows], [torch.tensor(l) for l in labs])
    want = ol.flatten(rows, labs)
    assert got["input_ids"].shape == (1, len(want["input_ids"]))
    assert got["input_ids"][0].tolist() == want["input_ids"]
    assert got["labels"][0].tolist() == want["labels"]
    assert got["position_ids"][0].tolist() == want["position_ids"]
    assert got["cu_seq_lens_q"].dtype == torch.int32 and got["cu_seq_lens_k"].dtype == torch.int32
    assert got["cu_seq_lens_q"].tolist() == want["cu_seq_lens_q"]
    assert got["cu_seq_lens_k"].tolist() == want["cu_seq_lens_k"]
    assert got["max_length_q"] == want["max_length_q"] and isinstance(got["max_length_q"], int)
    assert got["max_length_k"] == want["max_length_k"] and isinstance(got["max_length_k"], int)


def test_pack_rows_without_labels_uses_ids():
    got = collator.pack_rows([torch.tensor([5, 6, 7]), torch.tensor([8])])
    assert got["labels"][0].tolist() == [I, 6, 7, I]


def test_pack_rows_errors():
    with pytest.raises(ValueError):
        collator.pack_rows([])
    with pytest.raises(ValueError):
        collator.pack_rows([torch.tensor([1, 2])], [torch.tensor([1])])


@pytest.mark.parametrize("seed", range(4))
def test_shift_never_crosses_sequence_boundary(seed):
    rows = random_rows(seed + 50, n_rows=5)
    packed = collator.pack_rows([torch.tensor(r) for r in rows])
    ids = packed["input_ids"][0].tolist()
    tgt = shift_labels(packed["labels"])[0].tolist()
    assert tgt == ol.shift(packed["labels"][0].tolist())
    cu = packed["cu_seq_lens_q"].tolist()
    ends = set(c - 1 for c in cu[1:])
    for t, y in enumerate(tgt):
        if t in ends:
            assert y == I  # the last token of a row never predicts the next row
        elif y != I:
            assert y == ids[t + 1]


def test_shift_labels_batched_matches_oracle():
    lab = torch.tensor([[1, 2, 3, I], [I, 5, 6, 7]])
    got = shift_labels(lab)
    assert got.tolist() == [ol.shift(r) for r in lab.tolist()]


def test_pack_padded_drops_padding_and_passes_other_keys():
    ids = torch.tensor([[1, 2, 3, 0], [4, 5, 0, 0]])
    mask = torch.tensor([[1, 1, 1, 0], [1, 1, 0, 0]])
    labels = torch.tensor([[I, 2, 3, I], [I, 5, I, I]])
    pix = torch.zeros(3, 3)
    out = collator.pack_padded({"input_ids": ids, "attention_mask": mask, "labels": labels, "pixel_values": pix,
                                "num_image_tokens": [1, 2]})
    assert out["input_ids"][0].tolist() == [1, 2, 3, 4, 5]
    assert out["labels"][0].tolist() == [I, 2, 3, I, 5]
    assert out["cu_seq_lens_q"].tolist() == [0, 3, 5]
    assert out["pixel_values"] is pix and out["num_image_tokens"] == [1, 2]
    assert "attention_mask" not in out


class _FakeProcessor:
    """Stands in for SiQ_VLProcessor: tokenises a question/answer pair into
    synthetic ids with the chat-template skeleton and masks like the reference."""

    def __call__(self, batch, return_tensors, truncation, max_length, padding):
        rows, has = [], []
        for image, question, answer in batch:
            row = [S, 900 + len(question), NL] + [P] * image + [E, NL, S, A, NL]
            if answer is not None:
                row += [1000 + ord(c) for c in answer] + [E]
            rows.append(row)
            has.append(answer is not None)
        if truncation:
            rows = [r[:max_length] for r in rows]
        seq = max(len(r) for r in rows)
        ids = torch.tensor([r + [0] * (seq - len(r)) for r in rows])
        mask = torch.tensor([[1] * len(r) + [0] * (seq - len(r)) for r in rows])
        labels = collator.assistant_label_mask(ids, S, A, E, P, has_answer=has)
        return {"input_ids": ids, "attention_mask": mask, "labels": labels, "pixel_values": torch.ones(len(rows), 2)}


def test_packing_collator_end_to_end():
    feats = [{"image": 2, "question": "q1", "answer": "ab"}, None, {"image": 0, "question": "qq2", "answer": "xyz"},
             {"image": 1, "question": "q", "answer": None}]
    col = collator.SiQ_VLPackingCollator(_FakeProcessor(), return_raw_data=True)
    out = col(feats)
    rows = []
    for f in [f for f in feats if f is not None]:
        row = [S, 900 + len(f["question"]), NL] + [P] * f["image"] + [E, NL, S, A, NL]
        if f["answer"] is not None:
            row += [1000 + ord(c) for c in f["answer"]] + [E]
        rows.append(row)
    labs = ol.assistant_labels(rows, [True, True, False], S, A, E, P)
    want = ol.flatten(rows, labs)
    assert out["input_ids"][0].tolist() == want["input_ids"]
    assert out["labels"][0].tolist() == want["labels"]
    assert out["cu_seq_lens_q"].tolist() == want["cu_seq_lens_q"]
    assert out["questions"] == ["q1", "qq2", "q"] and out["answers"] == ["ab", "xyz", None]
    with pytest.raises(ValueError):
        col([None])
