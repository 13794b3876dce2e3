"""CPU oracle of the vision-token splice -- TEST INFRASTRUCTURE ONLY.

Restates SiQ_VLForCausalLM.forward's splice (siq_vl/model/modeling.py:252-270):
the embedding lookup, the row-major order of the image-token positions
(``nonzero``), the count check, and the assignment of the vision rows to those
positions; and its backward (IndexPutBackward zeroes the image rows' gradient
before the embedding's backward, which accumulates the rest per token id; the
vision rows get the gradient of their positions).

Parity pinning (tests/test_oracle_splice.py): a hand-worked known answer,
torch's own ops and autograd on the CPU (the library the reference runs),
the count-check message, and the conservation identities (every text row's
gradient lands in its id's row; every image row's in its vision row).
"""

from __future__ import annotations

import numpy as np


def image_positions(ids, image_id: int) -> np.ndarray:
    """Flat (row-major) indices of the image tokens -- nonzero()'s order."""
    return np.flatnonzero(np.asarray(ids).reshape(-1) == image_id)


def splice_fwd(ids, weight, vision, image_id: int) -> np.ndarray:
    ids = np.asarray(ids)
    weight = np.asarray(weight)
    vision = np.asarray(vision)
    pos = image_positions(ids, image_id)
    if pos.size != vision.shape[0]:
        raise ValueError(f"Shape Mismatch! Text has {pos.size} image placeholders, "
                         f"Vision Encoder produced {vision.shape[0]} tokens.")
    flat = ids.reshape(-1)
    out = weight[flat].copy()
    out[pos] = vision
    return out.reshape(*ids.shape, weight.shape[1])


def splice_bwd(grad, ids, image_id: int, vocab: int, padding_idx: int | None = None):
    """(d_weight [vocab, H], d_vision [n_image, H]) in float64."""
    ids = np.asarray(ids).reshape(-1)
    g = np.asarray(grad, dtype=np.float64).reshape(ids.size, -1)
    pos = image_positions(ids, image_id)
    d_vision = g[pos].copy()
    gm = g.copy()
    gm[pos] = 0.0
    d_weight = np.zeros((vocab, g.shape[1]))
    np.add.at(d_weight, ids, gm)
    if padding_idx is not None and padding_idx >= 0:
        d_weight[padding_idx] = 0.0
    return d_weight, d_vision
