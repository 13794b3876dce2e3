"""Bounds of the attention scheduler's work lists, checked on the CPU.

The dK/dV scheduler (siq_vl_amd/csrc/sched.hip) cuts kv tiles heavier than a
piece length S into pieces whose fp32 partial sums go to a fixed pool of split
slots; the work-item list and the slot pool have fixed capacities
(kv_item_cap, kSplitSlots in attn.h).  This test restates the scheduler's
integer arithmetic (piece length, pieces per tile, items, slots) and checks
the capacities against random and adversarial length mixes -- the skewed
config 5, many tiny sequences, one huge sequence, hkv 1..16, n_rep up to 16 --
so that a change of the constants or of the S rule that could overflow a list
fails here, on the CPU.  The scheduler also records any overflow in the plan
header (checked on the GPU by tests/test_gpu_plan.py).
"""

import random
import re
from pathlib import Path

import pytest

from siq_vl_amd import workloads as W

ATTN_H = Path(__file__).resolve().parents[1] / "siq_vl_amd" / "csrc" / "attn.h"


def _constants():
    text = ATTN_H.read_text()
    out = {}
    for name in ("kFwdBM", "kBwdBN", "kBwdBM", "kSplitTarget", "kMinSplitSteps", "kLongPiece"):
        m = re.search(r"constexpr int " + name + r"\s*=\s*(\d+)", text)
        assert m, name
        out[name] = int(m.group(1))
    m = re.search(r"constexpr int kSplitSlots\s*=\s*(\d+)\s*\*\s*kSplitTarget\s*\+\s*(\d+)", text)
    assert m
    out["kSplitSlots"] = int(m.group(1)) * out["kSplitTarget"] + int(m.group(2))
    out["kMaxSplitTiles"] = out["kSplitSlots"] // 2
    return out


C = _constants()


def kv_tile_steps(q_len, k_len, t, causal, n_rep):
    off = k_len - q_len
    qb0 = max(0, t * C["kBwdBN"] - off) // C["kBwdBM"] if causal else 0
    nqb = (q_len - qb0 * C["kBwdBM"] + C["kBwdBM"] - 1) // C["kBwdBM"] if q_len > qb0 * C["kBwdBM"] else 0
    return nqb * n_rep


def piece_length(steps, hkv):
    target, long_piece = C["kSplitTarget"], C["kLongPiece"]
    sl = (steps * hkv + target - 1) // target
    if sl > long_piece:
        half = (steps * hkv + 2 * target - 1) // (2 * target)
        sl = half if half > long_piece else long_piece
    sl = max(sl, C["kMinSplitSteps"])
    return min(sl, 1 << 30)


def schedule_counts(lengths, hkv, n_rep, causal=True):
    """(q tiles, kv tiles, items, split tiles, slots used x hkv) of the schedule."""
    tiles = []
    for n in lengths:
        nt = (n + C["kBwdBN"] - 1) // C["kBwdBN"]
        tiles += [kv_tile_steps(n, n, t, causal, n_rep) for t in range(nt)]
    steps = sum(tiles)
    S = piece_length(steps, hkv)
    items, split_tiles, slots = 0, 0, 0
    for w in tiles:
        np_ = (w + S - 1) // S if w > S else 1
        items += np_
        if np_ > 1:
            split_tiles += 1
            slots += np_
    qtiles = sum((n + C["kFwdBM"] - 1) // C["kFwdBM"] for n in lengths)
    return qtiles, len(tiles), items, split_tiles, slots * hkv


def caps(lengths):
    total, batch = sum(lengths), len(lengths)
    qcap = total // C["kFwdBM"] + batch + 1
    kvcap = total // C["kBwdBN"] + batch + 1 + 2 * C["kSplitTarget"] + 1
    return qcap, kvcap


def _check(lengths, hkv, n_rep, causal=True):
    qt, tiles, items, split_tiles, slots = schedule_counts(lengths, hkv, n_rep, causal)
    qcap, kvcap = caps(lengths)
    assert qt <= qcap
    assert items <= kvcap, (items, kvcap)
    assert split_tiles <= C["kMaxSplitTiles"]
    assert slots <= C["kSplitSlots"], (slots, C["kSplitSlots"])
    return items, slots


def _mixes(rng):
    yield list(W.attn_config(2).lengths)
    yield list(W.attn_config(3).lengths)
    yield list(W.attn_config(5).lengths)
    yield [16384]
    yield [65536]
    yield [1] * 4096
    yield [16384, 8192] + [81] * 101
    yield [4096] * 4 + [1] * 3000
    for _ in range(40):
        kind = rng.randrange(4)
        if kind == 0:
            yield [rng.randint(1, 600) for _ in range(rng.randint(1, 400))]
        elif kind == 1:
            yield [rng.randint(1, 32768) for _ in range(rng.randint(1, 8))]
        elif kind == 2:
            big = [rng.randint(2048, 40000) for _ in range(rng.randint(1, 3))]
            yield big + [rng.randint(1, 300) for _ in range(rng.randint(0, 500))]
        else:
            # many tiles just above the piece length: the most pieces per step
            yield [rng.choice([129, 257, 385, 513, 1025]) for _ in range(rng.randint(10, 300))]


@pytest.mark.parametrize("hkv", [1, 2, 4, 8, 16])
@pytest.mark.parametrize("n_rep", [1, 2, 6, 7, 16])
def test_schedule_fits_its_lists(hkv, n_rep):
    rng = random.Random(1000 * hkv + n_rep)
    for lengths in _mixes(rng):
        for causal in (True, False):
            _check(lengths, hkv, n_rep, causal)


def test_worst_case_slot_use_is_close_to_the_bound():
    # the bound is not vacuous: some schedule uses most of the slot pool
    rng = random.Random(7)
    worst = 0
    for hkv in (1, 2, 8):
        for lengths in _mixes(rng):
            worst = max(worst, _check(lengths, hkv, 6)[1])
    assert worst > C["kSplitSlots"] // 4


def test_piece_length_rule():
    # S >= hkv * steps / (2 kSplitTarget) for every total, the inequality the bounds rest on
    for steps in list(range(1, 5000)) + [10**5, 10**6, 10**7]:
        for hkv in (1, 2, 3, 8, 16):
            S = piece_length(steps, hkv)
            assert 2 * C["kSplitTarget"] * S >= steps * hkv
