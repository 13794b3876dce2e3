"""The committed golden fixtures are what the (pinned) oracle produces from
their own inputs: regenerating them bit for bit guards against drift between
tests/golden/*.npz, the generator and the oracle (CPU)."""

import importlib.util
from pathlib import Path

import numpy as np
import pytest

GOLDEN = Path(__file__).resolve().parent / "golden"


def _generator():
    spec = importlib.util.spec_from_file_location("make_golden", GOLDEN / "make_golden.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="module")
def regenerated():
    return _generator().build_all()


@pytest.mark.parametrize("name", ["attn_causal_gqa_d128", "attn_bidir_d64", "ce_small"])
def test_fixture_matches_generator(name, regenerated):
    stored = np.load(GOLDEN / f"{name}.npz", allow_pickle=False)
    fresh = regenerated[name]
    assert sorted(stored.files) == sorted(fresh)
    for key in stored.files:
        assert stored[key].dtype == np.asarray(fresh[key]).dtype, key
        assert np.array_equal(stored[key], fresh[key]), key


def test_ce_fixture_has_the_edge_cases():
    f = np.load(GOLDEN / "ce_small.npz", allow_pickle=False)
    y = f["labels"]
    assert (y == -100).sum() > 0 and int(f["bad"]) == 1
    assert int(f["count"]) == int(((y >= 0) & (y < f["weight"].shape[0])).sum())
    ignored = (y == -100) | (y >= f["weight"].shape[0])
    assert np.all(f["dh"][ignored] == 0)
