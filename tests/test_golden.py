"""The oracle against the committed golden fixtures (tests/golden/*.npz, written by
tests/golden/make_golden.py from the pinned oracle): any change of the oracle's results on these
seeded cases fails here."""

import importlib.util
from pathlib import Path

import numpy as np

GOLDEN = Path(__file__).resolve().parent / "golden"


def _maker():
    spec = importlib.util.spec_from_file_location("make_golden", GOLDEN / "make_golden.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _same(fresh: dict, stored, name: str):
    assert set(fresh) == set(stored.files), name
    for key, a in fresh.items():
        b = stored[key]
        assert a.shape == b.shape and a.dtype == b.dtype, (name, key)
        if a.dtype.kind in "biu":
            assert np.array_equal(a, b), (name, key)
        else:
            np.testing.assert_allclose(a, b, rtol=1e-12, atol=1e-12, err_msg=f"{name}: {key}")


def test_attention_golden():
    with np.load(GOLDEN / "attention_small.npz", allow_pickle=False) as stored:
        _same(_maker().attention_case(), stored, "attention_small")


def test_planner_golden():
    with np.load(GOLDEN / "planner_small.npz", allow_pickle=False) as stored:
        _same(_maker().planner_case(), stored, "planner_small")
