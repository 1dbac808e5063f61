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


def test_planner_loop_fixtures_prefix():
    """The full-size loop fixtures of configs 4 and 5 (planner_cfg4.npz / planner_cfg5.npz): the
    regenerated inputs have the stored digest and the oracle reproduces the first three steps."""
    mk = _maker()
    for cfg in (4, 5):
        fresh = mk.loop_case(cfg, steps=3)
        with np.load(GOLDEN / f"planner_cfg{cfg}.npz", allow_pickle=False) as stored:
            assert str(stored["digest"]) == str(fresh["digest"]), cfg
            assert np.array_equal(stored["T0"], fresh["T0"]) and np.array_equal(stored["layers"], fresh["layers"])
            for key, a in fresh.items():
                if key in ("digest", "T0", "layers", "full_steps"):
                    continue
                b = stored[key][:, :1] if key == "out_full" else stored[key][:, :3]
                a = a[:, :1] if key == "out_full" else a
                assert a.shape == b.shape and a.dtype == b.dtype, (cfg, key)
                if a.dtype.kind in "biu":
                    assert np.array_equal(a, b), (cfg, key)
                else:
                    np.testing.assert_allclose(a, b, rtol=1e-6, atol=1e-6, err_msg=f"config {cfg}: {key}")
