"""The committed golden fixtures reproduce: each case function of tests/golden/make_golden.py,
run again here, returns arrays equal to the ones in the committed .npz, bit for bit.

The store fixture needs the reference's own store built into oracle/_ref (make -C oracle with
the reference sources present); without it that case is skipped.
"""
from __future__ import annotations

import importlib.util
from pathlib import Path

import numpy as np
import pytest

GOLDEN = Path(__file__).resolve().parent / "golden"


def _maker():
    spec = importlib.util.spec_from_file_location("make_golden", GOLDEN / "make_golden.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _same(got: dict, name: str):
    with np.load(GOLDEN / name) as want:
        assert sorted(got) == sorted(want.files), name
        for k in want.files:
            a, b = np.asarray(got[k]), want[k]
            assert a.dtype == b.dtype and a.shape == b.shape, (name, k)
            assert a.tobytes() == b.tobytes(), (name, k)


@pytest.mark.parametrize("case,name", [("latest_match_cases", "latest_match.npz"),
                                       ("pack_cases", "pack.npz"),
                                       ("gather_cases", "gather.npz")])
def test_oracle_fixtures_reproduce(oracle_lib, case, name):
    _same(getattr(_maker(), case)(), name)


def test_store_fixture_reproduces(oracle_lib):
    import oracle
    if oracle.ref_store() is None:
        pytest.skip("oracle/_ref holds no reference store build")
    _same(_maker().store_cases(), "store.npz")
