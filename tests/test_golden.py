"""The oracle against the committed golden fixtures (CPU).

tests/golden/*.npz hold seeded inputs and outputs written by
tests/golden/make_golden.py.  Re-deriving every output here pins the oracle
against drift: a change to its arithmetic shows up as a fixture mismatch,
bit for bit.
"""
import os
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))

import make_golden as mg  # noqa: E402


def load(name):
    return np.load(os.path.join(HERE, "golden", f"{name}.npz"))


@pytest.mark.parametrize("name", list(mg.MAKERS))
def test_oracle_reproduces_fixture(name):
    ref = load(name)
    got = mg.build(name)
    assert sorted(got) == sorted(ref.files)
    for key in ref.files:
        a, b = np.asarray(got[key]), ref[key]
        assert a.shape == b.shape and a.dtype == b.dtype, key
        assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), key


def test_fixtures_are_small():
    total = sum(os.path.getsize(os.path.join(HERE, "golden", f)) for f in os.listdir(os.path.join(HERE, "golden"))
                if f.endswith(".npz"))
    assert total < 400_000
