"""The oracle still reproduces the committed golden vectors (tests/golden/make_golden.py), and the
vectors belong to the seeded inputs the parity tests build."""
from __future__ import annotations

import os

import numpy as np
import pytest

from tests.golden.make_golden import CASES, make

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.mark.parametrize("name", list(CASES))
def test_oracle_reproduces_golden(name):
    g = np.load(os.path.join(HERE, f"oracle_{name}.npz"))
    out, lens, ids = make(name)
    assert np.array_equal(lens, g["lengths"]) and np.array_equal(ids, g["ids"])
    assert np.allclose(out, g["out"], rtol=0, atol=1e-6), float(np.abs(out - g["out"]).max())
