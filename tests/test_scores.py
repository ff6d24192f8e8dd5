"""Scores from outputs on the CPU: kh_scores / kh_rank of libkh_hip.so against the restated score
helpers of oracle/postprocess.py, which are pinned by the reference's own vectors
(tests/tasks.test.ts:5-32 of the reference) and by closed forms."""
from __future__ import annotations

import math

import numpy as np
import pytest

from kleinhirn_amd import backend as B
from oracle import postprocess as P

RNG = np.random.default_rng(11)


def test_oracle_matches_the_reference_vectors():
    p = P.softmax([1, 2, 3])
    assert abs(sum(p) - 1) < 1e-6 and p[0] < p[1] < p[2]
    assert abs(p[2] - 0.6652409557748219) < 1e-6
    p = P.softmax([1000, 1001])
    assert math.isfinite(p[0]) and abs(p[1] - 0.7310585786300049) < 1e-6
    assert P.l2normalize([3, 4]) == [0.6000000238418579, 0.800000011920929]
    assert P.argmax_rows([1, 3, 2, 5, 5, 0], 3) == [1, 0]
    assert P.argmax_rows([1, 3, 2, 5], 2) == [1, 1]
    z = P.softmax([-2.595508098602295, -0.0128010343760252, 0.7721060514450073, -2.5513229370117188,
                   -2.819657802581787])
    assert P.argmax(z) == 2 and abs(z[2] - 0.6434125900268555) < 1e-6


def test_oracle_closed_forms():
    assert P.sigmoid([0.0]) == [0.5]
    assert P.softmax([0.0, 0.0, 0.0, 0.0]) == [0.25] * 4
    v = RNG.standard_normal(384).astype(np.float32)
    n = np.array(P.l2normalize(v.tolist()), dtype=np.float64)
    assert abs(np.linalg.norm(n) - 1) < 1e-6
    assert P.l2normalize([0.0, 0.0]) == [0.0, 0.0]  # the 1e-12 floor keeps zero rows finite
    assert P.rank([0.5, 2.0, 0.5, -1.0]) == [1, 0, 2, 3]


def test_option_softmax_closed_forms():
    """Julia's option probabilities (softmaxPrefix, src/julia.ts:57-65) where the exact value is
    known, and where it parts from the tasks softmax (which stores each exponential as f32 before
    the sum)."""
    assert P.softmax_prefix([0.0, 0.0, 0.0, 0.0]) == [0.25] * 4
    want = [1 / 6, 2 / 6, 3 / 6]
    got = P.softmax_prefix([0.0, math.log(2.0), math.log(3.0)])
    assert all(abs(g - w) < 6e-8 for g, w in zip(got, want)), got
    assert P.softmax_prefix([-1e4, 0.0]) == [0.0, 1.0]  # e^-10000 underflows: one option takes all
    assert P.softmax_prefix([7.5]) == [1.0]
    # the sum of the unrounded exponentials: the two softmaxes differ in the last bit on some rows
    x = (RNG.standard_normal((2000, 5)) * 3).astype(np.float32)
    diff = 0
    for row in x.tolist():
        a, b = P.softmax_prefix(row), P.softmax(row)
        assert max(abs(u - v) for u, v in zip(a, b)) <= 1.2e-7
        assert abs(sum(a) - 1) < 1e-6
        diff += a != b
    assert diff > 0


def test_library_matches_the_reference_vectors():
    s, i = B.scores(np.array([[1, 2, 3]], np.float32))
    assert abs(s[0, 2] - 0.6652409557748219) < 1e-6 and i[0] == 2
    s, _ = B.scores(np.array([[1000, 1001]], np.float32))
    assert abs(s[0, 1] - 0.7310585786300049) < 1e-6
    s, _ = B.scores(np.array([[3, 4]], np.float32), B.SCORES_L2)
    assert s[0].tolist() == [0.6000000238418579, 0.800000011920929]
    _, i = B.scores(np.array([[1, 3, 2], [5, 5, 0]], np.float32), B.SCORES_RAW)
    assert i.tolist() == [1, 0]


@pytest.mark.parametrize("kind", [B.SCORES_SOFTMAX, B.SCORES_SIGMOID, B.SCORES_RAW, B.SCORES_L2, B.SCORES_OPTIONS])
def test_library_equals_oracle_bit_for_bit(kind):
    for rows, cols in [(256, 3), (64, 384), (4096, 1), (7, 2)]:
        x = (RNG.standard_normal((rows, cols)) * 4).astype(np.float32)
        x[0, :] = x[0, 0]  # a row of ties
        got, gi = B.scores(x, kind)
        want, wi = P.scores(x, kind)
        assert np.array_equal(got, want), (kind, rows, cols)
        assert np.array_equal(gi, wi)


def test_rank_and_errors():
    v = np.array([0.25, 3.0, 0.25, -2.0, 3.0], np.float32)
    assert B.rank(v).tolist() == P.rank(v.tolist()) == [1, 4, 0, 2, 3]
    bad = np.array([[1.0, np.nan, np.inf]], np.float32)
    with pytest.raises(B.KhError, match="output: 2 of 3 values are not finite"):
        B.scores(bad)
    with pytest.raises(B.KhError, match="not finite"):
        B.rank(bad.ravel())
    with pytest.raises(B.KhError, match="scores kind 7"):
        B.scores(np.ones((1, 2), np.float32), 7)
