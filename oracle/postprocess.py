"""TEST INFRASTRUCTURE — the reference's score helpers restated on the CPU, to check kh_scores /
kh_read_scores / kh_rank against.

Only tests/ import this module; the product path never does.

JavaScript numbers are doubles and Float32Array stores round to f32, so each step is a Python
float operation followed, where the reference stores into a Float32Array, by a rounding to f32:
* softmax (src/tasks.ts:22-33): max, e^(x - max) stored f32, a double sum of the stored values,
  each stored value / sum stored f32;
* sigmoid of the multi-label classify (src/encoder.ts:506-507): 1 / (1 + e^-x) stored f32;
* l2normalize (src/tasks.ts:35-42): double sum of squares, max(sqrt, 1e-12), x / norm stored f32;
* softmaxPrefix of the Julia head's option logits (src/julia.ts:57-65): max, a double sum of
  e^(x - max) with nothing stored in between, each e^(x - max) / sum stored f32;
* argmaxRows (src/tasks.ts:72-84): strict '>' scan, ties to the lower index;
* rerank order (src/encoder.ts:541): by score descending, then index.
Pinned by the reference's own vectors (tests/tasks.test.ts:5-32 of the reference) in
tests/test_scores.py; softmax_prefix, which no reference test covers, by closed forms there.
"""
from __future__ import annotations

import math

import numpy as np

SOFTMAX, SIGMOID, RAW, L2, OPTIONS = 0, 1, 2, 3, 4


def f32(x: float) -> float:
    return float(np.float32(x))


def softmax(row) -> list[float]:
    mx = -math.inf
    for v in row:
        mx = max(mx, float(v))
    out = [f32(math.exp(float(v) - mx)) for v in row]
    s = 0.0
    for o in out:
        s += o
    return [f32(o / s) for o in out]


def softmax_prefix(row) -> list[float]:
    mx = -math.inf
    for v in row:
        mx = max(mx, float(v))
    s = 0.0
    for v in row:
        s += math.exp(float(v) - mx)
    return [f32(math.exp(float(v) - mx) / s) for v in row]


def sigmoid(row) -> list[float]:
    return [f32(1.0 / (1.0 + math.exp(-float(v)))) for v in row]


def l2normalize(row) -> list[float]:
    sq = 0.0
    for v in row:
        sq += float(v) * float(v)
    norm = max(math.sqrt(sq), 1e-12)
    return [f32(float(v) / norm) for v in row]


def argmax(row) -> int:
    best = 0
    for c in range(1, len(row)):
        if row[c] > row[best]:
            best = c
    return best


def argmax_rows(data, cols: int) -> list[int]:
    rows = len(data) // cols
    return [argmax(list(data[r * cols:(r + 1) * cols])) for r in range(rows)]


def scores(logits: np.ndarray, kind: int) -> tuple[np.ndarray, np.ndarray]:
    """[rows, cols] f32 -> (scores [rows, cols] f32, label index per row)."""
    out = np.empty(logits.shape, dtype=np.float32)
    idx = np.empty(logits.shape[0], dtype=np.int32)
    for r, row in enumerate(logits.tolist()):
        if kind == SOFTMAX:
            s = softmax(row)
            idx[r] = argmax(s)
        elif kind == OPTIONS:
            s = softmax_prefix(row)
            idx[r] = argmax(s)
        elif kind == SIGMOID:
            s = sigmoid(row)
            idx[r] = argmax(row)
        elif kind == L2:
            s = l2normalize(row)
            idx[r] = argmax(row)
        else:
            s = row
            idx[r] = argmax(row)
        out[r] = s
    return out, idx


def rank(values) -> list[int]:
    v = [float(x) for x in values]
    return sorted(range(len(v)), key=lambda i: (-v[i], i))
