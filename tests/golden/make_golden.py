"""Writes tests/golden/oracle_<case>.npz: the CPU oracle's outputs (f32 restatement of the reference's
WASM executor) for seeded subsets of the benchmark workloads, with the token ids they were made from.
The GPU parity tests compare the HIP runner against these vectors as well as against a live oracle
run; tests/test_golden.py checks that the oracle still reproduces them.

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from tests.helpers import oracle_outputs, workload_case  # noqa: E402

# name: (workload, sequences, layers, bucket length, max tokens) -- the cases of test_gpu_models.py
CASES = {
    "c1": ("c1", 1, None, 128, None),
    "c2": ("c2", 12, None, 512, None),
    "c3a": ("c3a", 2, 4, 512, None),
    "c3b": ("c3b", 10, None, 512, None),
    "c4": ("c4", 3, 6, 1024, 700),
    "c5": ("c5", 6, None, 512, None),
}


def make(name):
    w, batch, layers, length, max_len = CASES[name]
    case = workload_case(w, batch, layers, length, max_len)
    out = oracle_outputs(case)
    lens = np.array(case.lengths, dtype=np.int32)
    ids = np.concatenate(case.ids).astype(np.int32)
    return out, lens, ids


if __name__ == "__main__":
    for name in CASES:
        out, lens, ids = make(name)
        np.savez_compressed(os.path.join(HERE, f"oracle_{name}.npz"), out=out, lengths=lens, ids=ids)
        print(name, out.shape, float(np.abs(out).max()))
