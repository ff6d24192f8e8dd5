"""Writes tests/golden/oracle_<case>.npz: the CPU oracle's outputs (f32 restatement of the reference's
WASM executor) for seeded subsets of the benchmark workloads, with the token ids they were made from.
The GPU parity tests compare the HIP runner against these vectors as well as against a live oracle
run; tests/test_golden.py checks that the oracle still reproduces them.

Two sets:
  * CASES: small subsets (a few sequences, some at reduced depth) that the oracle re-runs in seconds;
    the ids are stored whole.
  * FULL: the benchmark shapes themselves -- all 256 sequences of c2 and c3b, c3a at its 12 layers,
    c4 at its 22 layers on the 8192 bucket with two sequences longer than 4096 tokens (global
    attention over 7179 keys, the sliding window at length), 256 c5 pairs. Their ids are stored as
    a sha256 of the int32 array (the case regenerates them from the seeded streams).

    python tests/golden/make_golden.py [name ...]
"""
from __future__ import annotations

import hashlib
import os
import sys
import time

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

# the benchmark shapes (test_gpu_full.py)
FULL = {
    "c2_full": ("c2", 256, None, 512, None),
    "c3b_full": ("c3b", 256, None, 512, None),
    "c3a_full": ("c3a", 4, None, 512, None),
    "c4_full": ("c4", 6, None, 8192, None),
    "c5_full": ("c5", 256, None, 512, None),
}

ALL_CASES = {**CASES, **FULL}


def ids_digest(ids: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(ids, dtype=np.int32).tobytes()).hexdigest()


def case_of(name):
    w, batch, layers, length, max_len = ALL_CASES[name]
    return workload_case(w, batch, layers, length, max_len)


def make(name, first: int | None = None):
    """The oracle's outputs for the case (only its first `first` sequences when given), the
    sequence lengths and the concatenated ids of the whole case."""
    case = case_of(name)
    lens = np.array(case.lengths, dtype=np.int32)
    ids = np.concatenate(case.ids).astype(np.int32)
    if first is not None:
        case.ids = case.ids[:first]
    out = oracle_outputs(case)
    return out, lens, ids


def write(name):
    t = time.time()
    out, lens, ids = make(name)
    path = os.path.join(HERE, f"oracle_{name}.npz")
    if name in FULL:
        np.savez_compressed(path, out=out, lengths=lens, ids_sha256=np.array(ids_digest(ids)))
    else:
        np.savez_compressed(path, out=out, lengths=lens, ids=ids)
    print(name, out.shape, float(np.abs(out).max()), f"{time.time() - t:.1f}s", flush=True)


if __name__ == "__main__":
    for name in sys.argv[1:] or list(ALL_CASES):
        write(name)
