"""Shared test harness: seeded model cases, the CPU oracle's outputs and the HIP runner's outputs
for the same inputs, and the reference's parity rules (src/encoder.ts, convert/k28_close_calls.py)."""
from __future__ import annotations

import copy
import json

import numpy as np

from kleinhirn_amd import configs, inputs, synth
from kleinhirn_amd.plan.build import build_plan


_WEIGHTS: dict = {}


def seeded_weights(spec: dict, head: dict) -> dict:
    """configs.make_weights(spec, head), generated once per process (a RoBERTa-base set takes
    seconds); each caller gets its own dict over the shared read-only arrays."""
    key = json.dumps([spec, head], sort_keys=True)
    if key not in _WEIGHTS:
        w = configs.make_weights(spec, head)
        for v in w.values():
            v.setflags(write=False)
        _WEIGHTS[key] = w
    return dict(_WEIGHTS[key])


class Case:
    """A model (spec, head, f32 weights) and a ragged batch of token ids."""

    def __init__(self, spec, head, ids, length, weights=None):
        self.spec = spec
        self.head = head
        self.ids = ids
        self.length = length
        self.weights = weights if weights is not None else seeded_weights(spec, head)

    @property
    def lengths(self):
        return [len(x) for x in self.ids]


def shrink(spec: dict, layers: int | None = None) -> dict:
    s = copy.deepcopy(spec)
    if layers is not None:
        s["layers"] = layers
    return s


def workload_case(name: str, batch: int, layers: int | None = None, length: int | None = None,
                  max_len: int | None = None) -> Case:
    """The first `batch` sequences of a benchmark workload (lengths clipped to max_len), optionally
    with fewer layers."""
    w = configs.ALL[name]() if name != "c5" else configs.c5(max(batch, 1))
    ids = w.ids()[:batch]
    if max_len is not None:
        ids = [np.concatenate([x[: max_len - 1], x[-1:]]) if len(x) > max_len else x for x in ids]
    spec = shrink(w.spec, layers)
    return Case(spec, w.head, ids, length or w.length)


def oracle_outputs(case: Case, threads: int = 8) -> np.ndarray:
    """Per sequence on a B = 1 plan of the bucket length, only the real rows (the reference's WASM
    schedule, src/wasm-backend.ts:141-149). Returns [B, cols] (pooled heads)."""
    from oracle.oracle import OracleRuntime
    plan = build_plan(case.spec, case.head, case.length, 1, False)
    rt = OracleRuntime(case.weights, [plan])
    p = rt.plan(plan, threads=threads)
    table = case.weights["embeddings.word.weight"]
    outs = []
    for seq in case.ids:
        ri = inputs.run_input(case.spec, table, [seq], case.length)
        p.upload(ri["embeddings"], ri["mask"], ri["typeIds"])
        p.run(len(seq))
        outs.append(p.read_output())
    return np.stack(outs)


def hip_outputs(case: Case, f16: bool, batch_plan: bool = True, backend=None, by_ids: bool = False):
    """All sequences on one batch plan of the bucket length (or one B = 1 plan per sequence)."""
    from kleinhirn_amd.backend import HipBackend
    W = configs.storage(case.weights, f16)
    be = backend or HipBackend(W)
    table = W["embeddings.word.weight"]
    if batch_plan:
        plan = build_plan(case.spec, case.head, case.length, len(case.ids), f16)
        be.check(plan)
        r = be.runner(plan)
        if by_ids:
            be.set_words(table)
            mask, tt = inputs.mask_and_types(case.spec, case.ids, case.length)
            ids = np.zeros(case.length * len(case.ids), dtype=np.int32)
            for b, seq in enumerate(case.ids):
                ids[b * case.length:b * case.length + len(seq)] = seq
            r.upload_ids(ids, mask, tt)
        else:
            r.upload(inputs.run_input(case.spec, table, case.ids, case.length))
        r.run(case.length * len(case.ids))
        out = r.read_output().reshape(len(case.ids), -1)
        r.destroy()
    else:
        plan = build_plan(case.spec, case.head, case.length, 1, f16)
        r = be.runner(plan)
        outs = []
        for seq in case.ids:
            r.upload(inputs.run_input(case.spec, table, [seq], case.length))
            r.run(len(seq))
            outs.append(r.read_output())
        out = np.stack(outs)
        r.destroy()
    if backend is None:
        be.dispose()
    return out


def cosine_rows(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    a = a.astype(np.float64)
    b = b.astype(np.float64)
    return (a * b).sum(1) / (np.linalg.norm(a, axis=1) * np.linalg.norm(b, axis=1))


def decision_parity(ref: np.ndarray, got: np.ndarray) -> dict:
    """Argmax agreement under the reference's close-call rule: a decision whose f32 top-2 gap is
    below 2 delta (delta = the run's largest logit deviation) can be flipped by rounding and is
    excluded (convert/k28_close_calls.py:1-8)."""
    delta = float(np.abs(ref - got).max())
    out = {"delta": delta, "n": len(ref)}
    if ref.shape[1] < 2:
        out.update(excluded=0, agree=len(ref), mismatched=0)
        return out
    top2 = np.sort(ref, axis=1)[:, -2:]
    gap = top2[:, 1] - top2[:, 0]
    flippable = gap < 2 * delta
    same = ref.argmax(1) == got.argmax(1)
    out.update(excluded=int(flippable.sum()), agree=int((same | flippable).sum()),
               mismatched=int((~same & ~flippable).sum()), identical=int(same.sum()))
    return out
