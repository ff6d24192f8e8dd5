"""A GLiNER2 span-head case shared by the CPU and GPU tests: the DeBERTa-v3 encoder of the c3b
workload cut to two layers, the gliner2 head of the reference's GLiNER manifests
(src/plan/spec.ts:213-246: hidden 768, a temperature, 16 marker slots by default), seeded weights
and seeded marker payloads (row indices inside each sequence, some slots masked)."""
from __future__ import annotations

import functools

import numpy as np

from kleinhirn_amd import configs, inputs
from kleinhirn_amd.plan.build import build_plan, pack_markers
from tests.helpers import workload_case

HEAD = {"type": "gliner2", "hidden": 768, "temperature": 0.5, "markers": 8}
LENGTH = 128


@functools.lru_cache(maxsize=4)
def case(batch: int = 3):
    c = workload_case("c3b", batch, 2, LENGTH, LENGTH)
    W = configs.make_weights(c.spec, HEAD)
    return c, W


def payloads(ids, markers: int = 8, seed: int = 7) -> list[np.ndarray]:
    """Per sequence: up to `markers` rows inside the sequence, every third slot masked, the last
    slot left empty (padded) when the sequence is long enough."""
    rng = np.random.default_rng(seed)
    out = []
    for seq in ids:
        n = len(seq)
        used = markers - 1 if n > markers else markers
        rows = rng.integers(0, n, size=used)
        mask = np.array([0.0 if k % 3 == 2 else 1.0 for k in range(used)], dtype=np.float32)
        groups = np.arange(used) // 2
        out.append(pack_markers(rows, mask, groups, markers))
    return out


def oracle_logits(c, W, packed) -> np.ndarray:
    """The oracle's logits per sequence on a B = 1 plan (the reference's WASM schedule)."""
    from oracle.oracle import OracleRuntime
    plan = build_plan(c.spec, HEAD, LENGTH, 1, False)
    p = OracleRuntime(W, [plan]).plan(plan, threads=8)
    table = W["embeddings.word.weight"]
    outs = []
    for seq, mk in zip(c.ids, packed):
        ri = inputs.run_input(c.spec, table, [seq], LENGTH)
        p.upload(ri["embeddings"], ri["mask"], ri.get("typeIds"), mk)
        p.run(len(seq))
        outs.append(p.read_output())
    return np.stack(outs)
