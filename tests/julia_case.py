"""A Julia decision-head case shared by the CPU and GPU tests: an encoder of the shape
specFromJuliaManifest gives (src/plan/spec.ts:248-277; ModernBERT layers with one RoPE theta, a
sliding window on two of every three layers, GeGLU, no biases, a final norm) at three layers over
seeded c4 ids cut to 200 tokens, the julia head (type row, two head layers, scorer over six option
slots), seeded weights, marker payloads and one qtype per sequence."""
from __future__ import annotations

import functools

import numpy as np

from kleinhirn_amd import configs, inputs
from kleinhirn_amd.plan import spec as S
from kleinhirn_amd.plan.build import build_plan, pack_markers
from tests.helpers import workload_case

LENGTH = 256
OPTIONS = 6
SPEC, HEAD = S.julia(384, 3, 6, 576, 50368, 1e-5, 160000.0, 64, 3, 2, 768, OPTIONS, 8192)


@functools.lru_cache(maxsize=2)
def case(batch: int = 3):
    c = workload_case("c4", batch, None, LENGTH, 200)
    W = configs.make_weights(SPEC, HEAD)
    return c.ids, W


def payloads(ids, seed: int = 11) -> tuple[list[np.ndarray], list[int]]:
    """Per sequence: the option markers (rows inside the sequence, as the [MASK] positions of
    src/julia.ts:174-183 with mask 1 for every given option), fewer options than slots on every
    other sequence, and a qtype in 0..2."""
    rng = np.random.default_rng(seed)
    packed, qtypes = [], []
    for b, seq in enumerate(ids):
        used = OPTIONS if b % 2 == 0 else OPTIONS - 2
        rows = np.sort(rng.integers(1, len(seq), size=used))
        packed.append(pack_markers(rows, np.ones(used, dtype=np.float32), None, OPTIONS))
        qtypes.append(int(b % S.JULIA_TYPES))
    return packed, qtypes


def oracle_logits(ids, W, packed, qtypes) -> np.ndarray:
    from oracle.oracle import OracleRuntime
    plan = build_plan(SPEC, HEAD, LENGTH, 1, False)
    p = OracleRuntime(W, [plan]).plan(plan, threads=8)
    table = W["embeddings.word.weight"]
    outs = []
    for seq, mk, q in zip(ids, packed, qtypes):
        ri = inputs.run_input(SPEC, table, [seq], LENGTH)
        p.upload(ri["embeddings"], ri["mask"], None, mk, q)
        p.run(len(seq))
        outs.append(p.read_output())
    return np.stack(outs)
