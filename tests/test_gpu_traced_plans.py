"""The reference's traced plan shapes (tests/helpers/plan-trace.ts:24-73) run on the GPU against the
oracle: the GLiNER-base plan (DeBERTa-v2, 12 layers, hidden 768, relative attention with 256 log
buckets, span head of width 1536 over 16 marker slots) at L = 512 and L = 1280, and the Julia-1 plan
(22 ModernBERT layers, hidden 384, window 64 on two of three layers, RoPE 160000, two head layers,
20 option slots) at L = 512. tests/test_plan_traces.py pins these plan documents to the reference's
frozen dispatch lists; here they execute, with seeded weights and marker payloads, through the C
ABI. Bars: f32 logits within 1e-3 of the oracle, f16 within 2e-2; masked slots exactly -1e4."""
from __future__ import annotations

import numpy as np
import pytest

from kleinhirn_amd import configs, inputs, synth
from kleinhirn_amd.plan import spec as S
from kleinhirn_amd.plan.build import build_plan, pack_markers
from tests.helpers import seeded_weights
from tests.plan_trace import GLINER_HEAD_HIDDEN, GLINER_SPECS, JULIA_SPEC

pytestmark = pytest.mark.gpu

VOCAB = 30000


def gliner_base(markers=16):
    spec, head = S.gliner(dict(GLINER_SPECS["base"], vocabSize=VOCAB), 1.0, GLINER_HEAD_HIDDEN["base"], markers)
    return spec, head


def julia_1():
    j = JULIA_SPEC
    return S.julia(j["hiddenSize"], j["layers"], j["heads"], j["intermediate"], VOCAB, j["normEps"], j["ropeTheta"],
                   j["localAttention"], j["globalEvery"], j["headLayers"], j["headFfn"], j["options"])


def sequences(lengths, seed):
    return synth.draw_ids(seed, lengths, VOCAB, 1, 2)


def payloads(ids, slots, seed, all_on=False):
    rng = np.random.default_rng(seed)
    out = []
    for b, seq in enumerate(ids):
        used = slots if all_on or b % 2 == 0 else slots - 3
        rows = np.sort(rng.integers(1, len(seq), size=used))
        mask = np.ones(used, np.float32) if all_on else np.array([0.0 if k % 4 == 3 else 1.0 for k in range(used)],
                                                                   np.float32)
        out.append(pack_markers(rows, mask, np.arange(used) // 2 if not all_on else None, slots))
    return out


def oracle(spec, head, W, L, ids, packed, qtypes=None):
    from oracle.oracle import OracleRuntime
    plan = build_plan(spec, head, L, 1, False)
    p = OracleRuntime(W, [plan]).plan(plan, threads=8)
    table = W["embeddings.word.weight"]
    outs = []
    for b, (seq, mk) in enumerate(zip(ids, packed)):
        ri = inputs.run_input(spec, table, [seq], L)
        if qtypes is None:
            p.upload(ri["embeddings"], ri["mask"], None, mk)
        else:
            p.upload(ri["embeddings"], ri["mask"], None, mk, qtypes[b])
        p.run(len(seq))
        outs.append(p.read_output())
    return np.stack(outs)


def hip(spec, head, W, L, ids, packed, f16, qtypes=None):
    from kleinhirn_amd.backend import HipBackend
    Ws = configs.storage(W, f16)
    be = HipBackend(Ws)
    B = len(ids)
    try:
        plan = build_plan(spec, head, L, B, f16)
        be.check(plan)
        r = be.runner(plan)
        ri = inputs.run_input(spec, Ws["embeddings.word.weight"], ids, L)
        ri["packedMarkers"] = np.concatenate(packed)
        if qtypes is not None:
            ri["qtype"] = list(qtypes)
        r.upload(ri)
        r.run(L * B)
        out = r.read_output().reshape(B, -1)
        r.destroy()
        return out
    finally:
        be.dispose()


@pytest.mark.parametrize("L,lengths", [(512, [480, 301, 77]), (1280, [1280, 333])], ids=["L512", "L1280"])
def test_gliner_base_traced_plan_matches_oracle(L, lengths):
    spec, head = gliner_base()
    W = seeded_weights(spec, head)
    ids = sequences(lengths, 31 + L)
    packed = payloads(ids, head["markers"], 5)
    ref = oracle(spec, head, W, L, ids, packed)
    K = head["markers"]
    masked = np.stack([mk[K:2 * K].view(np.float32) <= 0.5 for mk in packed])
    for f16, tol in ((False, 1e-3), (True, 2e-2)):
        got = hip(spec, head, W, L, ids, packed, f16)
        d = np.abs(got - ref).max()
        print(f"GLiNER-base L{L} {'f16' if f16 else 'f32'}: max |d| {d:.3e}")
        assert d <= tol, d
        assert np.all(got[masked] == -1e4) and np.all(ref[masked] == -1e4)


def test_julia_1_traced_plan_matches_oracle():
    spec, head = julia_1()
    W = seeded_weights(spec, head)
    L = 512
    ids = sequences([500, 260, 130], 97)
    packed = payloads(ids, head["options"], 9, all_on=True)
    qtypes = [0, 1, 2]
    ref = oracle(spec, head, W, L, ids, packed, qtypes)
    for f16, tol in ((False, 1e-3), (True, 2e-2)):
        got = hip(spec, head, W, L, ids, packed, f16, qtypes)
        d = np.abs(got - ref).max()
        print(f"Julia-1 L{L} {'f16' if f16 else 'f32'}: max |d| {d:.3e}")
        assert d <= tol, d
