"""Whole plans under masks that are not 0/1 prefixes (holes, fractional values, a masked first
row, a value of 0.4 past the last key), against the oracle, which restates the reference's rule
(src/wasm/plan.ts:573-582 keys and queries above 0.5, :474-495 the mask-weighted mean,
layernorm/embln MASKMUL). Families: BERT mean pooling in f32 (MiniLM, c1), DeBERTa-v3 with the
mask-multiplied embedding LayerNorm and a CLS head (c3b shape at 2 layers), and polyBERT's
DeBERTa-v2 with absolute positions, MASKMUL in the embedding and mean pooling. Bars: f32 within
1e-3 and cosine >= 0.9999; f16 cosine >= 0.999."""
from __future__ import annotations

import numpy as np
import pytest

from kleinhirn_amd import configs, inputs
from kleinhirn_amd.plan.build import build_plan
from tests.helpers import cosine_rows, workload_case
from tests.test_gpu_head_dims import polybert_case
from tests.test_gpu_ops import holed_mask

pytestmark = pytest.mark.gpu


def with_masks(case):
    L = case.length
    lens = [len(x) for x in case.ids]
    return holed_mask(L, lens, 11)


def oracle_masked(case, mask):
    from oracle.oracle import OracleRuntime
    L = case.length
    plan = build_plan(case.spec, case.head, L, 1, False)
    p = OracleRuntime(case.weights, [plan]).plan(plan, threads=8)
    table = case.weights["embeddings.word.weight"]
    outs = []
    for b, seq in enumerate(case.ids):
        ri = inputs.run_input(case.spec, table, [seq], L)
        m = mask[b * L:(b + 1) * L]
        nz = np.nonzero(m)[0]
        p.upload(ri["embeddings"], m, ri["typeIds"])
        p.run(int(nz[-1]) + 1 if len(nz) else 1)
        outs.append(p.read_output())
    return np.stack(outs)


def hip_masked(case, mask, f16):
    from kleinhirn_amd.backend import HipBackend
    W = configs.storage(case.weights, f16)
    be = HipBackend(W)
    try:
        B, L = len(case.ids), case.length
        r = be.runner(build_plan(case.spec, case.head, L, B, f16))
        ri = inputs.run_input(case.spec, W["embeddings.word.weight"], case.ids, L)
        ri["mask"] = mask
        r.upload(ri)
        r.run(L * B)
        out = r.read_output().reshape(B, -1)
        r.destroy()
        return out
    finally:
        be.dispose()


CASES = {
    "minilm-mean": lambda: workload_case("c1", 3, 2, 128, 100),
    "deberta-cls": lambda: workload_case("c3b", 4, 2, 128, 120),
    "polybert-mean": lambda: polybert_case(2),
}


@pytest.mark.parametrize("name", list(CASES))
def test_general_masks_match_oracle(name):
    case = CASES[name]()
    mask = with_masks(case)
    assert np.any((mask > 0) & (mask < 1)) and np.any(mask[: case.length] == 0)
    ref = oracle_masked(case, mask)
    got = hip_masked(case, mask, False)
    d = float(np.abs(got - ref).max())
    cos = cosine_rows(ref, got).min()
    print(f"{name} f32: max |d| {d:.2e} min cosine {cos:.7f}")
    assert d <= 1e-3 and cos >= 0.9999
    if name != "minilm-mean":
        got16 = hip_masked(case, mask, True)
        cos16 = cosine_rows(ref, got16).min()
        print(f"{name} f16: min cosine {cos16:.6f}")
        assert cos16 >= 0.999
