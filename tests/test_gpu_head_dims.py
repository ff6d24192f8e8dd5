"""Head dimensions other than 32 and 64 through a whole plan: the polyBERT shape (DeBERTa-v2 without
relative attention, hidden 600 over 12 heads: D = 50, intermediate 512, absolute positions, a
269-row vocabulary; data/k28/models.json of the reference, xushijie/polyBERT) with a mean-pooled
embedding head, against the oracle on seeded weights and ragged ids. Bars: f32 cosine >= 0.9999
and |d| <= 1e-3; f16 cosine >= 0.999."""
from __future__ import annotations

import numpy as np
import pytest

from kleinhirn_amd.plan import spec as S
from tests.helpers import Case, cosine_rows, hip_outputs, oracle_outputs

pytestmark = pytest.mark.gpu


def polybert_case(layers: int = 12) -> Case:
    spec = S.deberta_v2_absolute(600, layers, 12, 512, 269)
    head = S.embed_head("mean")
    rng = np.random.default_rng(271)
    ids = []
    for n in (60, 17, 128, 3):
        seq = rng.integers(5, 269, size=n)
        seq[0], seq[-1] = 2, 3
        ids.append(seq)
    return Case(spec, head, ids, 128)


def test_polybert_head_dim_50_matches_oracle():
    c = polybert_case()
    ref = oracle_outputs(c)
    got32 = hip_outputs(c, False)
    cos = cosine_rows(ref, got32)
    d = float(np.abs(got32 - ref).max())
    print(f"polyBERT f32: min cosine {cos.min():.7f} max |d| {d:.2e}")
    assert cos.min() >= 0.9999 and d <= 1e-3
    got16 = hip_outputs(c, True)
    cos16 = cosine_rows(ref, got16)
    print(f"polyBERT f16: min cosine {cos16.min():.6f}")
    assert cos16.min() >= 0.999
