"""Julia decision head through the C ABI (kh_upload_qtypes, kh_upload_markers, f32 logits)
against the oracle on the same seeded encoder, weights, payloads and qtypes. Bars: f32 logits
within 1e-3, masked slots exactly -1e4, f16 within 2e-2; a batch plan equals single plans; a
qtype past the type table is an error; the option probabilities after the head within 1e-3."""
from __future__ import annotations

import numpy as np
import pytest

from kleinhirn_amd import configs, inputs
from kleinhirn_amd.plan.build import build_plan
from tests import julia_case as J

pytestmark = pytest.mark.gpu

_ref = {}


def reference():
    if not _ref:
        ids, W = J.case(3)
        packed, qtypes = J.payloads(ids)
        _ref["v"] = (ids, W, packed, qtypes, J.oracle_logits(ids, W, packed, qtypes))
    return _ref["v"]


def hip_logits(ids, W, packed, qtypes, f16, batch_plan=True):
    from kleinhirn_amd.backend import HipBackend
    S = configs.storage(W, f16)
    be = HipBackend(S)
    table = S["embeddings.word.weight"]
    try:
        if batch_plan:
            r = be.runner(build_plan(J.SPEC, J.HEAD, J.LENGTH, len(ids), f16))
            ri = inputs.run_input(J.SPEC, table, ids, J.LENGTH)
            ri["packedMarkers"] = np.concatenate(packed)
            ri["qtype"] = qtypes
            r.upload(ri)
            r.run(J.LENGTH * len(ids))
            out = r.read_output().reshape(len(ids), -1)
            r.destroy()
            return out
        r = be.runner(build_plan(J.SPEC, J.HEAD, J.LENGTH, 1, f16))
        outs = []
        for seq, mk, q in zip(ids, packed, qtypes):
            ri = inputs.run_input(J.SPEC, table, [seq], J.LENGTH)
            ri["packedMarkers"] = mk
            ri["qtype"] = q
            r.upload(ri)
            r.run(len(seq))
            outs.append(r.read_output())
        r.destroy()
        return np.stack(outs)
    finally:
        be.dispose()


def masked(packed):
    return np.stack([mk[J.OPTIONS:2 * J.OPTIONS].view(np.float32) <= 0.5 for mk in packed])


@pytest.mark.parametrize("batch_plan", [True, False], ids=["batch", "single"])
def test_julia_f32_matches_oracle(batch_plan):
    ids, W, packed, qtypes, ref = reference()
    got = hip_logits(ids, W, packed, qtypes, False, batch_plan)
    m = masked(packed)
    assert m.any() and np.all(got[m] == np.float32(-1e4))
    assert np.abs(got[~m] - ref[~m]).max() <= 1e-3, np.abs(got[~m] - ref[~m]).max()


def test_julia_option_probabilities():
    """The step after the head (src/julia.ts:224-227): softmaxPrefix over each sequence's first
    min(markers, options) logits, kh_scores KH_SCORES_OPTIONS on the HIP logits against the oracle's
    restatement on the oracle logits."""
    from kleinhirn_amd import backend as B
    from oracle import postprocess as P
    ids, W, packed, qtypes, ref = reference()
    got = hip_logits(ids, W, packed, qtypes, False)
    m = masked(packed)
    for i in range(len(ids)):
        valid = int((~m[i]).sum())
        assert valid > 0 and not m[i, :valid].any(), "the live slots are a prefix"
        probs, label = B.scores(got[i, :valid], B.SCORES_OPTIONS)
        want = np.array(P.softmax_prefix(ref[i, :valid].tolist()), np.float32)
        assert np.abs(probs[0] - want).max() <= 1e-3 and abs(float(probs[0].sum()) - 1) < 1e-5
        assert label[0] == int(np.argmax(want)) or np.sort(want)[-1] - np.sort(want)[-2] < 1e-3


def test_julia_f16_matches_oracle_and_single_plans():
    ids, W, packed, qtypes, ref = reference()
    got = hip_logits(ids, W, packed, qtypes, True)
    m = masked(packed)
    d = np.abs(got[~m] - ref[~m]).max()
    print(f"julia f16: max |dlogit| {d:.5f}")
    assert d <= 2e-2 and np.all(got[m] == np.float32(-1e4))
    assert np.array_equal(got, hip_logits(ids, W, packed, qtypes, True, batch_plan=False))


def test_qtype_selects_rows_and_is_checked():
    from kleinhirn_amd.backend import HipBackend, KhError
    ids, W, packed, qtypes, _ = reference()
    S = configs.storage(W, True)
    be = HipBackend(S)
    try:
        r = be.runner(build_plan(J.SPEC, J.HEAD, J.LENGTH, 1, True))
        ri = inputs.run_input(J.SPEC, S["embeddings.word.weight"], [ids[0]], J.LENGTH)
        ri["packedMarkers"] = packed[0]
        outs = []
        for q in (0, 1, None):
            ri["qtype"] = q
            r.upload(ri)
            r.run(len(ids[0]))
            outs.append(r.read_output())
        assert not np.array_equal(outs[0], outs[1]) and np.array_equal(outs[0], outs[2])
        ri["qtype"] = 3
        r.upload(ri)
        with pytest.raises(KhError, match="qtype 3"):
            r.run(len(ids[0]))
        r.destroy()
    finally:
        be.dispose()
