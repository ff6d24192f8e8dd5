"""The two-stream split of small batches: below KH_SPLIT_T valid rows (and from KH_SPLIT_MIN) the
runner moves the second half of the sequences to a twin plan on its own stream and merges the
outputs. The golden cases hold fewer rows than the default minimum, so these tests lower it to 1 and
require the split run to equal the one-stream run (KH_NO_SPLIT=1) of the same upload, and both the
oracle's bars: pooled and token heads, host rows and device ids, and gather markers that move with
their sequences."""
from __future__ import annotations

import numpy as np
import pytest

from kleinhirn_amd import configs, inputs
from kleinhirn_amd.plan.build import build_plan
from tests.test_gpu_models import case_and_oracle, check_f32, decision_parity, token_case, token_oracle

pytestmark = pytest.mark.gpu


def both(monkeypatch, fn):
    """fn() with the split forced on, then with the split switched off; the split run must have
    used two streams, the other one."""
    monkeypatch.delenv("KH_NO_SPLIT", raising=False)
    monkeypatch.setenv("KH_SPLIT_MIN", "1")
    split, s_streams = fn()
    monkeypatch.setenv("KH_NO_SPLIT", "1")
    whole, w_streams = fn()
    assert (s_streams, w_streams) == (2, 1)
    return split, whole


def same(split, whole, f16=True):
    """Each half computes its sequences' rows as the whole batch does: f16 plans bit-identically
    (the batch-versus-single-plan identity); f32 plans pick their GEMM tiles by row count, and
    tiles of another width sum K in another order, so they agree to f32 rounding."""
    if f16:
        assert np.array_equal(split, whole), np.abs(split - whole).max()
    else:
        assert np.abs(split - whole).max() <= 1e-5, np.abs(split - whole).max()


def run_case(case, f16, by_ids=False, markers=None):
    from kleinhirn_amd.backend import HipBackend
    W = configs.storage(case.weights, f16)
    be = HipBackend(W)
    table = W["embeddings.word.weight"]
    B, L = len(case.ids), case.length
    plan = build_plan(case.spec, case.head, L, B, f16)
    r = be.runner(plan)
    if markers is not None:
        r.init_buffer("first", markers.tobytes())
    if by_ids:
        be.set_words(table)
        mask, tt = inputs.mask_and_types(case.spec, case.ids, L)
        ids = np.zeros(L * B, dtype=np.int32)
        for b, seq in enumerate(case.ids):
            ids[b * L:b * L + len(seq)] = seq
        r.upload_ids(ids, mask, tt)
    else:
        r.upload(inputs.run_input(case.spec, table, case.ids, L))
    r.run(L * B)
    out = r.read_output().reshape(B, -1)
    streams = r.info.streams
    # a second run of the same upload reuses the memoised split and the staged twin
    r.run(L * B)
    again = r.read_output().reshape(B, -1)
    assert np.array_equal(out, again)
    r.destroy()
    be.dispose()
    return out, streams


@pytest.mark.parametrize("key", ["c2", "c3b", "c5"])
@pytest.mark.parametrize("by_ids", [False, True], ids=["rows", "ids"])
def test_split_pooled_heads(monkeypatch, key, by_ids):
    case, ref = case_and_oracle(key)
    split, whole = both(monkeypatch, lambda: run_case(case, True, by_ids))
    same(split, whole)
    d = decision_parity(ref, split)
    assert d["mismatched"] == 0, d
    assert d["delta"] <= 2e-2, d


def test_split_f32_matches_oracle(monkeypatch):
    case, ref = case_and_oracle("c2")
    split, whole = both(monkeypatch, lambda: run_case(case, False))
    same(split, whole, f16=False)
    check_f32("c2", ref, split)


def test_split_token_head(monkeypatch):
    """Token rows of the twin's sequences land at (split + j) * L + i of the merged output."""
    case = token_case()
    split, whole = both(monkeypatch, lambda: run_case(case, False))
    same(split, whole, f16=False)
    got = split.reshape(len(case.ids), case.length, -1)
    for b, r in enumerate(token_oracle(case)):
        assert np.abs(r - got[b, :len(r)]).max() <= 1e-3
        assert not got[b, len(r):].any()


def test_split_moves_gather_markers(monkeypatch):
    """A marker of a sequence in the second half reaches the twin at that sequence's slot."""
    case, ref = case_and_oracle("c2")
    B = len(case.ids)
    moved = np.zeros(3 * B, dtype=np.uint32)
    moved[3 * (B - 2)] = 2  # sequence B - 2 (second half) takes its row 2
    split, whole = both(monkeypatch, lambda: run_case(case, True, markers=moved))
    same(split, whole)
    base, _ = run_case(case, True)
    # the unmoved sequences keep the oracle's decisions
    d = decision_parity(np.delete(ref, B - 2, axis=0), np.delete(split, B - 2, axis=0))
    assert d["mismatched"] == 0 and d["delta"] <= 2e-2, d
    assert not np.allclose(whole[B - 2], base[B - 2])
    assert np.array_equal(np.delete(whole, B - 2, axis=0), np.delete(base, B - 2, axis=0))


def test_twin_allocation_failure_runs_whole(monkeypatch):
    """A twin whose buffers cannot be allocated (forced with KH_TWIN_MAX_BYTES=0) is a clean
    KH_ENOMEM inside the library: the plan runs the batch whole on one stream from then on, with
    the one-stream result, and the oracle's bars still hold."""
    case, ref = case_and_oracle("c2")
    monkeypatch.delenv("KH_NO_SPLIT", raising=False)
    monkeypatch.setenv("KH_SPLIT_MIN", "1")
    monkeypatch.setenv("KH_TWIN_MAX_BYTES", "0")
    capped, streams = run_case(case, True)
    assert streams == 1
    monkeypatch.delenv("KH_TWIN_MAX_BYTES")
    monkeypatch.setenv("KH_NO_SPLIT", "1")
    whole, _ = run_case(case, True)
    assert np.array_equal(capped, whole)
    d = decision_parity(ref, capped)
    assert d["mismatched"] == 0 and d["delta"] <= 2e-2, d


def test_split_replaces_changed_markers_between_runs(monkeypatch):
    """New gather markers between two runs of one plan reach the twin's half: the table write
    waits for the twin's queued kernels, and the second run reads the new markers."""
    from kleinhirn_amd.backend import HipBackend
    case, _ = case_and_oracle("c2")
    monkeypatch.delenv("KH_NO_SPLIT", raising=False)
    monkeypatch.setenv("KH_SPLIT_MIN", "1")
    W = configs.storage(case.weights, True)
    be = HipBackend(W)
    B, L = len(case.ids), case.length
    r = be.runner(build_plan(case.spec, case.head, L, B, True))
    r.upload(inputs.run_input(case.spec, W["embeddings.word.weight"], case.ids, L))
    r.run(L * B)
    first = r.read_output().reshape(B, -1)
    moved = np.zeros(3 * B, dtype=np.uint32)
    moved[3 * (B - 1)] = 3
    r.run(L * B)                       # queued, not read: the write below must wait for it
    r.init_buffer("first", moved.tobytes())
    r.upload(inputs.run_input(case.spec, W["embeddings.word.weight"], case.ids, L))
    r.run(L * B)
    second = r.read_output().reshape(B, -1)
    assert r.info.streams == 2
    r.destroy()
    be.dispose()
    assert np.array_equal(first[:B - 1], second[:B - 1])
    assert not np.allclose(first[B - 1], second[B - 1])
