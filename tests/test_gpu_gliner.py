"""GLiNER2 span head through the C ABI (kh_upload_markers, the f32 logits output) against the
oracle on the same seeded DeBERTa-v3 encoder, weights and marker payloads. Bars: f32 logits within
1e-3 (logits / temperature 0.5); masked slots exactly -1e4; f16 logits within f16 storage rounding
of the encoder states (2e-2 at O(0.1-1) logits)."""
from __future__ import annotations

import numpy as np
import pytest

from kleinhirn_amd import configs, inputs
from kleinhirn_amd.plan.build import build_plan
from tests import gliner_case as G

pytestmark = pytest.mark.gpu

_ref = {}


def reference():
    if not _ref:
        c, W = G.case(3)
        packed = G.payloads(c.ids)
        _ref["v"] = (c, W, packed, G.oracle_logits(c, W, packed))
    return _ref["v"]


def hip_logits(c, W, packed, f16, batch_plan=True, by_ids=False):
    from kleinhirn_amd.backend import HipBackend
    S = configs.storage(W, f16)
    be = HipBackend(S)
    table = S["embeddings.word.weight"]
    B = len(c.ids)
    try:
        if batch_plan:
            r = be.runner(build_plan(c.spec, G.HEAD, G.LENGTH, B, f16))
            if by_ids:
                be.set_words(table)
                mask, _ = inputs.mask_and_types(c.spec, c.ids, G.LENGTH)
                ids = np.zeros(G.LENGTH * B, dtype=np.int32)
                for b, seq in enumerate(c.ids):
                    ids[b * G.LENGTH:b * G.LENGTH + len(seq)] = seq
                r.upload_ids(ids, mask, None, np.concatenate(packed))
            else:
                ri = inputs.run_input(c.spec, table, c.ids, G.LENGTH)
                ri["packedMarkers"] = np.concatenate(packed)
                r.upload(ri)
            r.run(G.LENGTH * B)
            out = r.read_output().reshape(B, -1)
            r.destroy()
            return out
        r = be.runner(build_plan(c.spec, G.HEAD, G.LENGTH, 1, f16))
        outs = []
        for seq, mk in zip(c.ids, packed):
            ri = inputs.run_input(c.spec, table, [seq], G.LENGTH)
            ri["packedMarkers"] = mk
            r.upload(ri)
            r.run(len(seq))
            outs.append(r.read_output())
        r.destroy()
        return np.stack(outs)
    finally:
        be.dispose()


def masked(packed):
    K = G.HEAD["markers"]
    return np.stack([mk[K:2 * K].view(np.float32) <= 0.5 for mk in packed])


@pytest.mark.parametrize("batch_plan", [True, False], ids=["batch", "single"])
def test_gliner_f32_matches_oracle(batch_plan):
    c, W, packed, ref = reference()
    got = hip_logits(c, W, packed, False, batch_plan)
    m = masked(packed)
    assert np.all(got[m] == np.float32(-1e4)) and np.all(ref[m] == np.float32(-1e4))
    assert np.abs(got[~m] - ref[~m]).max() <= 1e-3, np.abs(got[~m] - ref[~m]).max()


def test_gliner_f16_matches_oracle_and_single_plans():
    c, W, packed, ref = reference()
    got = hip_logits(c, W, packed, True)
    m = masked(packed)
    assert np.all(got[m] == np.float32(-1e4))
    d = np.abs(got[~m] - ref[~m]).max()
    print(f"gliner f16: max |dlogit| {d:.5f}")
    assert d <= 2e-2
    assert np.array_equal(got, hip_logits(c, W, packed, True, batch_plan=False))
    assert np.array_equal(got, hip_logits(c, W, packed, True, by_ids=True))


def test_marker_payloads_replace_and_reject():
    """A new payload changes only the slots it changes; a row past the plan length, a payload of
    the wrong size and markers for a plan without a markers input are errors."""
    from kleinhirn_amd.backend import HipBackend, KhError
    c, W, packed, _ = reference()
    S = configs.storage(W, True)
    be = HipBackend(S)
    try:
        B = len(c.ids)
        r = be.runner(build_plan(c.spec, G.HEAD, G.LENGTH, B, True))
        ri = inputs.run_input(c.spec, S["embeddings.word.weight"], c.ids, G.LENGTH)
        ri["packedMarkers"] = np.concatenate(packed)
        r.upload(ri)
        r.run(G.LENGTH * B)
        a = r.read_output().reshape(B, -1)
        K = G.HEAD["markers"]
        moved = [mk.copy() for mk in packed]
        moved[1][0] = (moved[1][0] + 1) % len(c.ids[1])
        moved[1][K] = np.float32(1.0).view(np.uint32)
        r._markers(np.concatenate(moved))
        r.run(G.LENGTH * B)
        b = r.read_output().reshape(B, -1)
        assert b[1, 0] != a[1, 0]
        keep = np.ones_like(a, dtype=bool)
        keep[1, 0] = False
        assert np.array_equal(a[keep], b[keep])
        bad = np.concatenate(packed)
        bad[0] = G.LENGTH
        r._markers(bad)
        with pytest.raises(KhError, match="plan length"):
            r.run(G.LENGTH * B)
        with pytest.raises(KhError, match="packed markers"):
            r._markers(np.concatenate(packed + [packed[0][:1]]))
        # a shorter payload replaces only its own values (the reference's put at offset 0)
        r._markers(np.concatenate(packed))
        r._markers(np.concatenate(moved)[:3 * K])
        r.run(G.LENGTH * B)
        short = r.read_output().reshape(B, -1)
        assert np.array_equal(short, a)
        with pytest.raises(ValueError, match="packedMarkers"):
            r.upload({k: v for k, v in ri.items() if k != "packedMarkers"})
        r.destroy()
        from kleinhirn_amd.plan import spec as SP
        pooled = be.runner(build_plan(c.spec, SP.embed_head("cls", normalize=False), G.LENGTH, 1, True))
        from kleinhirn_amd.backend import lib
        arr = np.zeros(3, dtype=np.uint32)
        assert lib().kh_upload_markers(pooled.h, arr.ctypes.data, 3) != 0
        pooled.destroy()
    finally:
        be.dispose()


def test_scheduler_rejects_marker_plans():
    """kh_sched runs pooled heads only: a GLiNER2 plan of one marker slot (one output row per
    sequence) is refused, since the scheduler uploads no marker payloads."""
    import ctypes
    from kleinhirn_amd.backend import HipBackend, lib
    c, W, _, _ = reference()
    be = HipBackend(configs.storage(W, True))
    try:
        r = be.runner(build_plan(c.spec, G.HEAD, G.LENGTH, 2, True, markers=1))
        assert r.info.out_rows == 2
        handles = (ctypes.c_void_p * 1)(r.h.value)
        h = ctypes.c_void_p()
        assert lib().kh_sched_create(handles, 1, ctypes.byref(h)) == 2  # KH_EUNSUPPORTED
        assert b"no markers" in lib().kh_last_error()
        r.destroy()
    finally:
        be.dispose()
