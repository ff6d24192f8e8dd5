"""GLiNER2 span head on the CPU: the plan the builder makes (src/plan/build.ts:358-377, 432-526),
the oracle's masklogits against the kernel's definition (src/kernels/masklogits.wgsl), and the
head's composition (gather at the marker rows, fc1 + ReLU, fc2, masked logits / temperature)
against a float64 restatement over the oracle's own final hidden states."""
from __future__ import annotations

import ctypes
import json

import numpy as np
import pytest

from kleinhirn_amd import inputs
from kleinhirn_amd.plan.build import build_plan, pack_markers, plan_json
from tests import gliner_case as G


def test_plan_layout():
    c, _ = G.case(1)
    p = build_plan(c.spec, G.HEAD, 128, 2, False)
    K = 8 * 2
    ops = p["segments"][-1]["ops"]
    assert [o["kernel"] for o in ops] == ["gather", "matmul", "matmul", "masklogits"]
    assert ops[0]["constants"] == {"K": 8, "D": 768, "L": 128} and ops[0]["bind"] == ["packed", "x", "states"]
    assert ops[1]["constants"] == {"M": K, "N": 768, "K": 768, "ACT": 1} and ops[1]["dispatch"] == [48, 1]
    assert ops[2]["constants"] == {"M": K, "N": 1, "K": 768, "ACT": 0}
    assert ops[3]["constants"] == {"K": 8, "TEMP": 0.5} and ops[3]["bind"] == ["raw", "packed", "logits"]
    size = {d["id"]: d["bytes"] for d in p["buffers"]}
    assert size["states"] == K * 768 * 4 and size["h1"] == K * 768 * 4 and size["raw"] == K * 4
    assert size["packed"] == 3 * K * 4 and size["logits"] == K * 4
    assert next(d for d in p["buffers"] if d["id"] == "logits")["usage"] == "logits"
    assert p["inputs"] == {"embeddings": "emb", "mask": "mask", "markers": "packed"}
    assert p["output"] == {"buffer": "logits", "bytes": K * 4, "dtype": "f32", "rows": K, "cols": 1}
    assert p["markers"] == 8
    # f16 storage keeps the f32 logits buffer
    p16 = build_plan(c.spec, G.HEAD, 128, 2, True)
    assert {d["id"]: d["bytes"] for d in p16["buffers"]}["logits"] == K * 4
    assert {d["id"]: d["bytes"] for d in p16["buffers"]}["raw"] == K * 2


def test_pack_markers_layout():
    mk = pack_markers([3, 9], [1.0, 0.0], [0, 1], markers=4)
    assert mk.dtype == np.uint32 and mk.size == 12
    assert list(mk[:4]) == [3, 9, 0, 0]
    assert list(mk[4:8].view(np.float32)) == [1.0, 0.0, 0.0, 0.0]
    assert list(mk[8:]) == [0, 1, 0, 0]
    with pytest.raises(ValueError):
        pack_markers([1, 2, 3], [1, 1, 1], markers=2)


def test_oracle_masklogits_matches_definition():
    """One op record on random raw values and payloads, with mask words at, below and above the
    0.5 threshold, negative, NaN-free; two sequences of K = 5."""
    from oracle.oracle import CODE, KhoOp, lib
    rng = np.random.default_rng(3)
    K, B, temp = 5, 2, 0.7
    raw = rng.normal(size=K * B).astype(np.float32)
    packed = np.zeros(3 * K * B, dtype=np.uint32)
    masks = np.array([1.0, 0.5, 0.5000001, 0.0, -2.0, 2.0, 0.49, 1.0, 0.0, 0.75], dtype=np.float32)
    for b in range(B):
        packed[b * 3 * K:b * 3 * K + K] = rng.integers(0, 100, size=K)
        packed[b * 3 * K + K:b * 3 * K + 2 * K] = masks[b * K:(b + 1) * K].view(np.uint32)
    out = np.full(K * B + 16, 7.0, dtype=np.float32)
    op = KhoOp()
    op.code, op.rows_fixed = CODE["masklogits"], -1
    op.p[0], op.p[1], op.p[2] = raw.ctypes.data, packed.ctypes.data, out.ctypes.data
    op.v[0], op.v[1] = K, K * B
    op.f[0] = temp
    mask = np.zeros(128, dtype=np.float32)
    kinfo = np.zeros(64, dtype=np.int32)
    scratch = np.zeros(16, dtype=np.float32)
    ops = (KhoOp * 1)(op)
    assert lib().kho_run(ops, 1, 128, 1, mask.ctypes.data, kinfo.ctypes.data, scratch.ctypes.data, 0, 1, 1,
                         16, 64, 32, 1 << 16) == 0
    want = np.where(masks > 0.5, raw / np.float32(temp), np.float32(-1e4)).astype(np.float32)
    assert np.array_equal(out[:K * B], want)
    assert np.all(out[K * B:] == 7.0)


def test_head_composition_over_oracle_states():
    """logits[k] = (relu(x[m_k] W1^T + b1) W2^T + b2) / T or -1e4, in float64 over the oracle's
    final hidden states x, equals the oracle's f32 logits to f32 rounding."""
    from oracle.oracle import OracleRuntime
    c, W = G.case(2)
    packed = G.payloads(c.ids)
    plan = build_plan(c.spec, G.HEAD, G.LENGTH, 1, False)
    p = OracleRuntime(W, [plan]).plan(plan, threads=8)
    table = W["embeddings.word.weight"]
    K = G.HEAD["markers"]
    for seq, mk in zip(c.ids, packed):
        ri = inputs.run_input(c.spec, table, [seq], G.LENGTH)
        p.upload(ri["embeddings"], ri["mask"], None, mk)
        p.run(len(seq))
        got = p.read_output()
        x = p.view("x").reshape(G.LENGTH, -1)[:, :768].astype(np.float64)
        states = x[mk[:K]]
        h1 = np.maximum(states @ W["head.fc1.weight"].astype(np.float64).T + W["head.fc1.bias"], 0)
        raw = h1 @ W["head.fc2.weight"].astype(np.float64).T + W["head.fc2.bias"]
        m = mk[K:2 * K].view(np.float32)
        want = np.where(m > 0.5, raw[:, 0] / G.HEAD["temperature"], -1e4)
        assert np.abs(got - want).max() <= 1e-4, np.abs(got - want).max()
        assert np.array_equal(got[m <= 0.5], np.full((m <= 0.5).sum(), -1e4, dtype=np.float32))


def test_plan_check_accepts_marker_heads():
    from kleinhirn_amd import backend as B
    c, _ = G.case(1)
    doc = json.dumps(plan_json(build_plan(c.spec, G.HEAD, 128, 2, True))).encode()
    assert B.lib().kh_plan_check(None, doc, len(doc)) == 0, B.lib().kh_last_error()
