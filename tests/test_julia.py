"""Julia decision head on the CPU: the plan the builder makes (src/plan/build.ts:378-430, the
rowSelect and typeRow buffer of 432-526), the oracle's type-row selection and MODE 1 add
(src/plan/wasm.ts:429-439, src/wasm/plan.ts:452-464) by the difference two qtypes make, and the
scorer's composition (gather, LayerNorm, fc1 + GELU, fc2, masklogits) against float64 over the
oracle's own head-stream states."""
from __future__ import annotations

import json

import numpy as np

from kleinhirn_amd import inputs
from kleinhirn_amd.plan import spec as S
from kleinhirn_amd.plan.build import build_plan, plan_json
from tests import julia_case as J


def test_plan_layout():
    p = build_plan(J.SPEC, J.HEAD, J.LENGTH, 2, True)
    names = [s["name"] for s in p["segments"]]
    assert names[-4:] == ["typed", "head0", "head1", "scorer"] and names[-5] == "final"
    typed = p["segments"][-4]["ops"]
    assert typed[0]["kernel"] == "add" and typed[0]["bind"] == ["tmp", "typeRow"]
    assert typed[0]["constants"] == {"TOTAL": J.LENGTH * 2 * 384, "N": 384, "MODE": 1, "L": J.LENGTH}
    h0 = {o["name"]: o for o in p["segments"][-3]["ops"]}
    assert h0["lnA"]["bind"][0] == "tmp" and h0["lnA"]["bind"][2] == "w:head.0.norm1.weight"
    assert h0["qkv"]["bind"][1:3] == ["w:head.0.in_proj.weight", "w:head.0.in_proj.bias"]
    assert h0["lin1"]["constants"]["N"] == 768 and h0["lin1"]["constants"]["ACT"] == 1
    assert "rope" not in h0
    sc = p["segments"][-1]["ops"]
    assert [o["kernel"] for o in sc] == ["gather", "layernorm", "matmul", "matmul", "masklogits"]
    K = J.OPTIONS * 2
    assert sc[1]["dispatch"] == [K, 1] and sc[2]["constants"]["ACT"] == 2 and sc[4]["constants"]["TEMP"] == 1.0
    assert p["rowSelect"] == {"table": "w:type_emb.weight", "dst": "typeRow", "rowBytes": 384 * 2}
    size = {d["id"]: d["bytes"] for d in p["buffers"]}
    assert size["typeRow"] == 2 * 384 * 2 and size["kNormed"] == K * 384 * 2 and size["logits"] == K * 4
    assert p["markers"] == J.OPTIONS and p["output"]["dtype"] == "f32"


def test_oracle_type_row_is_added_to_every_row():
    """With no head layers, the head stream after the run is final_norm(x) + type_emb[qtype] on
    every valid row: two runs differing in qtype differ by the difference of the two type rows."""
    from oracle.oracle import OracleRuntime
    ids, W = J.case(3)
    head = dict(J.HEAD, layers=0)
    plan = build_plan(J.SPEC, head, J.LENGTH, 1, False)
    p = OracleRuntime(W, [plan]).plan(plan, threads=8)
    seq = ids[0]
    ri = inputs.run_input(J.SPEC, W["embeddings.word.weight"], [seq], J.LENGTH)
    mk = J.payloads(ids)[0][0]
    rows = []
    for q in (0, 2):
        p.upload(ri["embeddings"], ri["mask"], None, mk, q)
        p.run(len(seq))
        rows.append(p.view("tmp").reshape(J.LENGTH, -1)[:len(seq), :384].astype(np.float64))
    te = W["type_emb.weight"].astype(np.float64)
    assert np.abs((rows[1] - rows[0]) - (te[2] - te[0])).max() <= 1e-5


def test_scorer_composition_over_oracle_states():
    from oracle.oracle import OracleRuntime
    ids, W = J.case(3)
    packed, qtypes = J.payloads(ids)
    plan = build_plan(J.SPEC, J.HEAD, J.LENGTH, 1, False)
    p = OracleRuntime(W, [plan]).plan(plan, threads=8)
    K = J.OPTIONS
    for seq, mk, q in zip(ids[:2], packed, qtypes):
        ri = inputs.run_input(J.SPEC, W["embeddings.word.weight"], [seq], J.LENGTH)
        p.upload(ri["embeddings"], ri["mask"], None, mk, q)
        p.run(len(seq))
        got = p.read_output()
        tmp = p.view("tmp").reshape(J.LENGTH, -1)[:, :384].astype(np.float64)
        st = tmp[mk[:K]]
        mean = st.mean(1, keepdims=True)
        var = ((st - mean) ** 2).mean(1, keepdims=True)
        kn = (st - mean) / np.sqrt(var + J.SPEC["block"]["norm"]["eps"]) * W["scorer.norm.weight"] + W["scorer.norm.bias"]
        h = kn @ W["scorer.fc1.weight"].astype(np.float64).T + W["scorer.fc1.bias"]
        from scipy.special import erf
        h = 0.5 * h * (1 + erf(h / np.sqrt(2)))
        raw = (h @ W["scorer.fc2.weight"].astype(np.float64).T + W["scorer.fc2.bias"])[:, 0]
        m = mk[K:2 * K].view(np.float32)
        want = np.where(m > 0.5, raw, -1e4)
        assert np.abs(got - want).max() <= 1e-4, np.abs(got - want).max()


def test_plan_check_accepts_the_julia_head():
    from kleinhirn_amd import backend as B
    doc = json.dumps(plan_json(build_plan(J.SPEC, J.HEAD, J.LENGTH, 2, True))).encode()
    assert B.lib().kh_plan_check(None, doc, len(doc)) == 0, B.lib().kh_last_error()
    assert S.JULIA_TYPES == 3
