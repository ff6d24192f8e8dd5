"""The Node-API path hip-backend.ts uses (kh_addon.node over libkh_hip.so), driven by
tests/node/run_plan.js: structural plan checks on the CPU, and on the GPU the same case as
the Python host, compared bit for bit and against the golden oracle vectors."""
from __future__ import annotations

import os
import shutil
import tempfile

import numpy as np
import pytest

from kleinhirn_amd import configs, inputs
from tests.node_case import ADDON, export_case, run_node
from kleinhirn_amd.plan.build import build_plan

pytestmark = pytest.mark.skipif(shutil.which("node") is None or not os.path.exists(ADDON),
                                reason="node or kh_addon.node missing")


def test_node_addon_checks_every_benchmark_plan():
    for name in ("c2", "c3b", "c4"):
        w = configs.ALL[name]()
        with tempfile.TemporaryDirectory() as d:
            export_case(d, build_plan(w.spec, w.head, w.length, 16, True), check_only=True)
            assert run_node(d)["ok"]


def test_node_addon_reports_unsupported_ops():
    w = configs.c2()
    plan = build_plan(w.spec, w.head, 64, 1, True)
    plan["segments"][0]["ops"][0]["kernel"] = "im2col"
    with tempfile.TemporaryDirectory() as d:
        export_case(d, plan, check_only=True)
        with pytest.raises(RuntimeError, match="im2col"):
            run_node(d)


@pytest.mark.gpu
def test_node_path_matches_python_path_and_golden():
    from tests.helpers import decision_parity, hip_outputs
    from tests.test_gpu_models import case_and_oracle
    case, ref = case_and_oracle("c2")
    W = configs.storage(case.weights, True)
    plan = build_plan(case.spec, case.head, case.length, len(case.ids), True)
    ri = inputs.run_input(case.spec, W["embeddings.word.weight"], case.ids, case.length)
    with tempfile.TemporaryDirectory() as d:
        export_case(d, plan, W, ri, rows=case.length * len(case.ids))
        res = run_node(d)
        got = np.fromfile(os.path.join(d, "out.bin"), dtype=np.float32).reshape(len(case.ids), -1)
    assert res["ok"] and res["info"]["launches"] > 0
    py = hip_outputs(case, f16=True)
    assert np.array_equal(got, py)
    d = decision_parity(ref, got)
    assert d["mismatched"] == 0, d


@pytest.mark.gpu
def test_node_gliner_head_matches_python_path():
    """A GLiNER2 span head through the addon (uploadMarkers, the f32 logits) equals the Python
    host's run of the same plan and payloads."""
    from tests import gliner_case as G
    from tests.test_gpu_gliner import hip_logits
    c, W = G.case(3)
    packed = G.payloads(c.ids)
    S = configs.storage(W, True)
    plan = build_plan(c.spec, G.HEAD, G.LENGTH, len(c.ids), True)
    ri = inputs.run_input(c.spec, S["embeddings.word.weight"], c.ids, G.LENGTH)
    ri["packedMarkers"] = np.concatenate(packed)
    with tempfile.TemporaryDirectory() as d:
        export_case(d, plan, S, ri, rows=G.LENGTH * len(c.ids))
        res = run_node(d)
        got = np.fromfile(os.path.join(d, "out.bin"), dtype=np.float32).reshape(len(c.ids), -1)
    assert res["ok"]
    assert np.array_equal(got, hip_logits(c, W, packed, True))


@pytest.mark.gpu
def test_node_julia_head_matches_python_path():
    """The Julia head through the addon (uploadMarkers, uploadQtypes) equals the Python host."""
    from tests import julia_case as J
    from tests.test_gpu_julia import hip_logits
    ids, W = J.case(3)
    packed, qtypes = J.payloads(ids)
    S = configs.storage(W, True)
    plan = build_plan(J.SPEC, J.HEAD, J.LENGTH, len(ids), True)
    ri = inputs.run_input(J.SPEC, S["embeddings.word.weight"], ids, J.LENGTH)
    ri["packedMarkers"] = np.concatenate(packed)
    ri["qtype"] = qtypes
    with tempfile.TemporaryDirectory() as d:
        export_case(d, plan, S, ri, rows=J.LENGTH * len(ids))
        res = run_node(d)
        got = np.fromfile(os.path.join(d, "out.bin"), dtype=np.float32).reshape(len(ids), -1)
    assert res["ok"]
    assert np.array_equal(got, hip_logits(ids, W, packed, qtypes, True))


def test_node_addon_checks_a_manifest_directory():
    """manifestCheck through the addon reads what kh_manifest_check reads."""
    from kleinhirn_amd import backend as B
    from oracle import manifest_format as MF
    w = configs.c2()
    rng = np.random.default_rng(1)
    weights = {MF.WORDS: rng.standard_normal((50, 16)).astype(np.float32),
               "x.weight": rng.standard_normal((8, 16)).astype(np.float32)}
    with tempfile.TemporaryDirectory() as d:
        path = MF.write_manifest(os.path.join(d, "m"), weights, "f16")
        export_case(d, build_plan(w.spec, w.head, 64, 1, True), check_only=True, manifest=path,
                    manifest_flags=B.LOAD_CHECK_ROWS)
        res = run_node(d)
        want = B.manifest_check(path, B.LOAD_CHECK_ROWS)
    got = res["manifest"]
    assert (got["version"], got["tensors"], got["wordsRows"], got["wordsWidth"]) == (
        want["version"], want["tensors"], want["words_rows"], want["words_width"]) == (3, 1, 50, 16)
    assert got["fileBytes"] == want["file_bytes"]


@pytest.mark.gpu
def test_node_manifest_load_and_device_gather_match_python_path():
    """loadManifest + uploadIds through the addon (weights and word table from the files, rows
    gathered on the device) against the Python host's tensor-by-tensor upload and host gather."""
    from oracle import manifest_format as MF
    from tests.helpers import hip_outputs
    from tests.test_gpu_models import case_and_oracle
    case, ref = case_and_oracle("c2")
    plan = build_plan(case.spec, case.head, case.length, len(case.ids), True)
    mask, tt = inputs.mask_and_types(case.spec, case.ids, case.length)
    ids = np.zeros(case.length * len(case.ids), dtype=np.int32)
    for b, seq in enumerate(case.ids):
        ids[b * case.length:b * case.length + len(seq)] = seq
    with tempfile.TemporaryDirectory() as d:
        path = MF.write_manifest(os.path.join(d, "m"), case.weights, "f16")
        export_case(d, plan, {}, {"embeddings": None, "mask": mask, "typeIds": tt},
                    rows=case.length * len(case.ids), manifest=path, ids=ids)
        res = run_node(d)
        got = np.fromfile(os.path.join(d, "out.bin"), dtype=np.float32).reshape(len(case.ids), -1)
    assert res["ok"] and res["manifest"]["tensors"] > 0
    from tests.helpers import decision_parity
    d = decision_parity(ref, got)
    assert d["mismatched"] == 0 and d["delta"] <= 2e-2, d  # the oracle's bars
    assert np.array_equal(got, hip_outputs(case, f16=True))


def test_node_addon_scores_and_rank_equal_the_oracle():
    import json
    import subprocess
    from oracle import postprocess as P
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((9, 3)) * 3).astype(np.float32)
    code = (f"const a = require({json.dumps(ADDON)});"
            f"const x = new Float32Array({json.dumps(x.ravel().tolist())});"
            "const r = a.scores(x, 3, 0);"
            "console.log(JSON.stringify({s: Array.from(r.scores), i: Array.from(r.index),"
            " o: Array.from(a.rank(new Float32Array([0.25, 3, 0.25, -2, 3])))}));")
    out = subprocess.run(["node", "-e", code], capture_output=True, text=True, timeout=60)
    assert out.returncode == 0, out.stderr
    res = json.loads(out.stdout)
    want, wi = P.scores(x, P.SOFTMAX)
    assert np.array_equal(np.array(res["s"], np.float32).reshape(9, 3), want)
    assert res["i"] == wi.tolist()
    assert res["o"] == [1, 4, 0, 2, 3]


@pytest.mark.gpu
def test_node_scheduler_matches_python_path():
    """schedCreate / schedRun through the addon: two copies of a batch-4 plan run the c2 case in
    length-ordered chunks; outputs equal the Python host's batch plan bit for bit."""
    from tests.node_case import export_sched_case
    from kleinhirn_amd.scheduler import type_words
    from tests.helpers import hip_outputs
    from tests.test_gpu_models import case_and_oracle
    case, ref = case_and_oracle("c2")
    W = configs.storage(case.weights, True)
    words = W.pop("embeddings.word.weight")
    plan = build_plan(case.spec, case.head, case.length, 4, True)
    with tempfile.TemporaryDirectory() as d:
        export_sched_case(d, plan, W, words, case.ids, type_words(case.spec, case.ids), token_budget=700)
        res = run_node(d)
        got = np.fromfile(os.path.join(d, "out.bin"), dtype=np.float32).reshape(len(case.ids), -1)
    assert res["ok"] and res["stats"]["sequences"] == len(case.ids)
    from tests.helpers import decision_parity
    d = decision_parity(ref, got)
    assert d["mismatched"] == 0 and d["delta"] <= 2e-2, d  # the oracle's bars
    assert np.array_equal(got, hip_outputs(case, f16=True))
