"""The plan builder against the reference's frozen dispatch traces.

The reference's gate for its plan executor (tests/plan_trace.test.ts:60-72) requires the dispatch
lists of 125 configurations -- GLiNER small and base (DeBERTa-v2 relative attention, span head)
and Julia-1 (ModernBERT with local/global windows and RoPE, decision head) at L 128/512/1280,
B 1/4, f16 and f32, in normal, 100-row, skip, pass and dispatch profile and capture modes -- to
equal the lists frozen in tests/golden/k28/dispatch-traces.json.gz (a copy of that data file:
tests/golden/k28_dispatch_traces.json.gz, source commit 54bfc4e). tests/plan_trace.py restates
the executor's encoding; here every configuration is built with kleinhirn_amd/plan and compared
event by event: buffer writes and copies, every dispatch's constants, binding list (buffers
numbered by first use, weights by name) and workgroup counts, the buffers' sizes, usages and the
sha256 of their build-time contents (the relidx and RoPE tables), the byte totals and the profile
keys. These are the plan documents the HIP runner executes (kh_plan_create)."""
from __future__ import annotations

import gzip
import json
import os

import pytest

from kleinhirn_amd.plan import spec as S
from kleinhirn_amd.plan.build import build_plan
from tests.plan_trace import (GLINER_HEAD_HIDDEN, GLINER_SPECS, GLINER_TEMPERATURE, JULIA_SPEC, all_configs,
                              first_difference, record)

FROZEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "k28_dispatch_traces.json.gz")


def frozen():
    with gzip.open(FROZEN) as fh:
        return json.loads(fh.read())


def plan_of(cfg):
    if cfg["shape"] == "julia-1":
        j = JULIA_SPEC
        spec, head = S.julia(j["hiddenSize"], j["layers"], j["heads"], j["intermediate"], 0, j["normEps"],
                             j["ropeTheta"], j["localAttention"], j["globalEvery"], j["headLayers"], j["headFfn"],
                             j["options"])
    else:
        spec, head = S.gliner(GLINER_SPECS[cfg["shape"]], GLINER_TEMPERATURE, GLINER_HEAD_HIDDEN[cfg["shape"]],
                              cfg["markers"])
    return build_plan(spec, head, cfg["length"], cfg["batch"], cfg["f16"], markers=cfg["markers"])


def test_frozen_file_covers_every_configuration():
    f = frozen()
    assert f["sourceCommit"] == "54bfc4e"
    assert list(f["traces"]) == [c["id"] for c in all_configs()]


def test_plan_builder_reproduces_the_frozen_dispatch_lists():
    f = frozen()["traces"]
    digests: dict = {}
    bad = []
    for cfg in all_configs():
        d = first_difference(f[cfg["id"]], record(plan_of(cfg), cfg), digests)
        if d:
            bad.append(f"{cfg['id']}: {d}")
    assert not bad, f"{len(bad)} of {len(f)} differ\n" + "\n".join(bad[:5])


def test_trace_comparison_catches_a_changed_plan():
    """The comparison is not vacuous: a constant, a binding or a table byte changed in the built
    plan is reported."""
    import numpy as np
    f = frozen()["traces"]
    cfg = next(c for c in all_configs() if c["id"] == "base-f16-B1-L1280K80-normal")
    plan = plan_of(cfg)
    assert first_difference(f[cfg["id"]], record(plan, cfg), {}) is None
    op = plan["segments"][1]["ops"][0]
    op["constants"]["N"] += 1
    assert "event" in first_difference(f[cfg["id"]], record(plan, cfg), {})
    op["constants"]["N"] -= 1
    op["bind"][0], op["bind"][3] = op["bind"][3], op["bind"][0]
    assert "event" in first_difference(f[cfg["id"]], record(plan, cfg), {})
    op["bind"][0], op["bind"][3] = op["bind"][3], op["bind"][0]
    rel = next(b for b in plan["buffers"] if b["id"] == "relidx")
    rel["init"] = np.array(rel["init"], copy=True)
    rel["init"].reshape(-1)[5] += 1
    assert "buffer" in first_difference(f[cfg["id"]], record(plan, cfg), {})


@pytest.mark.parametrize("value,js", [(1e-7, "1e-7"), (0.07216878364870323, "0.07216878364870323"), (1e-5, "0.00001"),
                                      (128.0, "128"), (3, "3"), (1e21, "1e+21"), (0.5, "0.5"), (160000.0, "160000")])
def test_js_number_strings(value, js):
    from tests.plan_trace import js_number
    assert js_number(value) == js
