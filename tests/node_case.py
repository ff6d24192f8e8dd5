"""Exports a plan, its weights and one RunInput as files for tests/node/run_plan.js, so the Node-API
path (the host side hip-backend.ts uses) runs the same case as the Python host."""
from __future__ import annotations

import json
import os
import subprocess

import numpy as np

from kleinhirn_amd.plan.build import plan_inits, plan_json

HERE = os.path.dirname(os.path.abspath(__file__))
ADDON = os.path.join(os.path.dirname(HERE), "kleinhirn_amd", "node", "kh_addon.node")
RUNNER = os.path.join(HERE, "node", "run_plan.js")


def export_case(dirname: str, plan: dict, weights: dict | None = None, run_input: dict | None = None,
                rows: int | None = None, check_only: bool = False, manifest: str | None = None,
                manifest_flags: int = 0, ids: "np.ndarray | None" = None) -> None:
    """Case files for run_plan.js. `manifest`: weights from that manifest.json (kh_load_manifest,
    or kh_manifest_check with check_only); `ids`: token ids for the device word gather."""
    os.makedirs(dirname, exist_ok=True)
    with open(os.path.join(dirname, "plan.json"), "w") as f:
        json.dump(plan_json(plan), f)
    meta = {"checkOnly": check_only, "weights": [], "inits": {}, "rows": rows or 0,
            "typeIds": bool(run_input is not None and run_input.get("typeIds") is not None),
            "manifest": manifest, "manifestFlags": manifest_flags, "ids": ids is not None,
            "markers": bool(run_input is not None and run_input.get("packedMarkers") is not None)}
    if ids is not None:
        np.ascontiguousarray(ids, dtype=np.int32).tofile(os.path.join(dirname, "ids.bin"))
    if not check_only:
        for i, (name, t) in enumerate((weights or {}).items()):
            t = np.ascontiguousarray(t)
            fn = f"w{i}.bin"
            t.tofile(os.path.join(dirname, fn))
            meta["weights"].append({"name": name, "dtype": 1 if t.dtype == np.float16 else 0,
                                    "shape": list(t.shape), "file": fn})
        for i, (bid, raw) in enumerate(plan_inits(plan).items()):
            fn = f"init{i}.bin"
            with open(os.path.join(dirname, fn), "wb") as f:
                f.write(raw)
            meta["inits"][bid] = fn
        if ids is None:
            np.ascontiguousarray(run_input["embeddings"]).tofile(os.path.join(dirname, "emb.bin"))
        np.ascontiguousarray(run_input["mask"], dtype=np.float32).tofile(os.path.join(dirname, "mask.bin"))
        if meta["typeIds"]:
            np.ascontiguousarray(run_input["typeIds"], dtype=np.uint32).tofile(os.path.join(dirname, "tt.bin"))
        if meta["markers"]:
            np.ascontiguousarray(run_input["packedMarkers"], dtype=np.uint32).tofile(os.path.join(dirname, "mk.bin"))
        if run_input.get("qtype") is not None:
            meta["qtype"] = [int(x) for x in np.atleast_1d(run_input["qtype"])]
    with open(os.path.join(dirname, "meta.json"), "w") as f:
        json.dump(meta, f)


def export_sched_case(dirname: str, plan: dict, weights: dict, words: np.ndarray, seqs: list, type_words: np.ndarray,
                      token_budget: int = 0) -> None:
    """Case files for the scheduler path of run_plan.js: the plan (two copies run under kh_sched),
    weights, the device word table and the sequences as ids + offsets."""
    export_case(dirname, plan, weights, {"embeddings": np.zeros(1, np.float16), "mask": np.zeros(1, np.float32)})
    with open(os.path.join(dirname, "meta.json")) as f:
        meta = json.load(f)
    np.ascontiguousarray(words).tofile(os.path.join(dirname, "words.bin"))
    meta["words"] = {"file": "words.bin", "dtype": 1 if words.dtype == np.float16 else 0,
                     "rows": int(words.shape[0]), "width": int(words.shape[1])}
    np.concatenate([np.asarray(x, np.int32) for x in seqs]).tofile(os.path.join(dirname, "ids.bin"))
    offs = np.zeros(len(seqs) + 1, np.float64)
    offs[1:] = np.cumsum([len(x) for x in seqs])
    offs.tofile(os.path.join(dirname, "offsets.bin"))
    np.ascontiguousarray(type_words, dtype=np.uint32).tofile(os.path.join(dirname, "tw.bin"))
    meta["sched"] = {"typeWords": True, "tokenBudget": token_budget, "cols": plan["output"]["cols"]}
    with open(os.path.join(dirname, "meta.json"), "w") as f:
        json.dump(meta, f)


def run_node(dirname: str, timeout: int = 120) -> dict:
    r = subprocess.run(["node", RUNNER, dirname], capture_output=True, text=True, timeout=timeout)
    if r.returncode != 0:
        raise RuntimeError(f"node run_plan.js failed: {r.stderr.strip()}")
    return json.loads(r.stdout.strip().splitlines()[-1])
