"""Canonical dispatch traces of a plan, as the reference's WebGPU executor would record them.

The reference freezes the dispatch lists of its plan executor for GLiNER (DeBERTa-v2 relative
attention, span head) and Julia-1 (ModernBERT, decision head) plans in
tests/golden/k28/dispatch-traces.json.gz (a copy: tests/golden/k28_dispatch_traces.json.gz), and
its gate (tests/plan_trace.test.ts:60-72) requires the executor to reproduce them. Each trace is
what PlanExecutor encodes for one call on a mock device (tests/helpers/plan-trace.ts:135-237,
tests/helpers/mock-gpu.ts): run-time buffer writes, copies, compute passes, and per dispatch the
pipeline (the WGSL source's sha256 prefix and the op constants), the bind group and the workgroup
counts; buffers are named b0, b1, ... by first use, with size, WebGPU usage flags and the sha256
of the bytes written at build.

This module restates that encoding (src/plan/executor.ts:75-329) over the plans of
kleinhirn_amd/plan, so tests/test_plan_traces.py can compare the two plan builders dispatch by
dispatch. The WGSL sources are not part of this build: a pipeline's source digest is compared by
consistency (one digest per kernel name and storage dtype) instead of by value.
"""
from __future__ import annotations

import hashlib
import json
import math

import numpy as np

# tests/helpers/plan-trace.ts:24-48
GLINER_SPECS = {
    "small": {"hiddenSize": 384, "layers": 12, "heads": 6, "intermediateSize": 1536,
              "positionBuckets": 256, "maxRelativePositions": 512, "layerNormEps": 1e-7},
    "base": {"hiddenSize": 768, "layers": 12, "heads": 12, "intermediateSize": 3072,
             "positionBuckets": 256, "maxRelativePositions": 512, "layerNormEps": 1e-7},
}
GLINER_HEAD_HIDDEN = {"small": 768, "base": 1536}
GLINER_TEMPERATURE = 1.0
JULIA_SPEC = {"layers": 22, "hiddenSize": 384, "heads": 6, "intermediate": 1152, "normEps": 1e-5,
              "ropeTheta": 160000, "localAttention": 64, "globalEvery": 3, "headLayers": 2,
              "headFfn": 1536, "options": 20}

# WebGPU GPUBufferUsage flags
MAP_READ, COPY_SRC, COPY_DST, STORAGE, QUERY_RESOLVE = 1, 4, 8, 128, 512
USAGE = {"rw": STORAGE | COPY_DST, "rwSrc": STORAGE | COPY_DST | COPY_SRC, "storage": STORAGE,
         "logits": STORAGE | COPY_SRC | COPY_DST}


def all_configs() -> list[dict]:
    """The 125 configurations of tests/helpers/plan-trace.ts:53-80, in the frozen file's order."""
    out = []
    shapes = [("small", [(128, 16), (512, 16)]), ("base", [(128, 16), (512, 16), (1280, 80)]),
              ("julia-1", [(128, 20), (512, 20)])]
    for shape, sizes in shapes:
        for f16 in (False, True):
            for batch in (1, 4):
                for length, markers in sizes:
                    modes = ["normal", "normal100", "pass"]
                    if batch == 1:
                        modes.append("dispatch")
                    if batch == 1 and not f16:
                        modes.append("capture")
                    if shape != "julia-1":
                        modes.append("skip")
                    for mode in modes:
                        out.append({"id": f"{shape}-{'f16' if f16 else 'f32'}-B{batch}-L{length}K{markers}-{mode}",
                                    "shape": shape, "f16": f16, "batch": batch, "length": length,
                                    "markers": markers, "mode": mode})
    return out


def js_number(x) -> str:
    """String(x) of a JavaScript number: integers without a fraction, the shortest round-trip digits
    otherwise, fixed notation for 1e-7 <= |x| < 1e21 and 'd.ddde-7' style exponents outside."""
    if isinstance(x, bool):
        x = int(x)
    if isinstance(x, int) or (isinstance(x, float) and x.is_integer() and abs(x) < 1e21):
        return str(int(x))
    r = repr(float(x))
    sign = "-" if r.startswith("-") else ""
    r = r.lstrip("-")
    if "e" in r:
        mant, exp = r.split("e")
        exp = int(exp)
    else:
        mant, exp = r, 0
    ip, _, fp = mant.partition(".")
    digits = (ip + fp).lstrip("0")
    # value = 0.digits * 10^point
    point = len(ip) + exp if ip != "0" else exp - (len(fp) - len(fp.lstrip("0")))
    digits = digits.rstrip("0") or "0"
    n = len(digits)
    if -6 < point <= 21:
        if point <= 0:
            s = "0." + "0" * (-point) + digits
        elif point >= n:
            s = digits + "0" * (point - n)
        else:
            s = digits[:point] + "." + digits[point:]
    else:
        e = point - 1
        s = digits[0] + ("." + digits[1:] if n > 1 else "") + ("e+" if e > 0 else "e-") + str(abs(e))
    return sign + s


def constants_key(c: dict) -> str:
    return ",".join(f"{k}={js_number(c[k])}" for k in sorted(c))


def _sha(b: bytes) -> str:
    return hashlib.sha256(b).hexdigest()


def init_bytes(init) -> bytes:
    return np.ascontiguousarray(init).tobytes() if isinstance(init, np.ndarray) else bytes(init)


class Tracer:
    """Records the canonical events of one call (tests/helpers/plan-trace.ts:100-133)."""

    def __init__(self, plan: dict):
        self.plan = plan
        self.decl = {b["id"]: b for b in plan["buffers"]}
        self.names: dict[str, str] = {}
        self.buffers: dict[str, dict] = {}
        self.events: list[str] = []
        self.pipes: list[tuple[str, str, bool]] = []  # (kernel, constants key, f16) per pipe event

    def ref(self, bid: str, size: int | None = None, usage: int | None = None) -> str:
        if bid.startswith("w:"):
            return bid
        n = self.names.get(bid)
        if n is None:
            n = f"b{len(self.names)}"
            self.names[bid] = n
            if bid in self.decl:
                d = self.decl[bid]
                entry = {"size": d["bytes"], "usage": USAGE[d["usage"]]}
                if d.get("init") is not None:
                    entry["init"] = _sha(init_bytes(d["init"]))  # one build-time write at offset 0
            else:
                entry = {"size": size, "usage": usage}
            self.buffers[n] = entry
        return n

    def ev(self, *a) -> None:
        self.events.append(json.dumps(list(a), separators=(",", ":")))

    def write(self, bid: str, nbytes: int) -> None:
        self.ev("write", self.ref(bid), 0, nbytes)

    def copy(self, src: str, so: int, dst: str, do: int, nbytes: int, **dst_decl) -> None:
        s = self.ref(src)
        self.ev("copy", s, so, self.ref(dst, **dst_decl), do, nbytes)

    def dispatch(self, op: dict, rows: int) -> None:
        o = next((a for a in op.get("alts", []) if rows <= a["maxRows"]), None)
        kernel = o["kernel"] if o else op["kernel"]
        disp = o["dispatch"] if o else op["dispatch"]
        key = constants_key(op["constants"])
        self.pipes.append((kernel, key, self.plan["f16"]))
        self.ev("pipe", "?" + "|" + key)
        bound = [[i, self.ref(b)] for i, b in enumerate(op["bind"])]
        self.ev("bind", 0, bound)
        self.ev("dispatch", dim(disp[0], rows), dim(disp[1], rows))


def dim(d, rows: int) -> int:
    """PlanExecutor.dim (src/plan/executor.ts:216-218)."""
    if d == "rows":
        return rows
    if d in ("rows8", "rows16", "rows32"):
        return math.ceil(rows / int(d[4:]))
    return int(d)


def record(plan: dict, cfg: dict) -> dict:
    """The canonical trace of one configuration's call (recordTrace, tests/helpers/plan-trace.ts:
    186-216) with PlanExecutor's upload and encode (src/plan/executor.ts:225-297, 336-367)."""
    t = Tracer(plan)
    L, B = plan["length"], plan["batch"]
    hidden = plan["embeddingSize"]
    mode = cfg["mode"]
    es = 2 if plan["f16"] else 4
    rows_in = L * B
    julia = plan.get("rowSelect") is not None
    k = (JULIA_SPEC["options"] if julia else cfg["markers"]) * B
    qtype = (0 if B == 1 else [0, 1, 2, 0]) if julia else None

    def upload():
        i = plan["inputs"]
        t.write(i["embeddings"], rows_in * hidden * es)
        t.write(i["mask"], rows_in * 4)
        if "kinfo" in t.decl:
            t.write("kinfo", 2 * B * 4)
        if i.get("markers"):
            t.write(i["markers"], 3 * k * 4)
        if i.get("typeIds"):
            t.write(i["typeIds"], rows_in * 4)

    segs = plan["segments"]
    maps = 1
    profile_keys = None
    gpu_build = sum(b["bytes"] for b in plan["buffers"]) + plan["output"]["bytes"]
    gpu_end = gpu_build
    staging = {"size": plan["output"]["bytes"], "usage": MAP_READ | COPY_DST}

    def row_select():
        rs = plan.get("rowSelect")
        if rs:
            qt = qtype if isinstance(qtype, list) else [qtype or 0]
            for b in range(B):
                q = qt[b] if b < len(qt) else 0
                t.copy(rs["table"], q * rs["rowBytes"], rs["dst"], b * rs["rowBytes"], rs["rowBytes"])

    if mode in ("normal", "normal100", "skip", "capture"):
        upload()
        seq_len = {"normal": L * B, "capture": 100, "normal100": 100 * B, "skip": 100 * B}[mode]
        skip = {1} if mode == "skip" else None
        rows = L if mode == "capture" else seq_len
        row_select()

        def kept(seg):
            if seg.get("skippable") and skip:
                return [op for i, op in enumerate(seg["ops"]) if i not in skip]
            return seg["ops"]

        if mode != "capture":
            t.ev("begin")
            for seg in segs:
                for op in kept(seg):
                    t.dispatch(op, rows)
            t.ev("end")
        else:
            cap_bytes = plan["captureSlots"] * plan["captureSlotBytes"]
            for seg in segs:
                t.ev("begin")
                for op in seg.get("captureOps", []):
                    t.dispatch(op, rows)
                for op in kept(seg):
                    t.dispatch(op, rows)
                t.ev("end")
                for c in seg.get("capture", []):
                    off = plan["captureSlotBytes"]
                    t.copy(c["buffer"], 0, "@capture", c["slot"] * off, off, size=cap_bytes, usage=COPY_DST | MAP_READ)
            gpu_end += cap_bytes
            maps += 1
        t.copy(plan["output"]["buffer"], 0, "@staging", 0, plan["output"]["bytes"], **staging)
    else:  # pass / dispatch profiles (PlanExecutor.profileForward)
        disp = mode == "dispatch"
        upload()
        rows = 100 if disp else L
        row_select()
        names = []
        p = 0
        if disp:
            for seg in segs:
                for op in seg["ops"]:
                    names.append(seg["prefix"] + op["name"])
                    t.ev("begin", 2 * p, 2 * p + 1)
                    p += 1
                    t.dispatch(op, rows)
                    t.ev("end")
        else:
            for seg in segs:
                names.append(seg["name"])
                t.ev("begin", 2 * p, 2 * p + 1)
                p += 1
                for op in seg["ops"]:
                    t.dispatch(op, rows)
                t.ev("end")
        t.copy(plan["output"]["buffer"], 0, "@staging", 0, plan["output"]["bytes"], **staging)
        t.events.append(json.dumps(["resolve", 0, 2 * p, t.ref("@resolve", 16 * p, QUERY_RESOLVE | COPY_SRC), 0],
                                   separators=(",", ":")))
        t.copy("@resolve", 0, "@tsstaging", 0, 16 * p, size=16 * p, usage=MAP_READ | COPY_DST)
        profile_keys = names
        maps = 2
    return {"gpuBytesBuild": gpu_build, "gpuBytesEnd": gpu_end, "maps": maps, "profileKeys": profile_keys,
            "buffers": t.buffers, "events": t.events, "pipes": t.pipes}


def first_difference(frozen: dict, ours: dict, digests: dict) -> str | None:
    """firstDifference (tests/helpers/plan-trace.ts:218-237), with each pipeline's source digest
    checked for consistency: every (kernel, dtype) pair maps to one digest, and a digest to one
    kernel name (kernels that touch only f32 data have one source for both dtypes), across all
    traces compared through the same `digests` map."""
    for k in ("gpuBytesBuild", "gpuBytesEnd", "maps"):
        if frozen[k] != ours[k]:
            return f"{k} frozen {frozen[k]}, now {ours[k]}"
    if json.dumps(frozen["profileKeys"]) != json.dumps(ours["profileKeys"]):
        return f"profile keys frozen {frozen['profileKeys']}, now {ours['profileKeys']}"
    fe, oe = frozen["events"], ours["events"]
    pipes = iter(ours["pipes"])
    for i in range(max(len(fe), len(oe))):
        a = fe[i] if i < len(fe) else None
        b = oe[i] if i < len(oe) else None
        if a is not None and b is not None and a.startswith('["pipe"') and b.startswith('["pipe"'):
            fd, fkey = json.loads(a)[1].split("|", 1)
            _, okey = json.loads(b)[1].split("|", 1)
            kernel, _, f16 = next(pipes)
            if fkey != okey:
                return f"event {i}: frozen {a}, now {b}"
            known = digests.setdefault((kernel, f16), fd)
            if known != fd:
                return f"event {i}: kernel {kernel} ({'f16' if f16 else 'f32'}) has WGSL digest {fd}, elsewhere {known}"
            owner = digests.setdefault(("digest", fd), kernel)
            if owner != kernel:
                return f"event {i}: digest {fd} belongs to {owner}, here {kernel}"
            continue
        if a != b:
            return f"event {i}: frozen {a}, now {b}"
    for key in sorted(set(frozen["buffers"]) | set(ours["buffers"])):
        if json.dumps(frozen["buffers"].get(key), sort_keys=True) != json.dumps(ours["buffers"].get(key), sort_keys=True):
            return f"buffer {key}: frozen {frozen['buffers'].get(key)}, now {ours['buffers'].get(key)}"
    return None
