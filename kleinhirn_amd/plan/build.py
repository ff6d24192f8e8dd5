"""Plan builder: ModelSpec + HeadSpec -> Plan (the op list a Backend executes).

A Python statement of the reference's plan builder (src/plan/build.ts:109-526) for the encoder
heads (classify, token, embed), producing plan dicts with the reference's field names so
``json.dumps(plan_json(plan))`` is the JSON the reference's ``JSON.stringify`` of a Plan gives
(typed-array ``init`` tables travel separately, as the C-ABI takes them). The GLiNER and Julia
heads of the reference are not described here.
"""
from __future__ import annotations

import math

import numpy as np

from .layers import add_workgroups, post_norm_layer, pre_norm_layer
from .spec import julia_head_layer, tensor_names_for

ACT = {"relu": 1, "gelu": 2, "tanh": 3, "silu": 4}


def act_code(act: str) -> int:
    if act not in ACT:
        raise ValueError(f"activation {act} has no kernel yet")
    return ACT[act]


def rel_bucket_index(i: int, j: int, span: int, max_pos: int) -> int:
    """Log-bucketed relative position of query i and key j, shifted by span and clamped to
    [0, 2 span - 1]; computed in double precision (src/plan/build.ts:22-33)."""
    rel = i - j
    mid = span >> 1
    a = abs(rel)
    r = rel
    if a > mid:
        log_pos = math.ceil(math.log(a / mid) / math.log((max_pos - 1) / mid) * (mid - 1)) + mid
        r = log_pos * (1 if rel > 0 else -1)
    return min(max(r + span, 0), 2 * span - 1)


def rel_pos_table(length: int, span: int, max_pos: int) -> np.ndarray:
    """relidx[i][j] as u32 [L * L] (src/plan/build.ts:35-45). Vectorised over i - j: the index
    depends on the difference only."""
    deltas = np.arange(-(length - 1), length)
    row = np.array([rel_bucket_index(int(dl), 0, span, max_pos) for dl in deltas], dtype=np.uint32)
    i = np.arange(length)[:, None]
    j = np.arange(length)[None, :]
    return row[(i - j) + (length - 1)].reshape(-1).astype(np.uint32)


def rope_table(length: int, theta: float, head_dim: int) -> np.ndarray:
    """[L][cos D | sin D] f32, entries d < D/2 of each half filled, f = i theta^(-2d/D) in double
    (src/plan/build.ts:47-60)."""
    half = head_dim // 2
    t = np.zeros((length, 2 * head_dim), dtype=np.float32)
    i = np.arange(length, dtype=np.float64)[:, None]
    d = np.arange(half, dtype=np.float64)[None, :]
    f = i * theta ** (-(2 * d) / head_dim)
    t[:, :half] = np.cos(f)
    t[:, head_dim:head_dim + half] = np.sin(f)
    return t.reshape(-1)


def writable_bindings(kernel: str, nbind: int) -> list[int]:
    """The written binding: the last, except add and rope which update binding 0
    (src/plan/build.ts:62-66)."""
    return [0] if kernel in ("add", "rope") else [nbind - 1]


def validate_segments(segments, known: set[str]) -> None:
    """Unknown buffers and a writable buffer bound twice are errors (src/plan/build.ts:68-87)."""
    for seg in segments:
        for op in seg.get("captureOps", []) + seg["ops"]:
            where = f"{seg['prefix']}{op['name']}"
            for bid in op["bind"]:
                if not bid.startswith("w:") and bid not in known:
                    raise ValueError(f"plan op {where}: unknown buffer {bid}")
            for wb in writable_bindings(op["kernel"], len(op["bind"])):
                bid = op["bind"][wb]
                if any(i != wb and o == bid for i, o in enumerate(op["bind"])):
                    raise ValueError(f"plan op {where}: writable buffer {bid} is bound twice")


def _elements_written(op: dict) -> int:
    k = op["kernel"]
    c = op["constants"]
    if k in ("matmul", "mmtile", "mmtile16", "mmtile8", "layernorm", "embln", "pool"):
        return c["N"]
    if k == "geglu":
        return c["I"]
    if k in ("attention", "mbattention", "mbflash", "attpv"):
        return c["H"] * c["D"]
    if k == "gather":
        return c["D"]
    if k == "im2col":
        return c["N"] * c["KS"]
    return 0


def build_plan(spec: dict, head: dict, length: int, batch: int, f16: bool, markers: int | None = None) -> dict:
    """src/plan/build.ts:109-526 for classify, token, embed and GLiNER2 heads. `markers` is the
    reference's BuildOptions.markers (marker slots per sequence of a GLiNER2 plan; the head's own
    count when None)."""
    if head["type"] not in ("classify", "token", "embed", "gliner2", "julia"):
        raise ValueError(f"head {head['type']} is not an encoder head of this runner")
    pooled = head["type"] not in ("gliner2", "julia")
    if head["type"] == "julia":
        markers = int(head["options"])
    else:
        markers = 0 if pooled else int(head["markers"] if markers is None else markers)
    if not pooled and markers < 1:
        raise ValueError("a marker head needs at least one marker slot")
    K = markers * batch
    names = tensor_names_for(spec)
    H = spec["hidden"]
    E = spec["embeddingSize"]

    def bytes_of(el):
        return math.ceil(el * (2 if f16 else 4) / 4) * 4

    M = length * batch
    eps = spec["block"]["norm"]["eps"]
    dims = {"hidden": H, "heads": spec["heads"], "headDim": spec["headDim"],
            "intermediate": spec["intermediate"], "rows": M, "length": length, "eps": eps}

    def ln(name, mode, bind, n=H, rows="rows"):
        return {"name": name, "kernel": "layernorm", "constants": {"N": n, "MODE": mode, "EPS": eps},
                "bind": bind, "dispatch": [rows, 1]}

    def mm(name, rows, n, k, act, bind, ydim):
        return {"name": name, "kernel": "matmul", "constants": {"M": rows, "N": n, "K": k, "ACT": act},
                "bind": bind, "dispatch": [math.ceil(n / 16), ydim]}

    segments = []
    # capture slots (the capture tool copies these buffers after their segment, an f32 row block
    # each; src/plan/build.ts:142-144)
    slot = [0]

    def take(*bufs):
        out = [{"buffer": b, "slot": slot[0] + i} for i, b in enumerate(bufs)]
        slot[0] += len(bufs)
        return out
    emb = spec["embed"]
    emb_w = f"w:{names.embedNormW}"
    emb_b = f"w:{names.embedNormB}" if names.embedNormB else "zero"
    absolute = emb["positions"] == "absolute"
    if absolute or emb["typeVocab"] > 0:
        type_table = "w:embeddings.type.weight" if emb["typeVocab"] > 0 else "zero"
        if emb["project"]:
            raise ValueError("embedding projection (ELECTRA) is not described here")
        segments.append({"name": "embed", "prefix": "", "capture": take("x"), "ops": [{
            "name": "embed", "kernel": "embln",
            "constants": {"N": E, "L": length, "OFFSET": emb["positionOffset"] if absolute else 0,
                          "MAXPOS": emb["maxPositions"] if absolute else 1, "EPS": emb["norm"]["eps"],
                          "MASKMUL": 1 if emb["maskMultiply"] else 0,
                          "POSIDS": 1 if emb.get("padId") is not None else 0},
            "bind": ["emb", "w:embeddings.position.weight" if absolute else "zero", type_table,
                     "typeIds", emb_w, emb_b, "mask", "x"],
            "dispatch": ["rows", 1]}]})
    elif emb["maskMultiply"]:
        # the capture tool records the plain norm too (captureOps run only when capturing)
        segments.append({"name": "embed", "prefix": "",
                         "ops": [ln("embed", 1, ["emb", "dummy", emb_w, emb_b, "mask", "x"])],
                         "captureOps": [ln("embedPlain", 0, ["emb", "dummy", emb_w, emb_b, "mask", "tmp"])],
                         "capture": take("tmp", "x")})
    else:
        segments.append({"name": "embed", "prefix": "",
                         "ops": [ln("embed", 0, ["emb", "dummy", emb_w, emb_b, "mask", "x"])],
                         "capture": take("x")})

    rel = spec["attention"].get("rel") if spec["attention"]["kind"] == "deberta-relative" else None
    if rel is not None:
        scale = math.sqrt((1 + len(rel["types"])) * (H / spec["heads"]))
        def attn_of(_l):
            return scale, 0
    else:
        win = spec["attention"].get("window")
        scale = (H / spec["heads"]) ** -0.5
        def attn_of(l):
            return scale, (0 if (not win or l % win["globalEvery"] == 0) else win["half"])
    rope = spec["attention"].get("rope")
    rope_split = bool(rope) and rope["thetaGlobal"] != rope["thetaLocal"]
    for l in range(spec["layers"]):
        t = names.layer(l)
        a_scale, a_window = attn_of(l)
        if spec["block"]["order"] == "post":
            rel_c = None
            if rel is not None:
                moff = rel_bucket_index(0, length - 1, rel["buckets"], rel["maxPositions"])
                nm = rel_bucket_index(length - 1, 0, rel["buckets"], rel["maxPositions"]) - moff + 1
                rel_c = {"moff": moff, "nm": nm}
            ops = post_norm_layer(dims, t, act_code(spec["ffn"]["act"]), a_scale,
                                  spec["attention"]["kind"] == "standard", rel_c)
        else:
            identity = spec["block"]["firstNormIdentity"] and l == 0
            ffn = ({"kind": "geglu"} if spec["ffn"]["kind"] == "geglu"
                   else {"kind": "mlp", "width": spec["intermediate"], "act": act_code(spec["ffn"]["act"])})
            tt = dict(t, attnNormW=None) if identity else t
            table = ("cossinG" if a_window == 0 else "cossinL") if rope_split else "cossin"
            ops = pre_norm_layer(dims, tt, "x", not identity, a_scale, a_window, bool(rope), ffn, table)
        segments.append({"name": f"layer{l}", "prefix": f"L{l}.", "ops": ops, "skippable": True,
                         "capture": take("x")})

    stream = "x"
    if spec["block"]["finalNorm"]:
        segments.append({"name": "final", "prefix": "", "capture": take("tmp"), "ops": [
            ln("final", 0, ["x", "dummy", f"w:{names.finalNormW}",
                            f"w:{names.finalNormB}" if names.finalNormB else "zero", "mask", "tmp"])]})
        stream = "tmp"

    if not pooled:
        return _marker_plan(spec, head, segments, stream, dims, length, batch, f16, markers, K, bytes_of, mm, ln,
                            absolute, take, slot)

    # Head (src/plan/build.ts:296-357)
    head_buffers = []
    per_row = head["type"] == "token"
    rows = M if per_row else batch
    rows16 = "rows16" if per_row else math.ceil(batch / 16)
    prev = stream
    width = H
    ops = []
    need_first = False
    if not per_row:
        pool = "first" if head["pool"] == "cls" else head["pool"]
        if pool == "first":
            need_first = True
            ops.append({"name": "gather", "kernel": "gather", "constants": {"K": 1, "D": H, "L": length},
                        "bind": ["first", stream, "states"], "dispatch": [1, 1]})
        else:
            ops.append({"name": "pool", "kernel": "pool",
                        "constants": {"L": length, "N": H, "MODE": 0 if pool == "mean" else 1},
                        "bind": [stream, "mask", "states"], "dispatch": [math.ceil(H / 64), batch]})
        head_buffers.append({"id": "states", "elements": batch * H, "final": False})
        prev = "states"
    steps = head.get("steps", [])
    for i, step in enumerate(steps):
        last = i == len(steps) - 1
        dst = "out" if last else f"hd{i}"
        if step["op"] == "norm":
            ops.append({"name": f"step{i}", "kernel": "layernorm",
                        "constants": {"N": width, "MODE": 0, "EPS": step["eps"]},
                        "bind": [prev, "dummy", f"w:{step['name']}.weight",
                                 f"w:{step['name']}.bias" if step["bias"] else "zero", "mask", dst],
                        "dispatch": ["rows" if per_row else batch, 1]})
            head_buffers.append({"id": dst, "elements": rows * width, "final": last})
            prev = dst
            continue
        if step["in"] != width:
            raise ValueError(f"head step {step['name']}: input {step['in']}, previous width {width}")
        ops.append(mm(f"step{i}", rows, step["out"], step["in"],
                      0 if step["act"] == "none" else act_code(step["act"]),
                      [prev, f"w:{step['name']}.weight",
                       f"w:{step['name']}.bias" if step["bias"] else "zero", dst], rows16))
        head_buffers.append({"id": dst, "elements": rows * step["out"], "final": last})
        prev = dst
        width = step["out"]
    if not steps:
        if per_row:
            raise ValueError("a token head needs at least one dense step")
        for b in head_buffers:
            if b["id"] == "states":
                b["final"] = True
    segments.append({"name": "head", "prefix": "head.", "ops": ops})

    # Buffers (src/plan/build.ts:432-505)
    all_ops = [op for s in segments for op in s.get("captureOps", []) + s["ops"]]
    cols: dict[str, int] = {}
    for op in all_ops:
        dst = op["bind"][writable_bindings(op["kernel"], len(op["bind"]))[0]]
        n = _elements_written(op)
        if n > 0:
            cols[dst] = max(cols.get(dst, 0), n)
    decls = []

    def st(bid, nbytes, usage="rw", init=None):
        d = {"id": bid, "bytes": int(nbytes), "usage": usage}
        if init is not None:
            d["init"] = init
        decls.append(d)

    st("emb", bytes_of(M * E))
    if absolute or emb["typeVocab"] > 0:
        st("typeIds", M * 4)
    for bid in ("x", "tmp"):
        if bid in cols:
            st(bid, bytes_of(M * cols[bid]), "rwSrc")
    for bid in ("normed", "qkv", "ctx", "attnOut", "mid", "gate", "ffnOut"):
        if bid in cols:
            st(bid, bytes_of(M * cols[bid]))
    st("mask", M * 4)
    if any("kinfo" in o["bind"] for o in all_ops):
        st("kinfo", 8 * batch)
    for bid in ("c2p", "p2c"):
        rel_ops = [o for o in all_ops if o["kernel"] == "attrel" and o["bind"][4] == bid]
        if rel_ops:
            st(bid, max(o["constants"]["ROWS"] * o["constants"]["H"] * o["constants"]["NM"] * 4
                        for o in rel_ops))
    score_ops = [o for o in all_ops if o["kernel"] == "attscore"]
    if score_ops:
        st("scores", max(o["constants"]["ROWS"] * o["constants"]["H"] * o["constants"]["L"] * 4
                         for o in score_ops))
    if any("dummy" in o["bind"] for o in all_ops):
        st("dummy", 4, "storage")
    for b in head_buffers:
        st(b["id"], bytes_of(b["elements"]), "logits" if b["final"] else "rw")
    if need_first:
        st("first", 3 * batch * 4, "rw", np.zeros(3 * batch, dtype=np.uint32))
    if rel is not None:
        table = rel_pos_table(length, rel["buckets"], rel["maxPositions"])
        st("relidx", table.nbytes, "rw", table)
    if rope and not rope_split:
        table = rope_table(length, rope["thetaGlobal"], spec["headDim"])
        st("cossin", table.nbytes, "rw", table)
    elif rope:
        g = rope_table(length, rope["thetaGlobal"], spec["headDim"])
        lt = rope_table(length, rope["thetaLocal"], spec["headDim"])
        st("cossinG", g.nbytes, "rw", g)
        st("cossinL", lt.nbytes, "rw", lt)
    zero_uses = [o for o in all_ops if "zero" in o["bind"]]
    if zero_uses:
        w = max(o["constants"]["N"] for o in zero_uses)
        st("zero", bytes_of(w), "rw", np.zeros(bytes_of(w), dtype=np.uint8))

    validate_segments(segments, {d["id"] for d in decls})
    inputs = {"embeddings": "emb", "mask": "mask"}
    if absolute or emb["typeVocab"] > 0:
        inputs["typeIds"] = "typeIds"
    out_rows = rows
    return {
        "f16": f16, "length": length, "batch": batch, "markers": 0, "embeddingSize": E,
        "buffers": decls, "segments": segments, "inputs": inputs,
        "output": {"buffer": prev, "bytes": bytes_of(out_rows * width), "dtype": "storage",
                   "rows": out_rows, "cols": width},
        "captureSlots": slot[0], "captureSlotBytes": length * H * 4,
    }


def _marker_plan(spec, head, segments, stream, dims, length, batch, f16, markers, K, bytes_of, mm, ln,
                 absolute, take, slot) -> dict:
    """Marker heads, whose output is one f32 logit per marker slot (K = markers x batch slots; the
    packed markers input holds per sequence K row indices, K mask words as f32 bits, K group ids):
    * gliner2 (src/plan/build.ts:358-377): the hidden states at the marker rows, fc1 with ReLU,
      fc2 to one raw logit, masklogits (raw / temperature where the mask is set, else -1e4);
    * julia (src/plan/build.ts:378-430): the type row of each sequence (rowSelect of type_emb by
      the run's qtype) added to every row of the final-norm stream, `layers` pre-norm layers with
      an MLP of width `ffn` (ReLU) and full attention without RoPE, then the scorer: gather,
      LayerNorm, fc1 with GELU, fc2, masklogits at temperature 1.
    Buffers as src/plan/build.ts:432-526 lays them out for a marker head."""
    H = spec["hidden"]
    E = spec["embeddingSize"]
    M = length * batch
    K16 = math.ceil(K / 16)
    row_select = None
    if head["type"] == "gliner2":
        hh = int(head["hidden"])
        segments.append({"name": "head", "prefix": "head.", "ops": [
            {"name": "gather", "kernel": "gather", "constants": {"K": markers, "D": H, "L": length},
             "bind": ["packed", stream, "states"], "dispatch": [1, 1]},
            mm("fc1", K, hh, H, 1, ["states", "w:head.fc1.weight", "w:head.fc1.bias", "h1"], K16),
            mm("fc2", K, 1, hh, 0, ["h1", "w:head.fc2.weight", "w:head.fc2.bias", "raw"], K16),
            {"name": "maskl", "kernel": "masklogits", "constants": {"K": markers, "TEMP": float(head["temperature"])},
             "bind": ["raw", "packed", "logits"], "dispatch": [1, 1]},
        ]})
    else:
        if stream != "tmp":
            raise ValueError("julia head expects a final norm")
        segments.append({"name": "typed", "prefix": "", "capture": take("tmp"), "ops": [
            {"name": "type", "kernel": "add", "constants": {"TOTAL": M * H, "N": H, "MODE": 1, "L": length},
             "bind": ["tmp", "typeRow"], "dispatch": [add_workgroups(M, H), 1]}]})
        row_select = {"table": "w:type_emb.weight", "dst": "typeRow", "rowBytes": bytes_of(H)}
        for i in range(int(head["layers"])):
            segments.append({"name": f"head{i}", "prefix": f"head{i}.", "capture": take("tmp"), "ops": pre_norm_layer(
                dims, julia_head_layer(i), "tmp", True, (H / spec["heads"]) ** -0.5, 0, False,
                {"kind": "mlp", "width": int(head["ffn"]), "act": 1})})
        segments.append({"name": "scorer", "prefix": "scorer.", "ops": [
            {"name": "gather", "kernel": "gather", "constants": {"K": markers, "D": H, "L": length},
             "bind": ["packed", "tmp", "states"], "dispatch": [1, 1]},
            ln("ln", 0, ["states", "dummy", "w:scorer.norm.weight", "w:scorer.norm.bias", "mask", "kNormed"], H, K),
            mm("fc1", K, H, H, 2, ["kNormed", "w:scorer.fc1.weight", "w:scorer.fc1.bias", "h1"], K16),
            mm("fc2", K, 1, H, 0, ["h1", "w:scorer.fc2.weight", "w:scorer.fc2.bias", "raw"], K16),
            {"name": "maskl", "kernel": "masklogits", "constants": {"K": markers, "TEMP": 1.0},
             "bind": ["raw", "packed", "logits"], "dispatch": [1, 1]},
        ]})
    all_ops = [op for s in segments for op in s.get("captureOps", []) + s["ops"]]
    cols: dict[str, int] = {}
    for op in all_ops:
        dst = op["bind"][writable_bindings(op["kernel"], len(op["bind"]))[0]]
        n = _elements_written(op)
        if n > 0:
            cols[dst] = max(cols.get(dst, 0), n)
    k_rows = {"states", "kNormed", "h1", "raw"}
    decls = []

    def st(bid, nbytes, usage="rw", init=None):
        d = {"id": bid, "bytes": int(nbytes), "usage": usage}
        if init is not None:
            d["init"] = init
        decls.append(d)

    emb = spec["embed"]
    st("emb", bytes_of(M * E))
    if absolute or emb["typeVocab"] > 0:
        st("typeIds", M * 4)
    for bid in ("x", "tmp"):
        if bid in cols:
            st(bid, bytes_of(M * cols[bid]), "rwSrc")
    for bid in ("normed", "qkv", "ctx", "attnOut", "mid", "gate", "ffnOut", "states", "kNormed", "h1", "raw"):
        if bid in cols:
            st(bid, bytes_of((K if bid in k_rows else M) * cols[bid]))
    st("mask", M * 4)
    if any("kinfo" in o["bind"] for o in all_ops):
        st("kinfo", 8 * batch)
    for bid in ("c2p", "p2c"):
        rel_ops = [o for o in all_ops if o["kernel"] == "attrel" and o["bind"][4] == bid]
        if rel_ops:
            st(bid, max(o["constants"]["ROWS"] * o["constants"]["H"] * o["constants"]["NM"] * 4
                        for o in rel_ops))
    score_ops = [o for o in all_ops if o["kernel"] == "attscore"]
    if score_ops:
        st("scores", max(o["constants"]["ROWS"] * o["constants"]["H"] * o["constants"]["L"] * 4
                         for o in score_ops))
    if any("dummy" in o["bind"] for o in all_ops):
        st("dummy", 4, "storage")
    st("packed", 3 * K * 4)
    st("logits", K * 4, "logits")
    rel = spec["attention"].get("rel") if spec["attention"]["kind"] == "deberta-relative" else None
    if rel is not None:
        table = rel_pos_table(length, rel["buckets"], rel["maxPositions"])
        st("relidx", table.nbytes, "rw", table)
    rope = spec["attention"].get("rope")
    if rope and rope["thetaGlobal"] == rope["thetaLocal"]:
        table = rope_table(length, rope["thetaGlobal"], spec["headDim"])
        st("cossin", table.nbytes, "rw", table)
    elif rope:
        g = rope_table(length, rope["thetaGlobal"], spec["headDim"])
        lt = rope_table(length, rope["thetaLocal"], spec["headDim"])
        st("cossinG", g.nbytes, "rw", g)
        st("cossinL", lt.nbytes, "rw", lt)
    if row_select:
        st("typeRow", bytes_of(batch * H))
    zero_uses = [o for o in all_ops if "zero" in o["bind"]]
    if zero_uses:
        w = max(o["constants"]["N"] for o in zero_uses)
        st("zero", bytes_of(w), "rw", np.zeros(bytes_of(w), dtype=np.uint8))
    validate_segments(segments, {d["id"] for d in decls})
    plan = {
        "f16": f16, "length": length, "batch": batch, "markers": markers, "embeddingSize": E,
        "buffers": decls, "segments": segments,
        "inputs": {"embeddings": "emb", "mask": "mask", "markers": "packed"},
        "output": {"buffer": "logits", "bytes": K * 4, "dtype": "f32", "rows": K, "cols": 1},
        "captureSlots": slot[0], "captureSlotBytes": length * H * 4,
    }
    if row_select:
        plan["rowSelect"] = row_select
    return plan


def pack_markers(indices, mask, groups=None, markers: int | None = None) -> np.ndarray:
    """The packed marker payload of one sequence (RunInput.packedMarkers, src/plan/executor.ts:28):
    [0, K) marker row indices, [K, 2K) the marker mask as f32 bits, [2K, 3K) group ids; the
    payloads of a batch plan follow each other. Shorter lists are padded with masked slots."""
    idx = np.asarray(indices, dtype=np.uint32)
    K = len(idx) if markers is None else markers
    if len(idx) > K:
        raise ValueError(f"{len(idx)} markers, the plan holds {K}")
    out = np.zeros(3 * K, dtype=np.uint32)
    out[:len(idx)] = idx
    out[K:K + len(idx)] = np.asarray(mask, dtype=np.float32).view(np.uint32)
    if groups is not None:
        out[2 * K:2 * K + len(idx)] = np.asarray(groups, dtype=np.uint32)
    return out


def plan_json(plan: dict) -> dict:
    """The plan without its typed-array init tables (they travel as separate byte buffers)."""
    out = dict(plan)
    out["buffers"] = [{k: v for k, v in d.items() if k != "init"} for d in plan["buffers"]]
    return out


def plan_inits(plan: dict) -> dict[str, bytes]:
    return {d["id"]: np.ascontiguousarray(d["init"]).tobytes() for d in plan["buffers"] if "init" in d}


def all_ops(plan: dict) -> list[dict]:
    return [op for s in plan["segments"] for op in s["ops"]]


__all__ = ["build_plan", "pack_markers", "plan_json", "plan_inits", "rel_pos_table", "rope_table",
           "rel_bucket_index", "act_code", "all_ops", "add_workgroups"]
