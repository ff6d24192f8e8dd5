"""Layer templates of the plan IR: post-norm and pre-norm encoder layers as op lists.

A Python statement of the reference's layer templates (src/plan/layers.ts:1-204) that produces
the same op dicts (kernel names, constants, bindings, dispatch dims), so plans built here are the
plans the reference's TypeScript builder hands to a Backend.
"""
from __future__ import annotations

import math

MAX_WORKGROUPS = 65535
SCORES_MAX_BYTES = 134217728  # f32 scores of the split attention must fit one 128 MiB binding


def add_workgroups(rows: int, hidden: int) -> int:
    """Grid-stride add dispatch, capped at 65535 workgroups (src/plan/layers.ts:28-32)."""
    return min(math.ceil(rows * hidden / 64), MAX_WORKGROUPS)


def _w(name, zero="zero"):
    return zero if name is None else f"w:{name}"


def _req(name, what):
    if name is None:
        raise ValueError(f"layer tensor {what} missing")
    return f"w:{name}"


def matmul(name: str, d: dict, n: int, k: int, act: int, bind: list[str]) -> dict:
    """Encoder matmul op: the 32x64 tile kernel with its smaller bit-equal alternatives when
    K % 32 == 0, else the 16x16 kernel (src/plan/layers.ts:36-49)."""
    constants = {"M": d["rows"], "N": n, "K": k, "ACT": act}
    if k % 32 == 0:
        return {
            "name": name, "kernel": "mmtile", "constants": constants, "bind": bind,
            "dispatch": [math.ceil(n / 64), "rows32"],
            "alts": [
                {"kernel": "mmtile8", "dispatch": [math.ceil(n / 32), "rows8"],
                 "maxRows": 16 * (127 // math.ceil(n / 32))},
                {"kernel": "mmtile16", "dispatch": [math.ceil(n / 32), "rows16"],
                 "maxRows": 32 * (95 // math.ceil(n / 64))},
            ],
        }
    return {"name": name, "kernel": "matmul", "constants": constants, "bind": bind,
            "dispatch": [math.ceil(n / 16), "rows16"]}


def matmul_attention(d: dict) -> bool:
    """Split (score / softmax / context) attention when D % 32 == 0, L % 32 == 0 and the f32 score
    matrix fits one binding (src/plan/layers.ts:54-56)."""
    return (d["headDim"] % 32 == 0 and d["length"] % 32 == 0
            and d["rows"] * d["heads"] * d["length"] * 4 <= SCORES_MAX_BYTES)


def relative_attention(d: dict, scale: float, rel: dict, t: dict) -> list[dict]:
    """DeBERTa attention as c2p, p2c, scores, relative softmax, context (src/plan/layers.ts:61-80)."""
    base = {"L": d["length"], "H": d["heads"], "D": d["headDim"]}
    rel_c = {"H": d["heads"], "D": d["headDim"], "ROWS": d["rows"], "NM": rel["nm"],
             "MOFF": rel["moff"], "L": d["length"]}
    tiles = d["heads"] * math.ceil(rel["nm"] / 64)
    return [
        {"name": "relC", "kernel": "attrel", "constants": {**rel_c, "PART": 0},
         "bind": ["qkv", _req(t.get("posKey"), "posKey"), "kinfo", "relidx", "c2p"],
         "dispatch": [tiles, "rows32"]},
        {"name": "relP", "kernel": "attrel", "constants": {**rel_c, "PART": 1},
         "bind": ["qkv", _req(t.get("posQuery"), "posQuery"), "kinfo", "relidx", "p2c"],
         "dispatch": [tiles, "rows32"]},
        {"name": "attS", "kernel": "attscore",
         "constants": {**base, "SCALE": 1 / scale, "ROWS": d["rows"]},
         "bind": ["qkv", "kinfo", "scores"],
         "dispatch": [d["heads"] * math.ceil(d["length"] / 64), "rows32"]},
        {"name": "attP", "kernel": "attsoftrel",
         "constants": {"L": d["length"], "H": d["heads"], "NM": rel["nm"], "MOFF": rel["moff"],
                       "INVSCALE": 1 / scale},
         "bind": ["mask", "relidx", "c2p", "p2c", "scores"], "dispatch": [d["heads"], "rows"]},
        {"name": "attV", "kernel": "attpv", "constants": {**base, "ROWS": d["rows"]},
         "bind": ["scores", "qkv", "mask", "kinfo", "ctx"],
         "dispatch": [d["heads"] * (d["headDim"] // 32), "rows32"]},
    ]


def standard_attention(d: dict, scale: float, window: int) -> list[dict]:
    """Split attention, else the flash kernel (D % 4 == 0, D <= 64, L % 32 == 0), else one
    workgroup per query row (src/plan/layers.ts:82-99)."""
    base = {"L": d["length"], "H": d["heads"], "D": d["headDim"]}
    if matmul_attention(d):
        return [
            {"name": "attS", "kernel": "attscore",
             "constants": {**base, "SCALE": scale, "ROWS": d["rows"]},
             "bind": ["qkv", "kinfo", "scores"],
             "dispatch": [d["heads"] * math.ceil(d["length"] / 64), "rows32"]},
            {"name": "attP", "kernel": "attsoftmax",
             "constants": {"L": d["length"], "H": d["heads"], "WINDOW": window},
             "bind": ["mask", "scores"], "dispatch": [d["heads"], "rows"]},
            {"name": "attV", "kernel": "attpv", "constants": {**base, "ROWS": d["rows"]},
             "bind": ["scores", "qkv", "mask", "kinfo", "ctx"],
             "dispatch": [d["heads"] * (d["headDim"] // 32), "rows32"]},
        ]
    constants = {**base, "SCALE": scale, "WINDOW": window}
    if d["headDim"] % 4 == 0 and d["headDim"] <= 64 and d["length"] % 32 == 0:
        return [{"name": "attn", "kernel": "mbflash", "constants": {**constants, "ROWS": d["rows"]},
                 "bind": ["qkv", "mask", "ctx"], "dispatch": [d["heads"], "rows32"]}]
    return [{"name": "attn", "kernel": "mbattention", "constants": constants,
             "bind": ["qkv", "mask", "ctx"], "dispatch": [d["heads"], "rows"]}]


def layernorm(name: str, d: dict, mode: int, bind: list[str]) -> dict:
    return {"name": name, "kernel": "layernorm",
            "constants": {"N": d["hidden"], "MODE": mode, "EPS": d["eps"]},
            "bind": bind, "dispatch": ["rows", 1]}


def add(name: str, d: dict, bind: list[str]) -> dict:
    return {"name": name, "kernel": "add",
            "constants": {"TOTAL": d["rows"] * d["hidden"], "N": d["hidden"], "MODE": 0,
                          "L": d["length"]},
            "bind": bind, "dispatch": [add_workgroups(d["rows"], d["hidden"]), 1]}


def post_norm_layer(d: dict, t: dict, act: int, attn_scale: float, standard: bool,
                    rel: dict | None) -> list[dict]:
    """qkv, attention, attnOut, lnA = LN(x + attnOut), ffn1, ffn2, lnF = LN(tmp + ffnOut)
    (src/plan/layers.ts:116-149)."""
    H = d["hidden"]
    I = d["intermediate"]
    ops = [matmul("qkv", d, 3 * H, H, 0, ["x", _req(t.get("qkvW"), "qkvW"), _w(t.get("qkvB")), "qkv"])]
    if standard:
        ops += standard_attention(d, attn_scale, 0)
    elif rel is not None and matmul_attention(d):
        ops += relative_attention(d, attn_scale, rel, t)
    else:
        ops.append({"name": "attn", "kernel": "attention",
                    "constants": {"L": d["length"], "H": d["heads"], "D": d["headDim"],
                                  "SCALE": attn_scale},
                    "bind": ["qkv", _req(t.get("posKey"), "posKey"),
                             _req(t.get("posQuery"), "posQuery"), "relidx", "mask", "ctx"],
                    "dispatch": [d["heads"], "rows"]})
    ops += [
        matmul("attnOut", d, H, H, 0, ["ctx", _req(t.get("attnOutW"), "attnOutW"),
                                       _w(t.get("attnOutB")), "attnOut"]),
        layernorm("lnA", d, 2, ["x", "attnOut", _req(t.get("attnNormW"), "attnNormW"),
                                _w(t.get("attnNormB")), "mask", "tmp"]),
        matmul("ffn1", d, I, H, act, ["tmp", _req(t.get("ffnInW"), "ffnInW"),
                                      _w(t.get("ffnInB")), "mid"]),
        matmul("ffn2", d, H, I, 0, ["mid", _req(t.get("ffnOutW"), "ffnOutW"),
                                    _w(t.get("ffnOutB")), "ffnOut"]),
        layernorm("lnF", d, 2, ["tmp", "ffnOut", _req(t.get("ffnNormW"), "ffnNormW"),
                                _w(t.get("ffnNormB")), "mask", "x"]),
    ]
    return ops


def pre_norm_layer(d: dict, t: dict, stream: str, first_norm: bool, attn_scale: float,
                   window: int, rope: bool, ffn: dict, rope_table: str = "cossin") -> list[dict]:
    """lnA (optional), qkv, rope (optional), attention, attnOut, addA, lnF, ffnIn, geglu, ffnOut
    (or lin1, lin2), addF; residual adds in storage precision (src/plan/layers.ts:161-204)."""
    H = d["hidden"]
    I = d["intermediate"]
    ops = []
    if first_norm:
        ops.append(layernorm("lnA", d, 0, [stream, "dummy", _req(t.get("attnNormW"), "attnNormW"),
                                          _w(t.get("attnNormB")), "mask", "normed"]))
    ops.append(matmul("qkv", d, 3 * H, H, 0, ["normed" if first_norm else stream,
                                              _req(t.get("qkvW"), "qkvW"), _w(t.get("qkvB")), "qkv"]))
    if rope:
        ops.append({"name": "rope", "kernel": "rope",
                    "constants": {"L": d["length"], "H": d["heads"], "D": d["headDim"]},
                    "bind": ["qkv", rope_table], "dispatch": ["rows", 2 * d["heads"]]})
    ops += standard_attention(d, attn_scale, window)
    ops.append(matmul("attnOut", d, H, H, 0, ["ctx", _req(t.get("attnOutW"), "attnOutW"),
                                              _w(t.get("attnOutB")), "attnOut"]))
    ops.append(add("addA", d, [stream, "attnOut"]))
    ops.append(layernorm("lnF", d, 0, [stream, "dummy", _req(t.get("ffnNormW"), "ffnNormW"),
                                      _w(t.get("ffnNormB")), "mask", "normed"]))
    if ffn["kind"] == "geglu":
        ops.append(matmul("ffnIn", d, 2 * I, H, 0, ["normed", _req(t.get("ffnInW"), "ffnInW"),
                                                    _w(t.get("ffnInB")), "mid"]))
        ops.append({"name": "geglu", "kernel": "geglu", "constants": {"I": I},
                    "bind": ["mid", "gate"], "dispatch": ["rows", 1]})
        ops.append(matmul("ffnOut", d, H, I, 0, ["gate", _req(t.get("ffnOutW"), "ffnOutW"),
                                                 _w(t.get("ffnOutB")), "ffnOut"]))
    else:
        ops.append(matmul("lin1", d, ffn["width"], H, ffn["act"],
                          ["normed", _req(t.get("ffnInW"), "ffnInW"), _w(t.get("ffnInB")), "mid"]))
        ops.append(matmul("lin2", d, H, ffn["width"], 0,
                          ["mid", _req(t.get("ffnOutW"), "ffnOutW"), _w(t.get("ffnOutB")), "ffnOut"]))
    ops.append(add("addF", d, [stream, "ffnOut"]))
    return ops
