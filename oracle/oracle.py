"""TEST INFRASTRUCTURE — host side of the CPU parity oracle (and CPU baseline).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this module; the
product path never does.

A Python statement of the reference's WASM executor host, src/plan/wasm.ts: weights with at least
16 output columns bound as a matmul weight are packed into 16-column panels at load
(src/plan/wasm.ts:28-51, 231-255); split attention sequences fuse into one attention op
(src/plan/wasm.ts:53-82); each op becomes one record of pointer, integer and float arguments
(src/plan/wasm.ts:329-407) run by kh_oracle.c. Buffers hold f32 (the oracle runs f32 plans only,
src/plan/wasm.ts:257-263) with 64 spare bytes after each (src/plan/wasm.ts:12-14).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libkh_oracle.so")

MATMUL = {"matmul", "mmtile", "mmtile8", "mmtile16"}
CODE = {"gemmP": 1, "gemmNT": 2, "layernorm": 3, "embln": 4, "add": 5, "gather": 6, "pool": 7,
        "geglu": 8, "rope": 9, "attscore": 11, "attsoftmax": 12, "attpv": 13, "attrel": 14,
        "attsoftrel": 15, "attstd": 16, "attrelf": 17, "masklogits": 18}
PAD_FLOATS = 16  # 64 spare bytes per allocation


class KhoOp(ctypes.Structure):
    _fields_ = [("code", ctypes.c_int32), ("rows_fixed", ctypes.c_int32), ("pad", ctypes.c_int32 * 2),
                ("p", ctypes.c_void_p * 8), ("v", ctypes.c_int32 * 14), ("f", ctypes.c_float * 2)]


def build(force: bool = False) -> str:
    """Compile kh_oracle.c (make in this directory)."""
    if force or not os.path.exists(LIB_PATH):
        subprocess.run(["make", "-s", "-C", HERE, "-B" if force else "all"], check=True)
    return LIB_PATH


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
        _lib.kho_run.restype = ctypes.c_int
        _lib.kho_run.argtypes = [ctypes.POINTER(KhoOp), ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                 ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t,
                                 ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                 ctypes.c_long]
        for name in ("kho_vexp", "kho_vgelu", "kho_gelu"):
            getattr(_lib, name).restype = ctypes.c_float
            getattr(_lib, name).argtypes = [ctypes.c_float]
        if _lib.kho_op_size() != ctypes.sizeof(KhoOp):
            raise RuntimeError("kh_oracle: op record layout differs from the host's")
    return _lib


def panel_weights(plans) -> set[str]:
    """Tensors bound as a matmul weight with N >= 16 (src/plan/wasm.ts:28-51)."""
    role: dict[str, str] = {}
    for plan in plans:
        for seg in plan["segments"]:
            for op in seg["ops"]:
                for i, bid in enumerate(op["bind"]):
                    if not bid.startswith("w:"):
                        continue
                    name = bid[2:]
                    r = ("kn" if op["constants"]["N"] >= 16 else "nk") if (op["kernel"] in MATMUL and i == 1) else "plain"
                    if role.get(name, r) != r:
                        raise ValueError(f"weight {name} is bound as {role[name]} and as {r}")
                    role[name] = r
    return {n for n, r in role.items() if r == "kn"}


def fuse_attention(ops: list[dict]) -> list[dict]:
    """attscore+attsoftmax+attpv -> mbattention; attrel c2p + attrel p2c + attscore + attsoftrel +
    attpv -> attention with SCALE = 1 / attscore's SCALE (src/plan/wasm.ts:53-82)."""
    out = []
    i = 0
    k = lambda j: ops[j]["kernel"] if j < len(ops) else None
    while i < len(ops):
        o = ops[i]
        if (o["kernel"] == "attscore" and k(i + 1) == "attsoftmax" and k(i + 2) == "attpv"
                and ops[i + 1]["bind"][1] == o["bind"][2] and ops[i + 2]["bind"][0] == o["bind"][2]):
            c = o["constants"]
            out.append({"name": f"{o['name']}+fused", "kernel": "mbattention",
                        "constants": {"L": c["L"], "H": c["H"], "D": c["D"], "SCALE": c["SCALE"],
                                      "WINDOW": ops[i + 1]["constants"]["WINDOW"]},
                        "bind": [o["bind"][0], ops[i + 1]["bind"][0], ops[i + 2]["bind"][4]],
                        "dispatch": o["dispatch"]})
            i += 3
        elif (o["kernel"] == "attrel" and o["constants"]["PART"] == 0 and k(i + 1) == "attrel"
              and ops[i + 1]["constants"]["PART"] == 1 and k(i + 2) == "attscore"
              and k(i + 3) == "attsoftrel" and k(i + 4) == "attpv"):
            s = ops[i + 2]
            out.append({"name": f"{s['name']}+fused", "kernel": "attention",
                        "constants": {"L": s["constants"]["L"], "H": s["constants"]["H"],
                                      "D": s["constants"]["D"], "SCALE": 1 / s["constants"]["SCALE"]},
                        "bind": [o["bind"][0], o["bind"][1], ops[i + 1]["bind"][1], o["bind"][3],
                                 ops[i + 3]["bind"][0], ops[i + 4]["bind"][4]],
                        "dispatch": s["dispatch"]})
            i += 5
        else:
            out.append(o)
            i += 1
    return out


class OracleRuntime:
    """The weight arena: f32 tensors, paneled where a plan binds them as a wide matmul weight."""

    def __init__(self, weights: dict[str, np.ndarray], plans: list[dict]):
        self.panels = panel_weights(plans)
        self.w: dict[str, np.ndarray] = {}
        for name, t in weights.items():
            t = np.asarray(t, dtype=np.float32)
            if name in self.panels:
                N, K = t.shape
                nb = -(-N // 16)
                pan = np.zeros((nb * 16, K), dtype=np.float32)
                pan[:N] = t
                # [ceil(N/16)][K][16]: element (n, k) at (n // 16) K 16 + k 16 + n % 16
                arr = pan.reshape(nb, 16, K).transpose(0, 2, 1).copy()
                self.w[name] = np.concatenate([arr.reshape(-1), np.zeros(PAD_FLOATS, np.float32)])
            else:
                self.w[name] = np.concatenate([t.reshape(-1), np.zeros(PAD_FLOATS, np.float32)])

    def plan(self, plan: dict, threads: int = 1) -> "OraclePlan":
        if plan["f16"]:
            raise ValueError("the oracle runs f32 plans")
        return OraclePlan(self, plan, threads)


class OraclePlan:
    """One plan: buffers, op records, upload / run / read_output like WasmPlan
    (src/plan/wasm.ts:275-483)."""

    def __init__(self, rt: OracleRuntime, plan: dict, threads: int = 1):
        self.rt = rt
        self.plan = plan
        self.threads = threads
        self.length = plan["length"]
        self.batch = plan["batch"]
        ops = fuse_attention([op for s in plan["segments"] for op in s["ops"]])
        used = {b for o in ops for b in o["bind"]} | {plan["output"]["buffer"]} | set(plan["inputs"].values())
        self.bufs: dict[str, np.ndarray] = {}
        for d in plan["buffers"]:
            if d["id"] not in used:
                continue
            nfl = -(-d["bytes"] // 4) + PAD_FLOATS
            buf = np.zeros(nfl, dtype=np.float32)
            if "init" in d:
                raw = np.ascontiguousarray(d["init"]).view(np.uint8)
                buf.view(np.uint8)[:raw.size] = raw
            self.bufs[d["id"]] = buf
        L = plan["length"]
        scratch = 0
        for o in ops:
            if o["kernel"] == "attention":
                scratch = max(scratch, 5 * L * L + (2 * L + 16) * o["constants"]["D"])
            elif o["kernel"] in ("mbattention", "mbflash"):
                scratch = max(scratch, L * L + (L + 16) * o["constants"]["D"])
        self.scratch_per_thread = (-(-scratch // 16)) * 16 if scratch else 0
        self.scratch = np.zeros(max(1, self.scratch_per_thread * max(1, threads)), dtype=np.float32)
        self.kinfo = np.zeros(2 * plan["batch"] + 16, dtype=np.int32)
        self.ops = ops
        self.recs = (KhoOp * len(ops))()
        for i, op in enumerate(ops):
            self._encode(op, self.recs[i])

    def _at(self, bid: str) -> int:
        if bid.startswith("w:"):
            arr = self.rt.w.get(bid[2:])
            if arr is None:
                raise KeyError(f"oracle plan: weight {bid} missing")
        else:
            arr = self.bufs.get(bid)
            if arr is None:
                raise KeyError(f"oracle plan: buffer {bid} missing")
        return arr.ctypes.data

    def view(self, bid: str, dtype=np.float32) -> np.ndarray:
        d = next(x for x in self.plan["buffers"] if x["id"] == bid)
        return self.bufs[bid].view(dtype)[: d["bytes"] // 4]

    def _encode(self, op: dict, r: KhoOp) -> None:
        c = op["constants"]
        k = op["kernel"]
        for i, bid in enumerate(op["bind"]):
            if bid.startswith("w:") and bid[2:] in self.rt.panels and not (k in MATMUL and i == 1):
                raise ValueError(f"oracle plan: {op['name']} reads the paneled weight {bid} as a plain tensor")
        b = lambda i: self._at(op["bind"][i])
        fixed = lambda d, n: n if isinstance(d, int) else -1
        ptr, ints, fl = [], [], []
        if k in MATMUL:
            code = CODE["gemmP"] if op["bind"][1][2:] in self.rt.panels else CODE["gemmNT"]
            rows = fixed(op["dispatch"][1], c["M"])
            ptr = [b(0), b(1), b(2), b(3)]
            ints = [c["N"], c["K"], c["ACT"], c["M"]]
        elif k == "layernorm":
            code, rows = CODE["layernorm"], fixed(op["dispatch"][0], op["dispatch"][0])
            ptr = [b(i) for i in range(6)]
            ints, fl = [c["N"], c["MODE"]], [c["EPS"]]
        elif k == "embln":
            code, rows = CODE["embln"], -1
            ptr = [b(i) for i in range(8)]
            ints = [c["N"], c["L"], c["OFFSET"], c["MAXPOS"], c["MASKMUL"], c["POSIDS"]]
            fl = [c["EPS"]]
        elif k == "add":
            code, rows = CODE["add"], -1
            ptr, ints = [b(0), b(1)], [c["TOTAL"], c["N"], c["MODE"], c["L"]]
        elif k == "gather":
            code, rows = CODE["gather"], -1
            nbytes = next(x["bytes"] for x in self.plan["buffers"] if x["id"] == op["bind"][0])
            ptr, ints = [b(0), b(1), b(2)], [c["K"], c["D"], c["L"], nbytes // 12]
        elif k == "masklogits":
            # total = the marker buffer's u32 count / 3 (src/plan/wasm.ts:393-394)
            code, rows = CODE["masklogits"], -1
            nbytes = next(x["bytes"] for x in self.plan["buffers"] if x["id"] == op["bind"][1])
            ptr, ints, fl = [b(0), b(1), b(2)], [c["K"], nbytes // 12], [c["TEMP"]]
        elif k == "pool":
            code, rows = CODE["pool"], -1
            ptr, ints = [b(0), b(1), b(2)], [c["L"], c["N"], c["MODE"], op["dispatch"][1]]
        elif k == "geglu":
            code, rows = CODE["geglu"], -1
            ptr, ints = [b(0), b(1)], [c["I"]]
        elif k == "rope":
            code, rows = CODE["rope"], -1
            ptr, ints = [b(0), b(1)], [c["L"], c["H"], c["D"]]
        elif k == "attscore":
            code, rows = CODE["attscore"], -1
            ptr, ints, fl = [b(0), b(2)], [c["L"], c["H"], c["D"]], [c["SCALE"]]
        elif k == "attsoftmax":
            code, rows = CODE["attsoftmax"], -1
            ptr, ints = [b(0), b(1)], [c["L"], c["H"], c["WINDOW"]]
        elif k == "attpv":
            code, rows = CODE["attpv"], -1
            ptr, ints = [b(0), b(1), b(4)], [c["L"], c["H"], c["D"]]
        elif k == "attrel":
            code, rows = CODE["attrel"], -1
            ptr = [b(0), b(1), b(3), b(4)]
            ints = [c["H"], c["D"], c["NM"], c["MOFF"], c["PART"], c["L"]]
        elif k == "attsoftrel":
            code, rows = CODE["attsoftrel"], -1
            ptr = [b(0), b(1), b(2), b(3), b(4)]
            ints, fl = [c["L"], c["H"], c["NM"], c["MOFF"]], [c["INVSCALE"]]
        elif k in ("mbattention", "mbflash"):
            code, rows = CODE["attstd"], -1
            ptr = [b(0), b(1), b(2)]
            ints, fl = [c["L"], c["H"], c["D"], c["WINDOW"]], [c["SCALE"]]
        elif k == "attention":
            code, rows = CODE["attrelf"], -1
            ptr = [b(i) for i in range(6)]
            ints, fl = [c["L"], c["H"], c["D"]], [c["SCALE"]]
        else:
            raise ValueError(f"oracle plan: kernel {k} has no computation")
        for v in ints:
            if int(v) != v:
                raise ValueError(f"oracle plan: {op['name']} argument {v} is not an integer")
        r.code = code
        r.rows_fixed = int(rows)
        for i, p in enumerate(ptr):
            r.p[i] = p
        for i, v in enumerate(ints):
            r.v[i] = int(v)
        for i, v in enumerate(fl):
            r.f[i] = float(v)

    def upload(self, embeddings: np.ndarray, mask: np.ndarray, type_ids: np.ndarray | None = None,
               markers: np.ndarray | None = None, qtype=None) -> None:
        """Copies the inputs into the plan's buffers (src/plan/wasm.ts:409-440)."""
        inp = self.plan["inputs"]

        def put(bid, src):
            src = np.ascontiguousarray(src)
            dst = self.bufs[bid].view(np.uint8)
            nbytes = next(x["bytes"] for x in self.plan["buffers"] if x["id"] == bid)
            if src.nbytes > nbytes:
                raise ValueError(f"oracle plan: input {bid} has {src.nbytes} B, the buffer {nbytes}")
            dst[:src.nbytes] = src.view(np.uint8).reshape(-1)

        if np.asarray(embeddings).dtype != np.float32:
            raise TypeError("the oracle takes f32 word rows")
        put(inp["embeddings"], embeddings)
        put(inp["mask"], np.asarray(mask, dtype=np.float32))
        if "typeIds" in inp:
            if type_ids is None:
                raise ValueError("plan needs typeIds")
            put(inp["typeIds"], np.asarray(type_ids, dtype=np.uint32))
        if "markers" in inp:
            if markers is None:
                raise ValueError("plan needs packed markers")
            put(inp["markers"], np.asarray(markers, dtype=np.uint32))
        rs = self.plan.get("rowSelect")
        if rs:
            # the type row of each sequence (src/plan/wasm.ts:429-439): qtypes[b] ?? 0
            q = list(qtype) if isinstance(qtype, (list, tuple, np.ndarray)) else [qtype or 0]
            table = self.rt.w[rs["table"][2:]].reshape(-1)
            n = rs["rowBytes"] // 4
            dst = self.bufs[rs["dst"]]
            for b in range(self.batch):
                r = int(q[b]) if b < len(q) else 0
                dst[b * n:(b + 1) * n] = table[r * n:(r + 1) * n]

    def run(self, rows: int, rb: int = 16, cb: int = 64, qb: int = 32, min_work: int = 1 << 16) -> None:
        if rows < 1 or rows > self.length * self.batch:
            raise ValueError(f"oracle plan: {rows} rows, the plan has {self.length * self.batch}")
        rc = lib().kho_run(self.recs, len(self.ops), self.length, self.batch,
                           self.bufs[self.plan["inputs"]["mask"]].ctypes.data, self.kinfo.ctypes.data,
                           self.scratch.ctypes.data, self.scratch_per_thread, rows, self.threads,
                           rb, cb, qb, min_work)
        if rc != 0:
            raise RuntimeError("oracle: unknown op code")

    def read_output(self) -> np.ndarray:
        o = self.plan["output"]
        return self.bufs[o["buffer"]][: o["rows"] * o["cols"]].copy()
