"""HIP backend over the C ABI of libkh_hip.so (include/kh_hip.h).

`HipBackend` and `HipPlanRunner` mirror the reference's Backend / PlanRunner seam
(src/backend.ts:14-46) method for method, so the parity tests and the benchmark drive the HIP
executor the way EncoderModel drives the WebGPU or WASM executors. There is no fallback: if the
library is missing or a call fails, the error surfaces (a GPU run never silently computes on the
CPU).
"""
from __future__ import annotations

import ctypes
import json
import os

import numpy as np

from .plan.build import plan_inits, plan_json

HERE = os.path.dirname(os.path.abspath(__file__))
# KH_LIB selects another build of the same library (A/B timing of kernel variants)
LIB_PATH = os.environ.get("KH_LIB") or os.path.join(HERE, "libkh_hip.so")

KH_F32, KH_F16, KH_U32 = 0, 1, 2
ERRORS = {1: "EINVAL", 2: "EUNSUPPORTED", 3: "EHIP", 4: "ENOMEM", 5: "ELOST"}

# every entry point declared in include/kh_hip.h
EXPORTS = [
    "kh_last_error", "kh_abi_version", "kh_ctx_create", "kh_ctx_destroy", "kh_weight_add",
    "kh_ctx_weight_bytes", "kh_words_set", "kh_plan_check", "kh_plan_create", "kh_plan_init_buffer",
    "kh_plan_info_get", "kh_upload", "kh_upload_ids", "kh_upload_markers", "kh_upload_qtypes", "kh_run", "kh_read_output", "kh_sync",
    "kh_last_run_ms", "kh_profile", "kh_packed_rows", "kh_plan_destroy", "kh_manifest_check",
    "kh_load_manifest", "kh_sha256", "kh_row_checksum", "kh_scores", "kh_read_scores", "kh_rank",
    "kh_sched_create", "kh_sched_run", "kh_sched_destroy", "kh_trace", "kh_trace_read", "kh_plan_read_buffer",
]

# kh_scores kinds
SCORES_SOFTMAX, SCORES_SIGMOID, SCORES_RAW, SCORES_L2, SCORES_OPTIONS = 0, 1, 2, 3, 4

# kh_load_manifest / kh_manifest_check flags
LOAD_NO_SHA256, LOAD_CHECK_ROWS, LOAD_NO_WORDS = 1, 2, 4


class KhError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"kh {ERRORS.get(code, code)}: {message}")
        self.code = code


class PlanInfo(ctypes.Structure):
    _fields_ = [("length", ctypes.c_int32), ("batch", ctypes.c_int32), ("markers", ctypes.c_int32),
                ("f16", ctypes.c_int32), ("bytes", ctypes.c_uint64), ("out_rows", ctypes.c_int32),
                ("out_cols", ctypes.c_int32), ("launches", ctypes.c_int32), ("streams", ctypes.c_int32)]


class ManifestInfo(ctypes.Structure):
    _fields_ = [("version", ctypes.c_int32), ("tensors", ctypes.c_int32), ("shards", ctypes.c_int32),
                ("words_dtype", ctypes.c_int32), ("words_rows", ctypes.c_int64), ("words_width", ctypes.c_int64),
                ("tensor_bytes", ctypes.c_uint64), ("file_bytes", ctypes.c_uint64), ("read_ms", ctypes.c_double),
                ("sha256_ms", ctypes.c_double), ("rows_ms", ctypes.c_double), ("upload_ms", ctypes.c_double)]

    def as_dict(self) -> dict:
        return {name: getattr(self, name) for name, _ in self._fields_}


class SchedStats(ctypes.Structure):
    _fields_ = [("chunks", ctypes.c_int32), ("sequences", ctypes.c_int32), ("tokens", ctypes.c_int64),
                ("wall_ms", ctypes.c_double), ("gpu_ms", ctypes.c_double), ("host_ms", ctypes.c_double)]

    def as_dict(self) -> dict:
        return {name: getattr(self, name) for name, _ in self._fields_}


class LaunchStat(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 48), ("kernel", ctypes.c_char * 24), ("ms", ctypes.c_float),
                ("reserved", ctypes.c_float), ("flops", ctypes.c_double), ("bytes", ctypes.c_double)]


_lib = None


def lib() -> ctypes.CDLL:
    """The in-tree libkh_hip.so; raises when it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is not built (python -m kleinhirn_amd.build)")
    L = ctypes.CDLL(LIB_PATH)
    vp, sz, i32, i64 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int32, ctypes.c_int64
    L.kh_last_error.restype = ctypes.c_char_p
    L.kh_last_error.argtypes = []
    L.kh_abi_version.restype = ctypes.c_int
    sigs = {
        "kh_ctx_create": [ctypes.c_int, ctypes.POINTER(vp)],
        "kh_ctx_destroy": [vp],
        "kh_weight_add": [vp, ctypes.c_char_p, ctypes.c_int, ctypes.POINTER(i64), ctypes.c_int, vp, sz],
        "kh_ctx_weight_bytes": [vp, ctypes.POINTER(ctypes.c_uint64)],
        "kh_words_set": [vp, ctypes.c_int, i64, i64, vp, sz],
        "kh_plan_check": [vp, ctypes.c_char_p, sz],
        "kh_plan_create": [vp, ctypes.c_char_p, sz, ctypes.POINTER(vp)],
        "kh_plan_init_buffer": [vp, ctypes.c_char_p, vp, sz],
        "kh_plan_info_get": [vp, ctypes.POINTER(PlanInfo)],
        "kh_upload": [vp, vp, sz, vp, sz, vp, sz],
        "kh_upload_ids": [vp, vp, sz, vp, sz, vp, sz],
        "kh_upload_markers": [vp, vp, sz],
        "kh_upload_qtypes": [vp, vp, sz],
        "kh_run": [vp, i32],
        "kh_read_output": [vp, vp, sz],
        "kh_sync": [vp],
        "kh_last_run_ms": [vp, ctypes.POINTER(ctypes.c_float)],
        "kh_profile": [vp, i32, ctypes.POINTER(LaunchStat), i32, ctypes.POINTER(i32)],
        "kh_packed_rows": [vp, ctypes.POINTER(i64)],
        "kh_plan_read_buffer": [vp, ctypes.c_char_p, i32, vp, sz],
        "kh_plan_destroy": [vp],
        "kh_manifest_check": [ctypes.c_char_p, ctypes.c_int, ctypes.POINTER(ManifestInfo)],
        "kh_load_manifest": [vp, ctypes.c_char_p, ctypes.c_int, ctypes.POINTER(ManifestInfo)],
        "kh_sha256": [vp, sz, ctypes.POINTER(ctypes.c_uint8)],
        "kh_row_checksum": [vp, sz, ctypes.c_uint32, ctypes.c_uint32, ctypes.POINTER(ctypes.c_uint32)],
        "kh_scores": [vp, i64, i32, ctypes.c_int, vp, vp],
        "kh_read_scores": [vp, ctypes.c_int, vp, sz, vp, sz],
        "kh_rank": [vp, i64, vp],
        "kh_sched_create": [ctypes.POINTER(vp), i32, ctypes.POINTER(vp)],
        "kh_sched_run": [vp, vp, vp, i64, vp, i64, vp, sz, ctypes.POINTER(SchedStats)],
        "kh_sched_destroy": [vp],
        "kh_trace": [vp, i32],
        "kh_trace_read": [vp, ctypes.POINTER(LaunchStat), i32, ctypes.POINTER(i32)],
    }
    for name, args in sigs.items():
        fn = getattr(L, name)
        fn.restype = ctypes.c_int
        fn.argtypes = args
    _lib = L
    return L


def _check(rc: int) -> None:
    if rc != 0:
        raise KhError(rc, lib().kh_last_error().decode("utf-8", "replace"))


def manifest_check(path: str, flags: int = 0) -> dict:
    """Reads and checks a manifest directory without a device (kh_manifest_check)."""
    info = ManifestInfo()
    _check(lib().kh_manifest_check(os.fsencode(path), flags, ctypes.byref(info)))
    return info.as_dict()


def sha256(data: bytes) -> str:
    """Hex SHA-256 through the library's implementation (kh_sha256)."""
    buf = np.frombuffer(bytes(data), dtype=np.uint8)
    out = (ctypes.c_uint8 * 32)()
    _check(lib().kh_sha256(buf.ctypes.data if buf.size else None, buf.size, out))
    return bytes(out).hex()


def row_checksum(row: bytes, row_id: int, salt: int) -> int:
    """words.bin row checksum through the library (kh_row_checksum)."""
    buf = np.frombuffer(bytes(row), dtype=np.uint8)
    out = ctypes.c_uint32()
    _check(lib().kh_row_checksum(buf.ctypes.data if buf.size else None, buf.size, row_id & 0xFFFFFFFF,
                                 salt & 0xFFFFFFFF, ctypes.byref(out)))
    return int(out.value)


def scores(logits: np.ndarray, kind: int = SCORES_SOFTMAX) -> tuple[np.ndarray, np.ndarray]:
    """Scores and label index per row of a [rows, cols] f32 array (kh_scores)."""
    x = np.ascontiguousarray(logits, dtype=np.float32)
    if x.ndim == 1:
        x = x[None]
    out = np.empty_like(x)
    idx = np.empty(x.shape[0], dtype=np.int32)
    _check(lib().kh_scores(x.ctypes.data, x.shape[0], x.shape[1], kind, out.ctypes.data, idx.ctypes.data))
    return out, idx


def rank(values: np.ndarray) -> np.ndarray:
    """Indices by score, highest first, ties in index order (kh_rank)."""
    x = np.ascontiguousarray(values, dtype=np.float32).ravel()
    order = np.empty(x.size, dtype=np.int32)
    _check(lib().kh_rank(x.ctypes.data if x.size else None, x.size, order.ctypes.data if x.size else None))
    return order


def _ptr(a: np.ndarray | None):
    return None if a is None else ctypes.c_void_p(a.ctypes.data)


class HipPlanRunner:
    """PlanRunner (src/backend.ts:14-28) of one plan on the HIP device."""

    def __init__(self, backend: "HipBackend", plan: dict):
        self.backend = backend
        self.plan = plan
        doc = json.dumps(plan_json(plan)).encode("utf-8")
        h = ctypes.c_void_p()
        _check(lib().kh_plan_create(backend.ctx, doc, len(doc), ctypes.byref(h)))
        self.h = h
        for bid, raw in plan_inits(plan).items():
            self.init_buffer(bid, raw)
        self.length = plan["length"]
        self.batch = plan["batch"]
        self.markers = plan["markers"]
        self._keep = None

    def init_buffer(self, bid: str, raw: bytes | np.ndarray) -> None:
        """BufferDecl.init of one buffer (src/plan/executor.ts:118-124)."""
        buf = np.ascontiguousarray(np.frombuffer(bytes(raw), dtype=np.uint8))
        _check(lib().kh_plan_init_buffer(self.h, bid.encode(), _ptr(buf), buf.nbytes))

    @property
    def info(self) -> PlanInfo:
        info = PlanInfo()
        _check(lib().kh_plan_info_get(self.h, ctypes.byref(info)))
        return info

    @property
    def bytes(self) -> int:
        return int(self.info.bytes)

    def _markers(self, packed) -> None:
        # RunInput.packedMarkers of plans with a markers input (src/plan/executor.ts:385-388)
        if "markers" not in self.plan["inputs"]:
            return
        if packed is None:
            raise ValueError("plan needs packedMarkers")
        packed = np.ascontiguousarray(packed, dtype=np.uint32)
        _check(lib().kh_upload_markers(self.h, _ptr(packed), packed.size))

    def _qtypes(self, qtype) -> None:
        # RunInput.qtype of plans with a rowSelect: one number, or one per sequence
        if not self.plan.get("rowSelect"):
            return
        q = np.atleast_1d(np.asarray(0 if qtype is None else qtype, dtype=np.int64))
        if np.any(q < 0):
            raise ValueError("qtype must not be negative")
        q = np.ascontiguousarray(q, dtype=np.uint32)
        _check(lib().kh_upload_qtypes(self.h, _ptr(q), q.size))

    def upload(self, inp: dict) -> None:
        """RunInput {embeddings, mask, typeIds?, packedMarkers?, qtype?} (src/plan/executor.ts:25-32)."""
        self._markers(inp.get("packedMarkers"))
        self._qtypes(inp.get("qtype"))
        emb = np.ascontiguousarray(inp["embeddings"])
        want = np.float16 if self.plan["f16"] else np.float32
        if emb.dtype != want:
            raise TypeError(f"word rows must be {np.dtype(want).name} for this plan")
        mask = np.ascontiguousarray(inp["mask"], dtype=np.float32)
        tt = inp.get("typeIds")
        tt = None if tt is None else np.ascontiguousarray(tt, dtype=np.uint32)
        _check(lib().kh_upload(self.h, _ptr(emb), emb.nbytes, _ptr(mask), mask.size, _ptr(tt),
                               0 if tt is None else tt.size))

    def upload_ids(self, ids: np.ndarray, mask: np.ndarray, type_ids: np.ndarray | None = None,
                   packed_markers: np.ndarray | None = None, qtype=None) -> None:
        self._markers(packed_markers)
        self._qtypes(qtype)
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        mask = np.ascontiguousarray(mask, dtype=np.float32)
        tt = None if type_ids is None else np.ascontiguousarray(type_ids, dtype=np.uint32)
        _check(lib().kh_upload_ids(self.h, _ptr(ids), ids.size, _ptr(mask), mask.size, _ptr(tt),
                                   0 if tt is None else tt.size))

    def run(self, seq_len: int, capture: bool = False) -> None:
        if capture:
            raise RuntimeError("capture is a WebGPU parity tool; the HIP runner has no capture")
        _check(lib().kh_run(self.h, int(seq_len)))

    def sync(self) -> None:
        _check(lib().kh_sync(self.h))

    def read_output(self) -> np.ndarray:
        o = self.plan["output"]
        out = np.empty(o["rows"] * o["cols"], dtype=np.float32)
        _check(lib().kh_read_output(self.h, _ptr(out), out.size))
        return out

    def read_scores(self, kind: int = SCORES_SOFTMAX) -> tuple[np.ndarray, np.ndarray]:
        """The output's scores and label per row (kh_read_scores; pooled heads)."""
        o = self.plan["output"]
        out = np.empty((o["rows"], o["cols"]), dtype=np.float32)
        idx = np.empty(o["rows"], dtype=np.int32)
        _check(lib().kh_read_scores(self.h, kind, out.ctypes.data, out.size, idx.ctypes.data, idx.size))
        return out, idx

    def read_capture(self):
        raise RuntimeError("capture is a WebGPU parity tool; the HIP runner has no capture")

    def assert_capturable(self) -> None:
        raise RuntimeError("capture is a WebGPU parity tool; the HIP runner has no capture")

    def last_run_ms(self) -> float:
        ms = ctypes.c_float()
        _check(lib().kh_last_run_ms(self.h, ctypes.byref(ms)))
        return float(ms.value)

    def packed_rows(self) -> int:
        n = ctypes.c_int64()
        _check(lib().kh_packed_rows(self.h, ctypes.byref(n)))
        return int(n.value)

    def read_buffer(self, bid: str, nbytes: int, half: int = 0) -> np.ndarray:
        """Raw bytes of plan buffer `bid` after the last run (`half` 1: the second half of a split
        batch), as uint8 (kh_plan_read_buffer)."""
        out = np.zeros(nbytes, dtype=np.uint8)
        _check(lib().kh_plan_read_buffer(self.h, bid.encode(), int(half), out.ctypes.data, out.nbytes))
        return out

    def profile(self, rows: int) -> list[dict]:
        cap = 4096
        arr = (LaunchStat * cap)()
        n = ctypes.c_int32()
        _check(lib().kh_profile(self.h, int(rows), arr, cap, ctypes.byref(n)))
        return [{"name": arr[i].name.decode(), "kernel": arr[i].kernel.decode(), "ms": float(arr[i].ms),
                 "flops": float(arr[i].flops), "bytes": float(arr[i].bytes)} for i in range(min(n.value, cap))]

    def trace(self, on: bool) -> None:
        """Record HIP events around every launch of the following runs (kh_trace)."""
        _check(lib().kh_trace(self.h, 1 if on else 0))

    def trace_read(self) -> list[dict]:
        """The launches recorded since the last read, with their GPU ms (kh_trace_read)."""
        n = ctypes.c_int32()
        _check(lib().kh_trace_read(self.h, None, 0, ctypes.byref(n)))
        cap = max(1, n.value)
        arr = (LaunchStat * cap)()
        _check(lib().kh_trace_read(self.h, arr, cap, ctypes.byref(n)))
        return [{"name": arr[i].name.decode(), "kernel": arr[i].kernel.decode(), "ms": float(arr[i].ms),
                 "flops": float(arr[i].flops), "bytes": float(arr[i].bytes)} for i in range(min(n.value, cap))]

    def destroy(self) -> None:
        if self.h:
            _check(lib().kh_plan_destroy(self.h))
            self.h = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


class HipBackend:
    """Backend (src/backend.ts:30-46) on one HIP device."""

    kind = "hip"

    def __init__(self, weights: dict[str, np.ndarray], device: int = 0):
        h = ctypes.c_void_p()
        _check(lib().kh_ctx_create(int(device), ctypes.byref(h)))
        self.ctx = h
        self.device = device
        for name, t in weights.items():
            self.add_weight(name, t)

    @classmethod
    def from_manifest(cls, path: str, device: int = 0, flags: int = 0) -> "HipBackend":
        """A backend whose weights (and device word table) come straight from a manifest directory
        (kh_load_manifest: loadWeights of src/webgpu-backend.ts:53-101 with the checks of
        src/weights.ts:150-173). `load_info` holds the sizes and timings of the load."""
        be = cls({}, device)
        info = ManifestInfo()
        _check(lib().kh_load_manifest(be.ctx, os.fsencode(path), flags, ctypes.byref(info)))
        be.load_info = info.as_dict()
        return be

    def add_weight(self, name: str, t: np.ndarray) -> None:
        t = np.ascontiguousarray(t)
        dtype = {np.dtype(np.float32): KH_F32, np.dtype(np.float16): KH_F16, np.dtype(np.uint32): KH_U32}[t.dtype]
        shape = (ctypes.c_int64 * max(1, t.ndim))(*t.shape)
        _check(lib().kh_weight_add(self.ctx, name.encode(), dtype, shape, t.ndim, _ptr(t), t.nbytes))

    def set_words(self, table: np.ndarray) -> None:
        """Device-resident word table for runs by token id (upload_ids)."""
        t = np.ascontiguousarray(table)
        dtype = KH_F16 if t.dtype == np.float16 else KH_F32
        _check(lib().kh_words_set(self.ctx, dtype, t.shape[0], t.shape[1], _ptr(t), t.nbytes))

    @property
    def weight_bytes(self) -> int:
        v = ctypes.c_uint64()
        _check(lib().kh_ctx_weight_bytes(self.ctx, ctypes.byref(v)))
        return int(v.value)

    def check(self, plan: dict) -> None:
        doc = json.dumps(plan_json(plan)).encode("utf-8")
        _check(lib().kh_plan_check(self.ctx, doc, len(doc)))

    def runner(self, plan: dict) -> HipPlanRunner:
        return HipPlanRunner(self, plan)

    def fit_batch(self, build, batch: int):
        """One packed plan holds any batch that fits the device: the largest asked size."""
        return build(batch)

    def prepare(self, work):
        return work()

    def call(self, start, read):
        return read(start())

    def info(self) -> dict:
        return {"backend": "hip", "device": self.device, "weightBytes": self.weight_bytes}

    def dispose(self) -> None:
        if self.ctx:
            _check(lib().kh_ctx_destroy(self.ctx))
            self.ctx = None

    def __del__(self):
        try:
            self.dispose()
        except Exception:
            pass
