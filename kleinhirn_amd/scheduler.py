"""Packed batch scheduling on one HIP backend (kh_sched_* of include/kh_hip.h).

The reference's runIdsBatch cuts a call into chunks of at most 16 sequences on plans of 1, 4, 8 or
16 (src/encoder.ts:380-436, src/cache.ts:9-18); here a few large packed plans take every chunk: the
library sorts the sequences by length, fills each plan up to its batch (or a token budget) and runs
plans of one shape in turn so host packing overlaps the device. Rows are gathered on the device
from the context's word table (HipBackend.set_words or HipBackend.from_manifest).
"""
from __future__ import annotations

import ctypes

import numpy as np

from .backend import HipBackend, SchedStats, _check, lib
from .plan.build import build_plan


def type_words(spec: dict, ids: list[np.ndarray], type_ids: list[np.ndarray] | None = None) -> np.ndarray:
    """The u32 word per token that kh_upload takes (type in the low 16 bits; for models with a
    padding id the position row, pad id + running count of non-pad ids, in the high 16 bits;
    src/encoder.ts:284-314), concatenated in sequence order."""
    emb = spec["embed"]
    pad = emb.get("padId")
    lens = np.array([len(x) for x in ids], dtype=np.int64)
    flat = np.concatenate([np.asarray(x, np.int64) for x in ids]) if len(ids) else np.zeros(0, np.int64)
    t = np.zeros(flat.size, dtype=np.uint32)
    if type_ids is not None and emb["typeVocab"] > 0:
        t[:] = np.concatenate([np.asarray(x, np.uint32) for x in type_ids])
    if pad is not None and flat.size:
        # position_rows per sequence: a running count of non-pad ids restarted at each sequence
        keep = (flat != pad).astype(np.int64)
        run = np.cumsum(keep)
        starts = np.concatenate([[0], np.cumsum(lens)[:-1]])
        before = np.repeat(run[starts] - keep[starts], lens)
        rows = np.where(keep == 1, pad + run - before, pad)
        if np.any(rows >= emb["maxPositions"]) or np.any(rows > 0xFFFF):
            raise ValueError("position row outside the position table")
        t |= rows.astype(np.uint32) << 16
    return t


class BatchScheduler:
    """`copies` plans of batch `batch` per length in `lengths`, scheduled by the library."""

    def __init__(self, backend: HipBackend, spec: dict, head: dict, f16: bool, lengths=(512,), batch: int = 256,
                 copies: int = 2):
        self.spec = spec
        self.runners = [backend.runner(build_plan(spec, head, L, batch, f16)) for L in lengths for _ in range(copies)]
        handles = (ctypes.c_void_p * len(self.runners))(*[r.h.value for r in self.runners])
        h = ctypes.c_void_p()
        _check(lib().kh_sched_create(handles, len(self.runners), ctypes.byref(h)))
        self.h = h
        self.cols = self.runners[0].plan["output"]["cols"]

    def run(self, ids: list[np.ndarray], type_ids: list[np.ndarray] | None = None,
            token_budget: int = 0) -> tuple[np.ndarray, dict]:
        """Outputs [len(ids), cols] in input order, and the run's statistics."""
        flat = np.ascontiguousarray(np.concatenate([np.asarray(x, np.int32) for x in ids]) if ids else
                                    np.zeros(1, np.int32), dtype=np.int32)
        offsets = np.zeros(len(ids) + 1, dtype=np.int64)
        offsets[1:] = np.cumsum([len(x) for x in ids])
        tw = type_words(self.spec, ids, type_ids) if ids else None
        out = np.empty((len(ids), self.cols), dtype=np.float32)
        st = SchedStats()
        _check(lib().kh_sched_run(self.h, flat.ctypes.data, offsets.ctypes.data, len(ids),
                                  tw.ctypes.data if tw is not None and tw.size else None, int(token_budget),
                                  out.ctypes.data if out.size else None, out.size, ctypes.byref(st)))
        return out, st.as_dict()

    def destroy(self) -> None:
        if getattr(self, "h", None):
            _check(lib().kh_sched_destroy(self.h))
            self.h = None
        for r in self.runners:
            r.destroy()
        self.runners = []

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass
