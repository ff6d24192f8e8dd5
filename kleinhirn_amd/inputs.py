"""RunInput packing for a batch plan: the caller side of the Backend seam.

A Python statement of what the reference's EncoderModel hands a PlanRunner (src/encoder.ts:271-314):
word rows gathered on the host at row b * L + i (rows past a sequence's end stay zero), a prefix
mask of ones, type ids as u32 per row with the RoBERTa/XLM-R position row (pad id + running count
of non-pad ids) in the high 16 bits.
"""
from __future__ import annotations

import numpy as np

from .plan.spec import position_rows


def mask_and_types(spec: dict, ids: list[np.ndarray], length: int,
                   type_ids: list[np.ndarray] | None = None) -> tuple[np.ndarray, np.ndarray]:
    """src/encoder.ts:284-314."""
    B = len(ids)
    mask = np.zeros(length * B, dtype=np.float32)
    tt = np.zeros(length * B, dtype=np.uint32)
    emb = spec["embed"]
    for b, seq in enumerate(ids):
        n = len(seq)
        if n > length:
            raise ValueError(f"sequence {b} of {n} tokens exceeds the bucket {length}")
        mask[b * length:b * length + n] = 1
        if type_ids is not None and emb["typeVocab"] > 0:
            t = np.asarray(type_ids[b], dtype=np.int64)
            if np.any(t < 0) or np.any(t >= emb["typeVocab"]):
                raise ValueError(f"token type outside the {emb['typeVocab']} type rows")
            tt[b * length:b * length + n] = t
        pad = emb.get("padId")
        if pad is not None:
            rows = position_rows(pad, [int(x) for x in seq])
            p = np.full(length, pad, dtype=np.int64)
            p[:n] = rows
            if np.any(p >= emb["maxPositions"]) or np.any(p > 0xFFFF):
                raise ValueError("position row outside the position table")
            tt[b * length:(b + 1) * length] |= (p.astype(np.uint32) << 16)
    return mask, tt


def word_rows(table: np.ndarray, ids: list[np.ndarray], length: int) -> np.ndarray:
    """Host-side gather of one E-wide word row per token at row b * L + i (src/encoder.ts:271-282)."""
    E = table.shape[1]
    out = np.zeros((length * len(ids), E), dtype=table.dtype)
    for b, seq in enumerate(ids):
        out[b * length:b * length + len(seq)] = table[np.asarray(seq, dtype=np.int64)]
    return out


def run_input(spec: dict, word_table: np.ndarray, ids: list[np.ndarray], length: int) -> dict:
    mask, tt = mask_and_types(spec, ids, length)
    return {"embeddings": word_rows(word_table, ids, length), "mask": mask, "typeIds": tt}
