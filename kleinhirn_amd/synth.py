"""Seeded synthetic weights and ragged inputs for the encoder benchmark configurations.

One PRNG for every consumer (the HIP runner, the CPU oracle, the benchmark): the linear
congruential generator of the reference's own op tests (tests/wasm_plan.test.ts:13-18),
``s = (s * 1103515245 + 12345) mod 2**32`` with ``u = s / 2**32`` in [0, 1). Normals come from
Box-Muller on two uniforms, cos branch only: ``z = sqrt(-2 ln(1 - u1)) cos(2 pi u2)``.

Each weight tensor has its own stream seeded with ``seed XOR fnv1a32(name)`` so tensors do not
depend on generation order. Values are N(0, 0.02) drawn in f64 and rounded once to f32; an f16
model casts that f32 value with round-to-nearest-even, as the reference converter's
``Float16Array`` cast does (src/convert/manifest.ts:197-206). LayerNorm gamma = 1, beta = 0.

The vectorised generator below computes the LCG in closed form (a jump-ahead affine map per
index), so a 250k x 384 word table takes well under a second in numpy.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

SEED = 20261201
LCG_A = 1103515245
LCG_C = 12345
MASK32 = 0xFFFFFFFF


def fnv1a32(text: str) -> int:
    """32-bit FNV-1a over the UTF-8 bytes (offset basis 2166136261, prime 16777619)."""
    h = 2166136261
    for byte in text.encode("utf-8"):
        h ^= byte
        h = (h * 16777619) & MASK32
    return h


class Lcg:
    """Scalar stream: next() returns u in [0, 1) after advancing the state."""

    def __init__(self, seed: int):
        self.s = seed & MASK32

    def next(self) -> float:
        self.s = (self.s * LCG_A + LCG_C) & MASK32
        return self.s / 4294967296.0

    def normal(self) -> float:
        u1 = self.next()
        u2 = self.next()
        return math.sqrt(-2.0 * math.log(1.0 - u1)) * math.cos(2.0 * math.pi * u2)

    def int_in(self, lo: int, hi: int) -> int:
        """lo + floor(u (hi - lo + 1)): uniform over [lo, hi]."""
        return lo + math.floor(self.next() * (hi - lo + 1))


def lcg_states(seed: int, count: int) -> np.ndarray:
    """The first `count` states after seed (state k = A^(k+1) seed + C (A^k + ... + 1)), uint64
    holding 32-bit values. Built by doubling: the states of the second half are the affine map
    of the first half's states."""
    out = np.empty(count, dtype=np.uint64)
    if count == 0:
        return out
    out[0] = (seed * LCG_A + LCG_C) & MASK32
    n = 1
    # affine map f^n: s -> a_n s + c_n (mod 2^32)
    a_n, c_n = LCG_A, LCG_C
    while n < count:
        take = min(n, count - n)
        out[n:n + take] = (out[:take] * np.uint64(a_n) + np.uint64(c_n)) & np.uint64(MASK32)
        # f^(2n) = f^n o f^n
        c_n = (a_n * c_n + c_n) & MASK32
        a_n = (a_n * a_n) & MASK32
        n += take
    return out


def uniforms(seed: int, count: int) -> np.ndarray:
    return lcg_states(seed, count).astype(np.float64) / 4294967296.0


def normals(seed: int, count: int) -> np.ndarray:
    """`count` Box-Muller normals (two uniforms each, cos branch only), f64."""
    u = uniforms(seed, 2 * count)
    u1 = u[0::2]
    u2 = u[1::2]
    return np.sqrt(-2.0 * np.log(1.0 - u1)) * np.cos(2.0 * np.pi * u2)


def tensor_values(name: str, shape, std: float = 0.02, seed: int = SEED) -> np.ndarray:
    """N(0, std) in f32 from the tensor's own stream (seed XOR fnv1a32(name))."""
    n = int(np.prod(shape)) if len(shape) else 1
    z = normals((seed ^ fnv1a32(name)) & MASK32, n)
    return (std * z).astype(np.float32).reshape(shape)


def to_f16(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even binary16 (numpy's cast is IEEE RNE)."""
    return np.asarray(x, dtype=np.float32).astype(np.float16)


# ---------------------------------------------------------------------------------------------
# Ragged batches (lengths count the special tokens)


def lognormal_lengths(stream: Lcg, batch: int, median: float = 45.0, sigma: float = 0.5,
                      lo: int = 8, hi: int = 512) -> list[int]:
    """n = clamp(round(exp(ln median + sigma z)), lo, hi) with round(x) = floor(x + 0.5)."""
    out = []
    for _ in range(batch):
        z = stream.normal()
        n = math.floor(math.exp(math.log(median) + sigma * z) + 0.5)
        out.append(min(max(n, lo), hi))
    return out


@dataclass
class Batch:
    """Token ids per sequence (special tokens included) and the type ids (all 0)."""
    ids: list[np.ndarray]
    lengths: list[int] = field(default_factory=list)

    def __post_init__(self):
        self.lengths = [len(x) for x in self.ids]

    @property
    def tokens(self) -> int:
        return int(sum(self.lengths))


def draw_ids(stream_seed: int, lengths, vocab: int, cls_id: int, sep_id: int,
             pairs: list[tuple[int, int]] | None = None) -> list[np.ndarray]:
    """Body ids uniform over [1000, vocab - 1] (1000 + floor(u (vocab - 1000))), from a stream of
    its own (seed `stream_seed`), wrapped in the family's special tokens. `pairs` packs
    `cls q sep sep p sep` (the XLM-R cross-encoder template) instead of `cls body sep`."""
    total = int(sum(lengths))
    u = uniforms(stream_seed & MASK32, total)
    body = (1000 + np.floor(u * (vocab - 1000))).astype(np.int64)
    out = []
    at = 0
    for b, n in enumerate(lengths):
        seq = body[at:at + n].copy()
        at += n
        seq[0] = cls_id
        seq[-1] = sep_id
        if pairs is not None:
            q, _p = pairs[b]
            seq[q + 1] = sep_id
            seq[q + 2] = sep_id
        out.append(seq)
    return out
