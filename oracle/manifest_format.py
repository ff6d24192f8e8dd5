"""TEST INFRASTRUCTURE — the manifest directory format restated on the CPU, to check the native
loader (kh_manifest_check / kh_load_manifest) against.

Only tests/ import this module; the product path never does.

* `row_checksum`: the words.bin row checksum, murmur3_32 over the row's little-endian u32 words
  seeded with salt ^ (row_id + 1) * 0x9e3779b1 (src/words-format.ts:18-32). Pinned by the
  reference's own vectors (tests/r4_words.test.ts:22-29 of the reference) in
  tests/test_manifest.py.
* `encode_words`: the table rows with a checksum after each; the salt is the first u32
  (little-endian) of the table's sha256 (src/words-encode.ts:8-26).
* `place_tensors`: tensors at 256-byte offsets, a shard closes before a tensor would pass the
  shard limit (src/convert/manifest.ts:220-245; SHARD_LIMIT, ALIGN at :14-15).
* `write_manifest`: a version-3 directory (manifest.json, shard-<i>.bin, words.bin) as
  buildManifest writes it (src/convert/manifest.ts:258-294), or a version-2 ("legacy") directory
  whose word table sits in the shards as keepOnCpu parts of at most `chunk_rows` rows
  (EMBED_CHUNK_ROWS, src/convert/manifest.ts:16; layout of tests/r4_words.test.ts:100-131).
SHA-256 itself is hashlib's.
"""
from __future__ import annotations

import hashlib
import json
import os
import struct

import numpy as np

SHARD_LIMIT = 95_000_000
ALIGN = 256
EMBED_CHUNK_ROWS = 60_000
FORMAT = "kleinhirn-weights-2"
WORDS = "embeddings.word.weight"

M32 = 0xFFFFFFFF


def _rotl(x: int, r: int) -> int:
    return ((x << r) | (x >> (32 - r))) & M32


def row_checksum(row: bytes, row_id: int, salt: int) -> int:
    if len(row) % 4:
        raise ValueError(f"words: row of {len(row)} bytes is not whole u32 words")
    h = (salt ^ ((row_id + 1) * 0x9E3779B1)) & M32
    for (k,) in struct.iter_unpack("<I", row):
        k = (k * 0xCC9E2D51) & M32
        k = _rotl(k, 15)
        k = (k * 0x1B873593) & M32
        h ^= k
        h = _rotl(h, 13)
        h = (h * 5 + 0xE6546B64) & M32
    h ^= len(row)
    h ^= h >> 16
    h = (h * 0x85EBCA6B) & M32
    h ^= h >> 13
    h = (h * 0xC2B2AE35) & M32
    h ^= h >> 16
    return h


def row_checksums(rows_u32: np.ndarray, salt: int) -> np.ndarray:
    """`row_checksum` of every row of a [rows, words] u32 array at once (row id = index)."""
    n, w = rows_u32.shape
    ids = np.arange(n, dtype=np.uint64)
    h = (np.uint64(salt) ^ (((ids + 1) * np.uint64(0x9E3779B1)) & np.uint64(M32))).astype(np.uint64)
    m = np.uint64(M32)

    def rotl(x, r):
        return ((x << np.uint64(r)) | (x >> np.uint64(32 - r))) & m

    for j in range(w):
        k = rows_u32[:, j].astype(np.uint64)
        k = (k * np.uint64(0xCC9E2D51)) & m
        k = rotl(k, 15)
        k = (k * np.uint64(0x1B873593)) & m
        h ^= k
        h = rotl(h, 13)
        h = (h * np.uint64(5) + np.uint64(0xE6546B64)) & m
    h ^= np.uint64(4 * w)
    h ^= h >> np.uint64(16)
    h = (h * np.uint64(0x85EBCA6B)) & m
    h ^= h >> np.uint64(13)
    h = (h * np.uint64(0xC2B2AE35)) & m
    h ^= h >> np.uint64(16)
    return h.astype(np.uint32)


def encode_words(table: bytes, rows: int, width: int, dtype: str) -> tuple[bytes, int]:
    data = width * (2 if dtype == "f16" else 4)
    if len(table) != rows * data:
        raise ValueError(f"words: table is {len(table)} bytes, expected {rows} x {data}")
    salt = struct.unpack("<I", hashlib.sha256(table).digest()[:4])[0]
    t = np.frombuffer(table, dtype="<u4").reshape(rows, data // 4)
    out = np.empty((rows, data // 4 + 1), dtype="<u4")
    out[:, :-1] = t
    out[:, -1] = row_checksums(t, salt)
    return out.tobytes(), salt


def place_tensors(sizes: list[int], limit: int = SHARD_LIMIT) -> tuple[list[tuple[int, int]], list[int]]:
    at, lengths, length = [], [], 0

    def pad(n):
        return n + (-n) % ALIGN

    for size in sizes:
        length = pad(length)
        if length + size > limit:
            if length:
                lengths.append(length)
            length = 0
        at.append((len(lengths), length))
        length += size
    if length:
        lengths.append(length)
    return at, lengths


def _cast(name: str, a: np.ndarray, dtype: str) -> bytes:
    a = np.ascontiguousarray(a, dtype=np.float16 if dtype == "f16" else np.float32)
    if not np.all(np.isfinite(a)):
        raise ValueError(f"{name}: not finite in {dtype}")
    return a.tobytes()


def write_manifest(directory: str, weights: dict[str, np.ndarray], dtype: str, version: int = 3,
                   limit: int = SHARD_LIMIT, chunk_rows: int = EMBED_CHUNK_ROWS, extra: dict | None = None) -> str:
    """Writes the directory; returns the path of manifest.json."""
    os.makedirs(directory, exist_ok=True)
    table = weights[WORDS]
    rows, width = table.shape
    items = []  # (entry, bytes)
    if version == 2:
        for r0 in range(0, rows, chunk_rows):
            part = table[r0:r0 + chunk_rows]
            items.append(({"name": WORDS, "dtype": dtype, "shape": list(part.shape), "keepOnCpu": True,
                           "rowStart": r0, "rowEnd": r0 + part.shape[0]}, _cast(WORDS, part, dtype)))
    for name, a in weights.items():
        if name != WORDS:
            items.append(({"name": name, "dtype": dtype, "shape": list(a.shape)}, _cast(name, a, dtype)))
    at, lengths = place_tensors([len(b) for _, b in items], limit)
    shards = [bytearray(n) for n in lengths]
    tensors = []
    for (entry, b), (shard, offset) in zip(items, at):
        shards[shard][offset:offset + len(b)] = b
        tensors.append({**entry, "shard": shard, "offset": offset, "byteLength": len(b)})
    shard_meta = []
    for i, sb in enumerate(shards):
        fname = f"shard-{i}.bin"
        with open(os.path.join(directory, fname), "wb") as f:
            f.write(sb)
        shard_meta.append({"file": fname, "bytes": len(sb), "sha256": hashlib.sha256(sb).hexdigest()})
    manifest = {"format": FORMAT, "version": version, "source": {}, "encoder": {}, "head": {},
                "tensors": tensors, "shards": shard_meta, **(extra or {})}
    if version == 3:
        wb, salt = encode_words(_cast(WORDS, table, dtype), rows, width, dtype)
        with open(os.path.join(directory, "words.bin"), "wb") as f:
            f.write(wb)
        manifest["words"] = {"file": "words.bin", "bytes": len(wb), "sha256": hashlib.sha256(wb).hexdigest(),
                             "dtype": dtype, "rows": rows, "width": width,
                             "rowBytes": width * (2 if dtype == "f16" else 4) + 4, "salt": salt}
    path = os.path.join(directory, "manifest.json")
    with open(path, "w") as f:
        json.dump(manifest, f, indent=1)
    return path
