"""Manifest directories on the CPU: the native reader (kh_manifest_check, kh_sha256,
kh_row_checksum of libkh_hip.so) against the format's restatement in oracle/manifest_format.py,
which is pinned by the reference's own checksum vectors (tests/r4_words.test.ts:22-29 of the
reference) and by hashlib. Directories are written by the restated converter
(src/convert/manifest.ts:220-294) into tmp_path; errors carry the reference's messages
(src/weights.ts:161-165, src/words.ts:98-113, src/weights.ts:79-83)."""
from __future__ import annotations

import hashlib
import json
import os
import subprocess
import sys

import numpy as np
import pytest

from kleinhirn_amd import backend as B
from oracle import manifest_format as MF

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
RNG = np.random.default_rng(7)


def test_oracle_row_checksum_matches_the_reference_vectors():
    a = bytes([1, 2, 3, 4, 5, 6, 7, 8])
    assert MF.row_checksum(a, 0, 0x12345678) == 1313458805
    assert MF.row_checksum(a, 5, 0x12345678) == 2842431045
    assert MF.row_checksum(bytes(16), 0, 0) == 3286763420
    assert MF.row_checksum(bytes([1, 2, 3, 4, 5, 6, 7, 9]), 0, 0x12345678) == 1982651642
    assert MF.row_checksum(a, 0, 0x12345679) == 1216509786
    with pytest.raises(ValueError, match="whole u32"):
        MF.row_checksum(bytes(6), 0, 0)


def test_vectorised_row_checksums_equal_the_scalar_form():
    rows = RNG.integers(0, 2**32, size=(37, 9), dtype=np.uint64).astype(np.uint32)
    salt = 0xDEADBEEF
    got = MF.row_checksums(rows, salt)
    for i in range(rows.shape[0]):
        assert got[i] == MF.row_checksum(rows[i].astype("<u4").tobytes(), i, salt)


def test_library_row_checksum_matches_the_reference_vectors_and_the_oracle():
    a = bytes([1, 2, 3, 4, 5, 6, 7, 8])
    assert B.row_checksum(a, 0, 0x12345678) == 1313458805
    assert B.row_checksum(a, 5, 0x12345678) == 2842431045
    assert B.row_checksum(bytes(16), 0, 0) == 3286763420
    assert B.row_checksum(bytes([1, 2, 3, 4, 5, 6, 7, 9]), 0, 0x12345678) == 1982651642
    assert B.row_checksum(a, 0, 0x12345679) == 1216509786
    for n in (0, 4, 12, 1536, 772):
        row = RNG.integers(0, 256, size=n, dtype=np.uint8).tobytes()
        rid, salt = int(RNG.integers(0, 2**31)), int(RNG.integers(0, 2**32))
        assert B.row_checksum(row, rid, salt) == MF.row_checksum(row, rid, salt)
    with pytest.raises(B.KhError, match="whole u32"):
        B.row_checksum(bytes(6), 0, 0)


SHA_LENGTHS = [0, 1, 3, 55, 56, 57, 63, 64, 65, 119, 120, 127, 128, 1000, (1 << 20) + 7]


def test_library_sha256_equals_hashlib():
    assert B.sha256(b"abc") == "ba7816bf8f01cfea414140de5dae2223b00361a396177a9cb410ff61f20015ad"
    for n in SHA_LENGTHS:
        data = RNG.integers(0, 256, size=n, dtype=np.uint8).tobytes()
        assert B.sha256(data) == hashlib.sha256(data).hexdigest(), n


def test_portable_sha256_equals_hashlib():
    """The path without the CPU's SHA extensions (forced with KH_SHA256_PORTABLE in a fresh
    process, since the choice is made once per process)."""
    code = (
        "import hashlib, numpy as np\n"
        "from kleinhirn_amd import backend as B\n"
        "rng = np.random.default_rng(3)\n"
        f"for n in {SHA_LENGTHS!r}:\n"
        "    d = rng.integers(0, 256, size=n, dtype=np.uint8).tobytes()\n"
        "    assert B.sha256(d) == hashlib.sha256(d).hexdigest(), n\n"
        "print('ok')\n")
    env = dict(os.environ, KH_SHA256_PORTABLE="1")
    out = subprocess.run([sys.executable, "-c", code], cwd=ROOT, env=env, capture_output=True, text=True, timeout=300)
    assert out.returncode == 0 and "ok" in out.stdout, out.stderr


def small_weights(rows=10, width=8):
    return {
        MF.WORDS: RNG.standard_normal((rows, width)).astype(np.float32),
        "a": RNG.standard_normal(3).astype(np.float32),
        "b": RNG.standard_normal((2, 2)).astype(np.float32),
        "layer.w": RNG.standard_normal((16, 8)).astype(np.float32),
    }


@pytest.mark.parametrize("dtype", ["f16", "f32"])
def test_version3_directory_reads_with_every_check(tmp_path, dtype):
    w = small_weights()
    path = MF.write_manifest(str(tmp_path), w, dtype)
    info = B.manifest_check(path, B.LOAD_CHECK_ROWS)
    es = 2 if dtype == "f16" else 4
    assert info["version"] == 3
    assert info["tensors"] == 3 and info["shards"] == 1
    assert info["tensor_bytes"] == es * (3 + 4 + 128)
    assert (info["words_rows"], info["words_width"]) == (10, 8)
    assert info["words_dtype"] == (B.KH_F16 if dtype == "f16" else B.KH_F32)
    m = json.load(open(path))
    assert info["file_bytes"] == m["shards"][0]["bytes"] + m["words"]["bytes"]
    # the restated converter's words.bin rows carry the checksum the reader checks
    wb = open(os.path.join(str(tmp_path), "words.bin"), "rb").read()
    rb = m["words"]["rowBytes"]
    for i in range(10):
        row = wb[i * rb:(i + 1) * rb]
        assert int.from_bytes(row[-4:], "little") == B.row_checksum(row[:-4], i, m["words"]["salt"])


def test_shards_split_at_the_limit_on_256_byte_offsets(tmp_path):
    w = {MF.WORDS: np.zeros((4, 4), np.float32)}
    for i in range(6):
        w[f"t{i}"] = RNG.standard_normal(100 + 37 * i).astype(np.float32)
    at, lengths = MF.place_tensors([400 + 148 * i for i in range(6)], limit=1200)
    assert all(off % MF.ALIGN == 0 for _, off in at)
    # (the offset is padded before the limit test, so a closed shard may end in up to 255 pad bytes)
    assert len(lengths) > 1 and all(n < 1200 + MF.ALIGN for n in lengths)
    path = MF.write_manifest(str(tmp_path), w, "f32", limit=1200)
    info = B.manifest_check(path)
    assert info["shards"] == len(lengths) and info["tensors"] == 6


def test_legacy_directory_joins_the_keepOnCpu_parts_in_row_order(tmp_path):
    w = small_weights(rows=6, width=4)
    path = MF.write_manifest(str(tmp_path), w, "f16", version=2, chunk_rows=4)
    m = json.load(open(path))
    parts = [t for t in m["tensors"] if t.get("keepOnCpu")]
    assert [p["rowStart"] for p in parts] == [0, 4]
    # put the second part first in the list: the reader sorts by rowStart
    m["tensors"] = [parts[1]] + [t for t in m["tensors"] if t is not parts[1]]
    json.dump(m, open(path, "w"))
    info = B.manifest_check(path)
    assert info["version"] == 2
    assert (info["words_rows"], info["words_width"], info["words_dtype"]) == (6, 4, B.KH_F16)
    assert info["tensors"] == 3  # keepOnCpu parts stay off the device


def _rewrite(path, fn):
    m = json.load(open(path))
    fn(m)
    json.dump(m, open(path, "w"))


def _flip(file, at):
    b = bytearray(open(file, "rb").read())
    b[at] ^= 1
    open(file, "wb").write(b)


def test_damaged_shard_fails_its_sha256(tmp_path):
    path = MF.write_manifest(str(tmp_path), small_weights(), "f16")
    _flip(os.path.join(str(tmp_path), "shard-0.bin"), 300)
    with pytest.raises(B.KhError, match="sha256 mismatch on shard-0.bin"):
        B.manifest_check(path)
    B.manifest_check(path, B.LOAD_NO_SHA256)  # the caller may skip hashing


def test_words_bin_size_layout_and_rows(tmp_path):
    d = str(tmp_path)
    path = MF.write_manifest(d, small_weights(), "f16")
    wfile = os.path.join(d, "words.bin")
    good = open(wfile, "rb").read()
    open(wfile, "wb").write(good[:-4])
    with pytest.raises(B.KhError, match=r"words.bin is \d+ bytes, manifest says \d+"):
        B.manifest_check(path)
    open(wfile, "wb").write(good)
    # a damaged row whose file digest is updated: only the row checksums see it
    _flip(wfile, 3 * 20 + 5)
    _rewrite(path, lambda m: m["words"].update(sha256=hashlib.sha256(open(wfile, "rb").read()).hexdigest()))
    B.manifest_check(path)
    with pytest.raises(B.KhError, match="words.bin row 3 fails its checksum"):
        B.manifest_check(path, B.LOAD_CHECK_ROWS)
    _rewrite(path, lambda m: m["words"].update(rowBytes=18))
    with pytest.raises(B.KhError, match="words: rowBytes 18 is not 8 f16 values and a checksum"):
        B.manifest_check(path)
    _rewrite(path, lambda m: m["words"].update(rowBytes=20, sha256="0" * 64))
    with pytest.raises(B.KhError, match="sha256 mismatch on words.bin"):
        B.manifest_check(path)


def test_manifest_without_a_word_table_or_with_other_cpu_tensors(tmp_path):
    d = str(tmp_path)
    path = MF.write_manifest(d, small_weights(), "f32", version=2, chunk_rows=4)
    saved = json.load(open(path))
    _rewrite(path, lambda m: m.update(tensors=[t for t in m["tensors"] if not t.get("keepOnCpu")]))
    with pytest.raises(B.KhError, match="manifest has neither words.bin nor a keepOnCpu word table"):
        B.manifest_check(path)
    B.manifest_check(path, B.LOAD_NO_WORDS)
    json.dump(saved, open(path, "w"))
    _rewrite(path, lambda m: [t.update(keepOnCpu=True) for t in m["tensors"] if t["name"] == "a"])
    with pytest.raises(B.KhError, match="only the word table stays on the CPU"):
        B.manifest_check(path)


def test_tensor_layout_errors(tmp_path):
    d = str(tmp_path)
    path = MF.write_manifest(d, small_weights(), "f32")
    saved = json.load(open(path))
    _rewrite(path, lambda m: m["tensors"][-1].update(offset=m["shards"][0]["bytes"] - 8))
    with pytest.raises(B.KhError, match="runs past the end of shard-0.bin"):
        B.manifest_check(path)
    json.dump(saved, open(path, "w"))
    _rewrite(path, lambda m: m["tensors"][0].update(shape=[4]))
    with pytest.raises(B.KhError, match="bytes for shape of 4 elements"):
        B.manifest_check(path)
    json.dump(saved, open(path, "w"))
    _rewrite(path, lambda m: m["tensors"][0].update(dtype="bf16"))
    with pytest.raises(B.KhError, match="dtype bf16"):
        B.manifest_check(path)
    json.dump(saved, open(path, "w"))
    os.remove(os.path.join(d, "shard-0.bin"))
    with pytest.raises(B.KhError, match="cannot open"):
        B.manifest_check(path)
    with pytest.raises(B.KhError, match="cannot open"):
        B.manifest_check(os.path.join(d, "missing.json"))
