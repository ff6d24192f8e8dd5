"""Weights and word table straight from a manifest directory (kh_load_manifest) give the same
outputs, bit for bit, as the same weights handed over tensor by tensor (kh_weight_add, the
loadWeights path of src/webgpu-backend.ts:53-101) and the host word gather. Directories are written
by the restated converter (oracle/manifest_format.py) from the c2 golden case's weights."""
from __future__ import annotations

import os
import tempfile

import numpy as np
import pytest

from kleinhirn_amd import backend as B
from kleinhirn_amd import configs, inputs
from kleinhirn_amd.plan.build import build_plan
from oracle import manifest_format as MF
from tests.helpers import decision_parity, hip_outputs
from tests.test_gpu_models import case_and_oracle

pytestmark = pytest.mark.gpu


def run_ids(be, case, f16=True):
    """One batch plan fed token ids: rows gathered from the context's device word table."""
    plan = build_plan(case.spec, case.head, case.length, len(case.ids), f16)
    r = be.runner(plan)
    mask, tt = inputs.mask_and_types(case.spec, case.ids, case.length)
    ids = np.zeros(case.length * len(case.ids), dtype=np.int32)
    for b, seq in enumerate(case.ids):
        ids[b * case.length:b * case.length + len(seq)] = seq
    r.upload_ids(ids, mask, tt)
    r.run(case.length * len(case.ids))
    out = r.read_output().reshape(len(case.ids), -1)
    r.destroy()
    return out


@pytest.mark.parametrize("version", [3, 2])
def test_manifest_load_equals_tensor_by_tensor_upload(version):
    case, ref = case_and_oracle("c2")
    want = hip_outputs(case, f16=True)
    with tempfile.TemporaryDirectory() as d:
        path = MF.write_manifest(d, case.weights, "f16", version=version, chunk_rows=20_000)
        be = B.HipBackend.from_manifest(path, flags=B.LOAD_CHECK_ROWS)
        info = be.load_info
        print(f"v{version}: {info['file_bytes'] / 1e6:.1f} MB read in {info['read_ms']:.1f} ms, "
              f"sha256 {info['sha256_ms']:.1f} ms, rows {info['rows_ms']:.1f} ms, upload {info['upload_ms']:.1f} ms")
    W = configs.storage(case.weights, True)
    assert (info["words_rows"], info["words_width"]) == W["embeddings.word.weight"].shape
    assert be.weight_bytes == sum(t.nbytes for n, t in W.items() if n != MF.WORDS)
    loaded = hip_outputs(case, f16=True, backend=be)                        # host gather
    d = decision_parity(ref, loaded)
    assert d["mismatched"] == 0 and d["delta"] <= 2e-2, d                   # the oracle's bars
    assert np.array_equal(loaded, want)
    assert np.array_equal(run_ids(be, case), want)                          # device table from the files
    be.dispose()


def test_failed_manifest_load_uploads_nothing():
    case, _ = case_and_oracle("c2")
    weights = {MF.WORDS: case.weights[MF.WORDS][:100], "a.weight": case.weights["head.dense.weight"]}
    with tempfile.TemporaryDirectory() as d:
        path = MF.write_manifest(d, weights, "f16")
        b = bytearray(open(os.path.join(d, "shard-0.bin"), "rb").read())
        b[10] ^= 1
        open(os.path.join(d, "shard-0.bin"), "wb").write(b)
        be = B.HipBackend({})
        with pytest.raises(B.KhError, match="sha256 mismatch on shard-0.bin"):
            B._check(B.lib().kh_load_manifest(be.ctx, os.fsencode(path), 0, None))
        assert be.weight_bytes == 0
        be.dispose()
