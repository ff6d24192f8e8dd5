"""CPU checks of the host side: the synthetic-input generator against the realized statistics the
benchmark protocol fixes, the plan builder against the reference's plan contracts, and the C ABI
library (exports, plan lowering and its error paths) without a GPU."""
from __future__ import annotations

import json
import math
import os
import re

import numpy as np
import pytest

from kleinhirn_amd import configs, inputs, synth
from kleinhirn_amd.plan import spec as S
from kleinhirn_amd.plan.build import all_ops, build_plan, plan_json, rel_bucket_index, rope_table

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

# ---- generator -------------------------------------------------------------------------------


def test_fnv1a32_known_answers():
    assert synth.fnv1a32("") == 0x811C9DC5
    assert synth.fnv1a32("a") == 0xE40C292C
    assert synth.fnv1a32("foobar") == 0xBF9CF968


def test_vectorised_lcg_equals_scalar_stream():
    for seed in (0, 1, 20261201, 0xFFFFFFFF):
        st = synth.Lcg(seed)
        want = [st.next() for _ in range(1000)]
        assert np.array_equal(synth.uniforms(seed, 1000), np.array(want))
    st = synth.Lcg(5)
    want = [st.normal() for _ in range(100)]
    assert np.allclose(synth.normals(5, 100), want, rtol=0, atol=1e-12)


# realized statistics of the seeded batches (seed 20261201): tokens, sum of n^2, extremes, first lengths
STATS = {
    "c2": dict(T=12801, sq=834755, mx=158, mn=11, first=[27, 33, 74, 68, 42, 33, 47, 55]),
    "c3b": dict(T=13205, sq=894405, mx=186, long=7),
    "c4": dict(T=261292, sq=1337173134, mx=8180, mn=949),
    "c5": dict(T=1213121, sq=418728231, mx=512),
}


@pytest.mark.parametrize("name", list(STATS))
def test_ragged_batches_reproduce_the_fixed_statistics(name):
    w = configs.ALL[name]()
    n = np.array(w.lengths, dtype=np.int64)
    s = STATS[name]
    assert n.sum() == s["T"] and (n * n).sum() == s["sq"] and n.max() == s["mx"]
    if "mn" in s:
        assert n.min() == s["mn"]
    if "first" in s:
        assert list(n[:8]) == s["first"]
    if "long" in s:
        assert int((n > 129).sum()) == s["long"]
    if name == "c2":
        assert sorted(n)[len(n) // 2] == 43  # upper median


def test_c5_pairs_are_clamped_to_the_position_table():
    w = configs.c5()
    assert max(w.lengths) <= 512
    assert sum(1 for q, p in w.pairs if q + p + 4 == 512) >= 5
    ids = w.ids()[:3]
    for (q, p), seq in zip(w.pairs[:3], ids):
        assert seq[0] == 0 and seq[q + 1] == 2 and seq[q + 2] == 2 and seq[-1] == 2 and len(seq) == q + p + 4


def test_weights_f16_cast_is_round_to_nearest_even():
    x = np.array([1.0 + 2 ** -11, 1.0 + 3 * 2 ** -11, 65504.0, 2 ** -24], dtype=np.float32)
    h = synth.to_f16(x).astype(np.float32)
    assert list(h) == [1.0, 1.0 + 2 ** -9, 65504.0, 2 ** -24]
    w = synth.tensor_values("layers.0.qkv.weight", (64, 64))
    assert w.dtype == np.float32 and abs(float(w.std()) - 0.02) < 0.002


def test_position_rows_and_type_packing():
    assert S.position_rows(1, [0, 5, 1, 7]) == [2, 3, 1, 4]
    spec = configs.roberta_base_spec()
    mask, tt = inputs.mask_and_types(spec, [np.array([0, 9, 9, 2])], 6)
    assert list(mask) == [1, 1, 1, 1, 0, 0]
    assert list(tt >> 16) == [2, 3, 4, 5, 1, 1]


# ---- plan builder ----------------------------------------------------------------------------


def kernels(plan):
    return [op["kernel"] for op in all_ops(plan)]


def test_post_norm_layer_ops_and_attention_forms():
    spec = configs.roberta_base_spec()
    head = S.roberta_classify_head(768, 3)
    small = build_plan(spec, head, 128, 1, True)     # split attention (scores fit one binding)
    big = build_plan(spec, head, 512, 64, True)      # flash kernel
    layer = [o["kernel"] for o in small["segments"][1]["ops"]]
    assert layer == ["mmtile", "attscore", "attsoftmax", "attpv", "mmtile", "layernorm", "mmtile", "mmtile", "layernorm"]
    assert [o["kernel"] for o in big["segments"][1]["ops"]][1] == "mbflash"
    assert kernels(small)[0] == "embln" and small["segments"][-1]["ops"][0]["kernel"] == "gather"
    assert small["output"]["rows"] == 1 and small["output"]["cols"] == 3
    ln = small["segments"][1]["ops"][5]
    assert ln["constants"]["MODE"] == 2 and ln["bind"][:2] == ["x", "attnOut"]


def test_modernbert_layers_tables_and_windows():
    spec = configs.modernbert_small_spec()
    plan = build_plan(spec, S.embed_head("cls", normalize=False), 128, 1, True)
    ids = [b["id"] for b in plan["buffers"]]
    assert "cossinG" in ids and "cossinL" in ids and "cossin" not in ids
    for l in range(spec["layers"]):
        seg = next(s for s in plan["segments"] if s["name"] == f"layer{l}")
        names = [o["name"] for o in seg["ops"]]
        assert ("lnA" in names) == (l != 0)  # layer 0 has no attn_norm
        rope = next(o for o in seg["ops"] if o["kernel"] == "rope")
        assert rope["bind"][1] == ("cossinG" if l % 3 == 0 else "cossinL")
        attn = next(o for o in seg["ops"] if "WINDOW" in o["constants"])
        assert attn["constants"]["WINDOW"] == (0 if l % 3 == 0 else 64)
    table = lambda n: next(b for b in plan["buffers"] if b["id"] == n)["init"]
    assert np.array_equal(table("cossinG"), rope_table(128, 160000, 64))
    t = rope_table(4, 10000, 8).reshape(4, 16)
    assert t[1, 0] == np.float32(math.cos(1.0)) and t[2, 8 + 1] == np.float32(math.sin(2 * 10000 ** -0.25))
    assert np.all(t[:, 4:8] == 0) and np.all(t[:, 12:] == 0)


def test_deberta_plan_relative_constants():
    spec = configs.deberta_v3_base_spec()
    plan = build_plan(spec, S.deberta_classify_head(768, 2), 128, 1, False)
    assert kernels(plan)[0] == "layernorm" and all_ops(plan)[0]["constants"]["MODE"] == 1
    rel = [o for o in all_ops(plan) if o["kernel"] == "attrel"]
    assert rel[0]["constants"]["MOFF"] == rel_bucket_index(0, 127, 256, 512)
    score = next(o for o in all_ops(plan) if o["kernel"] == "attscore")
    assert abs(score["constants"]["SCALE"] - 1 / math.sqrt(3 * 64)) < 1e-12
    fused = build_plan(spec, S.deberta_classify_head(768, 2), 512, 32, False)
    assert "attention" in kernels(fused)


def test_validate_segments_rejects_double_bound_writable_buffer():
    from kleinhirn_amd.plan.build import validate_segments
    seg = [{"name": "s", "prefix": "", "ops": [{"name": "bad", "kernel": "layernorm", "bind": ["x", "b", "w:w", "zero", "mask", "x"]}]}]
    with pytest.raises(ValueError, match="bound twice"):
        validate_segments(seg, {"x", "b", "zero", "mask"})


# ---- C ABI (no GPU: library load, exports, structural plan check) ------------------------------


def header_symbols():
    text = open(os.path.join(ROOT, "include", "kh_hip.h")).read()
    return sorted(set(re.findall(r"\b(kh_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    from kleinhirn_amd.backend import EXPORTS, lib
    L = lib()
    declared = header_symbols()
    assert declared, "no declarations found"
    for name in declared:
        assert hasattr(L, name), f"{name} declared in include/kh_hip.h but not exported"
    assert sorted(EXPORTS) == declared
    assert L.kh_abi_version() == 1


def _check(plan):
    import ctypes
    from kleinhirn_amd.backend import lib
    doc = json.dumps(plan_json(plan)).encode()
    rc = lib().kh_plan_check(None, doc, len(doc))
    return rc, lib().kh_last_error().decode()


@pytest.mark.parametrize("name", ["c1", "c2", "c3a", "c3b", "c4", "c5"])
def test_every_benchmark_plan_lowers(name):
    w = configs.ALL[name]() if name != "c5" else configs.c5(8)
    for B in (1, 8):
        for f16 in (False, True):
            rc, msg = _check(build_plan(w.spec, w.head, w.length, B, f16))
            assert rc == 0, msg


def test_plan_check_names_unsupported_ops_and_bad_json():
    from kleinhirn_amd.backend import lib
    plan = build_plan(configs.roberta_base_spec(), S.roberta_classify_head(768, 3), 64, 1, True)
    plan["segments"][1]["ops"].append({"name": "conv", "kernel": "im2col", "constants": {"N": 768, "KS": 3, "L": 64},
                                       "bind": ["qkv", "mask", "x"], "dispatch": [1, 1]})
    rc, msg = _check(plan)
    assert rc == 2 and "conv" in msg and "im2col" in msg
    bad = b'{"segments": [}'
    assert lib().kh_plan_check(None, bad, len(bad)) == 1
    assert "plan JSON" in lib().kh_last_error().decode()


def test_no_device_fails_loudly_without_fallback():
    """On a host without a GPU the context cannot be created: the library reports a HIP error, it
    never computes on the CPU."""
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    from kleinhirn_amd.backend import HipBackend, KhError
    with pytest.raises(KhError):
        HipBackend({})


def test_scheduler_type_words_equal_the_per_sequence_packing():
    """The scheduler's per-token type words (vectorised position rows) equal mask_and_types'
    words of the same sequences (src/encoder.ts:284-314)."""
    from kleinhirn_amd import configs, inputs
    from kleinhirn_amd.scheduler import type_words
    for name in ("c2", "c3b"):
        w = configs.ALL[name]()
        ids = w.ids()[:9]
        ids[3] = np.array([w.spec["embed"].get("padId") or 0] * 3 + list(ids[3][:5]), dtype=np.int32)
        L = max(len(x) for x in ids)
        _, tt = inputs.mask_and_types(w.spec, ids, L)
        want = np.concatenate([tt[b * L:b * L + len(x)] for b, x in enumerate(ids)])
        assert np.array_equal(type_words(w.spec, ids), want)
