"""Model-level parity: whole plans of the five benchmark families through the C ABI against the
CPU oracle (f32 restatement of the reference's WASM executor) on the same seeded weights and ids.

Bars: f32 plans give identical argmax and logits within 1e-3 absolute,
embedding cosine >= 0.9999; f16 plans give embedding cosine >= 0.999 and identical decisions on
every decision f16 rounding cannot flip (top-2 gap >= 2 delta, convert/k28_close_calls.py:1-8).
Sequences are subsets of the benchmark batches so the oracle finishes in seconds."""
from __future__ import annotations

import os

import numpy as np
import pytest

from kleinhirn_amd import configs, inputs
from kleinhirn_amd.plan.build import build_plan
from tests.helpers import cosine_rows, decision_parity, hip_outputs, oracle_outputs, workload_case

pytestmark = pytest.mark.gpu

CASES = {
    # name: (workload, batch, layers, bucket length, max tokens)
    "c1": ("c1", 1, None, 128, None),
    "c2": ("c2", 12, None, 512, None),
    "c3a": ("c3a", 2, 4, 512, None),
    "c3b": ("c3b", 10, None, 512, None),
    "c4": ("c4", 3, 6, 1024, 700),
    "c5": ("c5", 6, None, 512, None),
}

_cache: dict = {}


GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def case_and_oracle(key):
    """The seeded case and the oracle's outputs for it: the committed golden vectors (made by
    tests/golden/make_golden.py from the same case), and for c2 also a live oracle run."""
    if key not in _cache:
        w, batch, layers, length, max_len = CASES[key]
        case = workload_case(w, batch, layers, length, max_len)
        g = np.load(os.path.join(GOLDEN, f"oracle_{key}.npz"))
        assert np.array_equal(np.concatenate(case.ids).astype(np.int32), g["ids"]), "golden ids differ from the case"
        ref = g["out"]
        if key == "c2":
            live = oracle_outputs(case)
            assert np.allclose(live, ref, rtol=0, atol=1e-6)
        _cache[key] = (case, ref)
    return _cache[key]


def check_f32(key, ref, got):
    if key in ("c1", "c4"):
        cos = cosine_rows(ref, got)
        assert cos.min() >= 0.9999, f"{key}: min cosine {cos.min()}"
        assert np.abs(ref - got).max() <= 1e-3
    else:
        assert np.abs(ref - got).max() <= 1e-3, f"{key}: max |dlogit| {np.abs(ref - got).max()}"
        if ref.shape[1] > 1:
            assert np.array_equal(ref.argmax(1), got.argmax(1)), f"{key}: argmax differs"


@pytest.mark.parametrize("key", list(CASES))
def test_f32_plan_matches_oracle(key):
    case, ref = case_and_oracle(key)
    got = hip_outputs(case, f16=False)
    print(f"{key} f32: max|d| {np.abs(ref - got).max():.3e}")
    check_f32(key, ref, got)


@pytest.mark.parametrize("key", [k for k in CASES if k != "c1"])
def test_f16_plan_matches_oracle(key):
    case, ref = case_and_oracle(key)
    got = hip_outputs(case, f16=True)
    if key == "c4":
        cos = cosine_rows(ref, got)
        print(f"{key} f16: min cosine {cos.min():.6f}")
        assert cos.min() >= 0.999
        return
    d = decision_parity(ref, got)
    print(f"{key} f16: {d}")
    assert d["mismatched"] == 0, d
    # the f32 reference logits of these random-weight heads are O(0.1-1); f16 storage keeps them
    # within a few 1e-3
    assert d["delta"] <= 2e-2, d


def test_batch_plan_equals_single_plans():
    """Packed batch result equals per-sequence B = 1 results (the reference checks batch vs single
    bit-identity for the WASM path, src/wasm/plan.ts:942-950)."""
    case, _ = case_and_oracle("c2")
    a = hip_outputs(case, f16=True, batch_plan=True)
    b = hip_outputs(case, f16=True, batch_plan=False)
    assert np.array_equal(a, b)


def test_device_word_gather_equals_host_gather():
    case, _ = case_and_oracle("c5")
    a = hip_outputs(case, f16=True)
    b = hip_outputs(case, f16=True, by_ids=True)
    assert np.array_equal(a, b)


@pytest.mark.parametrize("key", ["c3b", "c4"])
def test_device_ids_without_position_tables(key):
    """Plans whose embedding is a plain layernorm of the word rows (DeBERTa, ModernBERT) gather the
    rows from the device word table inside that layernorm; the ids path meets the oracle's bars and
    stays within f16 rounding of the host-rows path."""
    case, ref = case_and_oracle(key)
    rows = hip_outputs(case, f16=True)
    ids = hip_outputs(case, f16=True, by_ids=True)
    if key == "c4":
        assert cosine_rows(ref, ids).min() >= 0.999
        assert cosine_rows(rows, ids).min() >= 0.9999
    else:
        d = decision_parity(ref, ids)
        assert d["mismatched"] == 0 and d["delta"] <= 2e-2, d
        assert np.abs(rows - ids).max() <= 2e-2


@pytest.mark.parametrize("tile", [None, "9", "12", "14"], ids=["picked", "192x256", "128x384", "256x256"])
def test_fused_product_steps_match_separate_ops(monkeypatch, tile):
    """ModernBERT: GEMM + GeGLU, GEMM + RoPE and GEMM + residual add run fused in the product's
    epilogue; with fusion off (KH_NO_FUSION) the separate kernels run. Both apply the same f32
    formulas to the same f16 products, so the results are identical, whatever tile the products
    run in (KH_GEMM_TILE forces one for every product)."""
    case, ref = case_and_oracle("c4")
    if tile:
        monkeypatch.setenv("KH_GEMM_TILE", tile)
    fused = hip_outputs(case, f16=True)
    monkeypatch.setenv("KH_NO_FUSION", "1")
    separate = hip_outputs(case, f16=True)
    print(f"fused vs separate: max |d| {np.abs(fused - separate).max():.3e}")
    assert np.array_equal(fused, separate)
    assert cosine_rows(ref, fused).min() >= 0.999


def test_fused_products_with_biases_match_separate_ops(monkeypatch):
    """A ModernBERT with attention and MLP biases (spec bias=True): the fused GeGLU epilogue takes
    each half's bias from that half's rows of the FFN-in product, as the separate product does."""
    from kleinhirn_amd.plan import spec as S
    from tests.helpers import Case
    base, _ = case_and_oracle("c4")
    spec = S.modernbert(384, 2, 6, 576, 50368, bias=True)
    case = Case(spec, base.head, base.ids, base.length)
    for name in ("layers.0.mlp_in.bias", "layers.0.wqkv.bias", "layers.1.attn_out.bias"):
        assert np.abs(case.weights[name]).max() > 0, name  # seeded N(0, 0.02) biases, not zeros
    fused = hip_outputs(case, f16=True)
    monkeypatch.setenv("KH_NO_FUSION", "1")
    separate = hip_outputs(case, f16=True)
    assert np.array_equal(fused, separate), np.abs(fused - separate).max()


def _layernorm_launches(case, f16=True):
    """Outputs and the number of LayerNorm launches of one forward of the case's batch plan."""
    from kleinhirn_amd.backend import HipBackend
    W = configs.storage(case.weights, f16)
    be = HipBackend(W)
    r = be.runner(build_plan(case.spec, case.head, case.length, len(case.ids), f16))
    r.upload(inputs.run_input(case.spec, W["embeddings.word.weight"], case.ids, case.length))
    r.trace(True)
    r.run(case.length * len(case.ids))
    out = r.read_output().reshape(len(case.ids), -1)
    launches = r.trace_read()
    r.trace(False)
    r.destroy()
    be.dispose()
    return out, sum(1 for l in launches if l["kernel"] == "layernorm")


def test_fused_residual_layernorm_matches_separate_ops(monkeypatch):
    """XLM-R MiniLM (post-LN, 384-wide rows): the out projection and FFN out run with the residual
    + LayerNorm (MODE 2) in the product's epilogue, one 128 x 384 tile per row band, the lanes,
    sums and shuffles of the separate LayerNorm; with fusion off (KH_NO_FUSION) the separate
    kernels run. The outputs are identical, and the fused forward launches no LayerNorm of its own
    (the embedding's runs in the embedding kernel)."""
    case, ref = case_and_oracle("c5")
    fused, n_fused = _layernorm_launches(case)
    monkeypatch.setenv("KH_NO_FUSION", "1")
    separate, n_separate = _layernorm_launches(case)
    print(f"LayerNorm launches fused {n_fused}, separate {n_separate}; max |d| {np.abs(fused - separate).max():.3e}")
    assert n_separate == n_fused + 2 * case.spec["layers"], (n_fused, n_separate)
    assert np.array_equal(fused, separate)
    assert cosine_rows(ref, fused).min() >= 0.999


@pytest.mark.parametrize("key", ["c2", "c3b", "c4", "c5"])
def test_cls_tail_on_sequence_rows_equals_full_forward(monkeypatch, key):
    """A pooled-CLS head reads row 0 of each sequence after the last attention, so the runner runs
    the rest of the encoder on one row per sequence (and the last attention on each sequence's
    first query tile); with KH_NO_PRUNE every row runs. The kept rows go through the same f16
    kernels in the same accumulation order, so the outputs are identical."""
    case, ref = case_and_oracle(key)
    pruned = hip_outputs(case, f16=True)
    monkeypatch.setenv("KH_NO_PRUNE", "1")
    full = hip_outputs(case, f16=True)
    print(f"{key} pruned vs full: max |d| {np.abs(pruned - full).max():.3e}")
    assert np.array_equal(pruned, full)


def test_cls_tail_f32_matches_full_forward_and_oracle(monkeypatch):
    """f32: the B-row products of the pruned tail are too small for the MFMA tiles and run on the
    wavefront-per-output kernel (another summation order), so the bar is the f32 parity bar."""
    case, ref = case_and_oracle("c2")
    pruned = hip_outputs(case, f16=False)
    monkeypatch.setenv("KH_NO_PRUNE", "1")
    full = hip_outputs(case, f16=False)
    print(f"c2 f32 pruned vs full: max |d| {np.abs(pruned - full).max():.3e}")
    assert np.abs(pruned - full).max() <= 1e-4
    check_f32("c2", ref, pruned)


def test_cls_tail_with_empty_sequences_and_moved_markers(monkeypatch):
    """Sequences cut to 0 rows by the run's row count gather zero states in both forms; a marker
    other than row 0 switches the runner back to the full forward (the gather then reads that row)."""
    from kleinhirn_amd.backend import HipBackend
    case, _ = case_and_oracle("c2")
    W = configs.storage(case.weights, True)
    be = HipBackend(W)
    table = W["embeddings.word.weight"]
    B, L = len(case.ids), case.length
    plan = build_plan(case.spec, case.head, L, B, True)
    rows = L * (B - 2) + 5  # sequence B - 2 keeps at most 5 rows, sequence B - 1 none

    def run(markers=None):
        r = be.runner(plan)
        if markers is not None:
            r.init_buffer("first", markers.tobytes())
        r.upload(inputs.run_input(case.spec, table, case.ids, L))
        r.run(rows)
        out = r.read_output().reshape(B, -1)
        r.destroy()
        return out

    moved = np.zeros(3 * B, dtype=np.uint32)
    moved[3 * 1] = 2  # sequence 1 takes its row 2
    pruned, pruned_moved = run(), run(moved)
    monkeypatch.setenv("KH_NO_PRUNE", "1")
    full, full_moved = run(), run(moved)
    assert np.array_equal(pruned, full)
    assert np.array_equal(pruned_moved, full_moved)
    assert not np.array_equal(pruned_moved[1], pruned[1])
    assert np.array_equal(np.delete(pruned_moved, 1, axis=0), np.delete(pruned, 1, axis=0))


@pytest.mark.parametrize("key", ["c2", "c5", "c4"])
def test_read_scores_equals_scores_of_the_output(key):
    """kh_read_scores on the device output equals kh_scores of kh_read_output, and its labels
    equal the oracle's decisions wherever f16 rounding cannot flip them."""
    from kleinhirn_amd import backend as B
    from oracle import postprocess as P
    case, ref = case_and_oracle(key)
    kind = {"c2": B.SCORES_SOFTMAX, "c5": B.SCORES_RAW, "c4": B.SCORES_L2}[key]
    W = configs.storage(case.weights, True)
    be = B.HipBackend(W)
    plan = build_plan(case.spec, case.head, case.length, len(case.ids), True)
    r = be.runner(plan)
    r.upload(inputs.run_input(case.spec, W["embeddings.word.weight"], case.ids, case.length))
    r.run(case.length * len(case.ids))
    out = r.read_output().reshape(len(case.ids), -1)
    s, idx = r.read_scores(kind)
    s2, idx2 = B.scores(out, kind)
    assert np.array_equal(s, s2) and np.array_equal(idx, idx2)
    want, widx = P.scores(ref.astype(np.float32), kind)
    if kind == B.SCORES_SOFTMAX:
        d = decision_parity(ref, out)
        assert d["mismatched"] == 0, d
    if kind == B.SCORES_L2:
        assert cosine_rows(want, s).min() >= 0.999
    r.destroy()
    be.dispose()


TOKEN_HEAD = {"type": "token", "steps": [{"op": "dense", "name": "head.tok", "in": 768, "out": 5, "act": "none",
                                          "bias": True}]}


def token_case():
    """A token-classification head (one dense step per row, src/plan/build.ts token branch) on two
    RoBERTa-base layers and six ragged c2 sequences."""
    from tests.helpers import Case
    c = workload_case("c2", 6, 2, 512)
    return Case(c.spec, TOKEN_HEAD, c.ids, c.length)


def token_oracle(case) -> list:
    """The oracle's rows of each sequence (a B = 1 plan per sequence), [len, classes] each."""
    from oracle.oracle import OracleRuntime
    plan = build_plan(case.spec, case.head, case.length, 1, False)
    p = OracleRuntime(case.weights, [plan]).plan(plan, threads=8)
    table = case.weights["embeddings.word.weight"]
    outs = []
    for seq in case.ids:
        ri = inputs.run_input(case.spec, table, [seq], case.length)
        p.upload(ri["embeddings"], ri["mask"], ri["typeIds"])
        p.run(len(seq))
        outs.append(p.read_output().reshape(case.length, -1)[:len(seq)])
    return outs


@pytest.mark.parametrize("f16", [False, True], ids=["f32", "f16"])
def test_token_head_matches_oracle(f16):
    """Per-token logits of the token head: row i of sequence b at b * L + i, zeros past each
    sequence; f32 within 1e-3 with identical argmax, f16 with identical decisions outside close calls."""
    case = token_case()
    ref = token_oracle(case)
    got = hip_outputs(case, f16).reshape(len(case.ids), case.length, -1)
    for b, r in enumerate(ref):
        n = len(r)
        assert not got[b, n:].any(), f"sequence {b}: rows past the sequence are not zero"
        if f16:
            d = decision_parity(r, got[b, :n])
            assert d["mismatched"] == 0, (b, d)
            assert cosine_rows(r, got[b, :n]).min() >= 0.999
        else:
            assert np.abs(r - got[b, :n]).max() <= 1e-3, (b, np.abs(r - got[b, :n]).max())
            assert np.array_equal(r.argmax(1), got[b, :n].argmax(1))
