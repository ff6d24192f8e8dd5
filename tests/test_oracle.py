"""The CPU oracle's op computations against f64 numpy restatements, the way the reference checks its
WASM executor (tests/wasm_plan.test.ts:1-401): one-op plans on LCG-random inputs with odd sizes,
NaN-filled padding rows that must never be read, prefix masks, two sequences, windows; tolerance
2e-5 of the largest reference value (tests/wasm_plan.test.ts:30-38). Plus the mask-sentinel cases
(tests/mask_sentinel.test.ts:36-60), closed forms of exp and GELU, and invariance under thread
count and batching (src/wasm/plan.ts:942-950)."""
from __future__ import annotations

import ctypes
import math

import numpy as np
import pytest
from scipy.special import erf

from kleinhirn_amd import configs
from kleinhirn_amd.plan.build import rel_pos_table
from oracle import oracle as O
from tests.helpers import Case, oracle_outputs


class Rand:
    """The reference's test LCG: seed = seed * 1103515245 + 12345 (mod 2^32), value in [-1, 1)
    (tests/wasm_plan.test.ts:13-18)."""

    def __init__(self, seed=12345):
        self.s = seed

    def arr(self, n, scale=1.0):
        out = np.empty(n, dtype=np.float32)
        for i in range(n):
            self.s = (self.s * 1103515245 + 12345) & 0xFFFFFFFF
            out[i] = (self.s / 4294967296 * 2 - 1) * scale
        return out


R = Rand()


def gelu(v):
    return 0.5 * v * (1 + erf(v / math.sqrt(2)))


ACT = [lambda v: v, lambda v: np.maximum(v, 0), gelu, np.tanh, lambda v: v / (1 + np.exp(-v))]


def close(got, want, what, tol=2e-5):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    assert got.shape == want.shape, f"{what}: shape {got.shape} vs {want.shape}"
    scale = max(1.0, float(np.abs(want).max()))
    assert np.isfinite(got).all(), f"{what}: non-finite"
    err = np.abs(got - want).max()
    assert err <= tol * scale, f"{what}: error {err} > {tol * scale}"


def mini(L, buffers, ops, out, weights=None, batch=1, panels=()):
    """One-plan runtime in the shape of the reference test's mini() (tests/wasm_plan.test.ts:49-66)."""
    bufs = []
    for bid, v in buffers.items():
        if isinstance(v, np.ndarray):
            bufs.append({"id": bid, "bytes": v.nbytes, "usage": "rw", "init": v})
        else:
            bufs.append({"id": bid, "bytes": 4 * v, "usage": "rw"})
    plan = {"f16": False, "length": L, "batch": batch, "markers": 0, "embeddingSize": 1, "buffers": bufs,
            "segments": [{"name": "s", "prefix": "", "ops": ops}], "inputs": {"embeddings": "mask", "mask": "mask"},
            "output": {"buffer": out, "bytes": 4 * buffers[out], "dtype": "f32", "rows": buffers[out], "cols": 1},
            "captureSlots": 0, "captureSlotBytes": 0}
    rt = O.OracleRuntime(weights or {}, [plan])
    return rt.plan(plan)


def prefix_mask(L, lens):
    m = np.zeros(L * len(lens), dtype=np.float32)
    for b, n in enumerate(lens):
        m[b * L:b * L + n] = 1
    return m


@pytest.mark.parametrize("N", [37, 3, 16, 40])
def test_matmul_all_activations(N):
    M = 9 if N == 40 else 7
    K = 19
    W = R.arr(N * K).reshape(N, K)
    B = R.arr(N)
    for act in range(5):
        for fixed in (False, True):
            p = mini(M, {"mask": M, "a": M * K, "c": M * N},
                     [{"name": "mm", "kernel": "mmtile", "constants": {"M": M, "N": N, "K": K, "ACT": act},
                       "bind": ["a", "w:w", "w:b", "c"], "dispatch": [1, 1 if fixed else "rows32"]}], "c",
                     {"w": W, "b": B})
            A = R.arr(M * K, 2)
            p.view("a")[:] = A
            rows = M if fixed else 5
            p.run(1 if fixed else rows)
            want = ACT[act](A.reshape(M, K)[:rows].astype(np.float64) @ W.T.astype(np.float64) + B)
            close(p.view("c")[:rows * N].reshape(rows, N), want, f"N {N} act {act} fixed {fixed}")


def test_layernorm_and_embln():
    N, rows = 21, 5
    w, bias = R.arr(N), R.arr(N)

    def ref(v, scale):
        v = np.asarray(v, dtype=np.float64)
        mean = v.mean()
        var = ((v - mean) ** 2).mean()
        return ((v - mean) / np.sqrt(var + 1e-5) * w + bias) * scale

    for mode in (0, 1, 2):
        p = mini(rows, {"mask": rows, "a": rows * N, "b": rows * N, "o": rows * N},
                 [{"name": "ln", "kernel": "layernorm", "constants": {"N": N, "MODE": mode, "EPS": 1e-5},
                   "bind": ["a", "b", "w:w", "w:bias", "mask", "o"], "dispatch": ["rows", 1]}], "o",
                 {"w": w, "bias": bias})
        a, b = R.arr(rows * N, 3), R.arr(rows * N, 3)
        mask = np.array([1, 1, 0, 1, 0], np.float32)
        p.view("a")[:] = a
        p.view("b")[:] = b
        p.view("mask")[:] = mask
        p.run(rows)
        want = [ref(a[r * N:(r + 1) * N] + (b[r * N:(r + 1) * N] if mode == 2 else 0), mask[r] if mode == 1 else 1)
                for r in range(rows)]
        close(p.view("o"), np.concatenate(want), f"mode {mode}")
    # embln: L 6, offset 2, 9 position rows (clamped), 3 types, POSIDS from the high 16 bits
    L, P = 6, 9
    pos, typ = R.arr(P * N), R.arr(3 * N)
    for posids in (0, 1):
        for maskmul in (0, 1):
            p = mini(L, {"mask": 2 * L, "word": 2 * L * N, "tt": 2 * L, "o": 2 * L * N},
                     [{"name": "e", "kernel": "embln",
                       "constants": {"N": N, "L": L, "OFFSET": 2, "MAXPOS": P, "EPS": 1e-5, "MASKMUL": maskmul, "POSIDS": posids},
                       "bind": ["word", "w:pos", "w:typ", "tt", "w:w", "w:bias", "mask", "o"], "dispatch": ["rows", 1]}],
                     "o", {"pos": pos.reshape(P, N), "typ": typ.reshape(3, N), "w": w, "bias": bias}, batch=2)
            word = R.arr(2 * L * N)
            types = np.array([(i % 3) | ((((i * 5) % P) << 16) if posids else 0) for i in range(2 * L)], np.uint32)
            mask = prefix_mask(L, [4, 6])
            p.view("word")[:] = word
            p.view("mask")[:] = mask
            p.view("tt", np.uint32)[:] = types
            p.run(2 * L)
            want = []
            for r in range(2 * L):
                prow = min((types[r] >> 16) if posids else (r % L) + 2, P - 1)
                v = word[r * N:(r + 1) * N] + pos[prow * N:(prow + 1) * N] + typ[(types[r] & 0xFFFF) * N:((types[r] & 0xFFFF) + 1) * N]
                want.append(ref(v.astype(np.float64), mask[r] if maskmul else 1))
            close(p.view("o"), np.concatenate(want), f"embln posids {posids} maskmul {maskmul}")


def test_add_gather_pool_geglu_rope():
    L, N, B = 7, 6, 2
    for mode in (0, 1):
        p = mini(L, {"mask": B * L, "dst": B * L * N, "src": B * L * N},
                 [{"name": "a", "kernel": "add", "constants": {"TOTAL": B * L * N, "N": N, "MODE": mode, "L": L},
                   "bind": ["dst", "src"], "dispatch": [1, 1]}], "dst", batch=B)
        d, s = R.arr(B * L * N), R.arr(B * L * N)
        p.view("dst")[:] = d
        p.view("src")[:] = s
        p.run(B * L)
        i = np.arange(B * L * N)
        close(p.view("dst"), d + (s[(i // (N * L)) * N + i % N] if mode else s), f"add {mode}")
    K = 3
    marks = np.array([2, 0, 5, 0, 0, 0, 0, 0, 0, 6, 1, 3, 0, 0, 0, 0, 0, 0], np.uint32)
    p = mini(L, {"mask": B * L, "mk": marks, "x": B * L * N, "st": B * K * N},
             [{"name": "g", "kernel": "gather", "constants": {"K": K, "D": N, "L": L}, "bind": ["mk", "x", "st"],
               "dispatch": [1, 1]}], "st", batch=B)
    x = R.arr(B * L * N)
    p.view("x")[:] = x
    p.run(B * L)
    want = [x[(g // K * L + marks[g // K * 3 * K + g % K]) * N:][:N] for g in range(B * K)]
    close(p.view("st"), np.concatenate(want), "gather")
    for mode in (0, 1):
        p = mini(L, {"mask": B * L, "x": B * L * N, "o": B * N},
                 [{"name": "p", "kernel": "pool", "constants": {"L": L, "N": N, "MODE": mode},
                   "bind": ["x", "mask", "o"], "dispatch": [1, B]}], "o", batch=B)
        x = R.arr(B * L * N)
        mask = prefix_mask(L, [3, 7])
        xx = x.reshape(B * L, N).copy()
        xx[mask == 0] = np.nan  # padding rows are never read
        p.view("x")[:] = xx.reshape(-1)
        p.view("mask")[:] = mask
        p.run(B * L)
        want = []
        for b, n in enumerate([3, 7]):
            seq = xx[b * L:b * L + n].astype(np.float64)
            want.append(seq.max(0) if mode else seq.mean(0))
        close(p.view("o"), np.concatenate(want), f"pool {mode}")
    I = 5
    p = mini(L, {"mask": L, "mid": L * 2 * I, "g": L * I},
             [{"name": "gg", "kernel": "geglu", "constants": {"I": I}, "bind": ["mid", "g"], "dispatch": ["rows", 1]}], "g")
    mid = R.arr(L * 2 * I, 3)
    p.view("mid")[:] = mid
    p.run(L)
    m2 = mid.reshape(L, 2 * I).astype(np.float64)
    close(p.view("g"), (gelu(m2[:, :I]) * m2[:, I:]).reshape(-1), "geglu")
    H, D = 2, 6
    table = np.zeros((L, 2 * D), np.float32)
    for i in range(L):
        for d in range(D // 2):
            f = i * 10000 ** (-(2 * d) / D)
            table[i, d], table[i, D + d] = math.cos(f), math.sin(f)
    p = mini(L, {"mask": B * L, "qkv": B * L * 3 * H * D, "cs": table.reshape(-1)},
             [{"name": "r", "kernel": "rope", "constants": {"L": L, "H": H, "D": D}, "bind": ["qkv", "cs"],
               "dispatch": ["rows", 2 * H]}], "qkv", batch=B)
    qkv = R.arr(B * L * 3 * H * D)
    p.view("qkv")[:] = qkv
    p.run(B * L)
    want = qkv.astype(np.float64).reshape(B * L, 3 * H * D).copy()
    q = qkv.reshape(B * L, 3 * H * D)
    for r in range(B * L):
        for s in range(2 * H):
            for d in range(D // 2):
                a, b = q[r, s * D + d], q[r, s * D + d + D // 2]
                c, sn = table[r % L, d], table[r % L, D + d]
                want[r, s * D + d] = a * c - b * sn
                want[r, s * D + d + D // 2] = b * c + a * sn
    close(p.view("qkv"), want.reshape(-1), "rope")


def attention_ref(qkv, mask, L, B, H, D, scale, window, rows, rel=None):
    """f64 attention over padded sequences (tests/wasm_plan.test.ts:297-334)."""
    hd = H * D
    out = np.zeros((rows, hd))
    for i in range(rows):
        b, il = divmod(i, L)
        if mask[i] <= 0.5:
            continue
        for h in range(H):
            keys, s = [], []
            for j in range(L):
                if mask[b * L + j] <= 0.5 or (window and abs(il - j) > window):
                    continue
                q = qkv[i, h * D:(h + 1) * D].astype(np.float64)
                k = qkv[b * L + j, (H + h) * D:(H + h + 1) * D].astype(np.float64)
                v = q @ k
                if rel is not None:
                    idx, pk, pq = rel
                    pp = idx[il * L + j]
                    v += q @ pk[pp, h * D:(h + 1) * D] + k @ pq[pp, h * D:(h + 1) * D]
                keys.append(j)
                s.append(v / scale if rel is not None else v * scale)
            s = np.array(s)
            e = np.exp(s - s.max())
            pm = e / e.sum()
            for n, j in enumerate(keys):
                out[i, h * D:(h + 1) * D] += pm[n] * qkv[b * L + j, (2 * H + h) * D:(2 * H + h + 1) * D]
    return out


SPAN = 4


def rel_table(L):
    i = np.arange(L)[:, None]
    j = np.arange(L)[None, :]
    return np.clip(i - j + SPAN, 0, 2 * SPAN - 1).astype(np.uint32).reshape(-1)


@pytest.mark.parametrize("L,D,lens,window", [(7, 5, [5], 0), (9, 6, [4, 9], 0), (9, 6, [9, 6], 2), (12, 8, [12], 0)])
def test_attention_split_and_fused(L, D, lens, window):
    B, H = len(lens), 2
    hd = H * D
    rows = lens[0] if B == 1 else B * L
    qkv = R.arr(B * L * 3 * hd, 2).reshape(B * L, 3 * hd)
    mask = prefix_mask(L, lens)
    qkv[mask == 0] = np.nan  # stale padding rows never enter a sum
    want = attention_ref(qkv, mask, L, B, H, D, 0.3, window, rows)
    base = {"L": L, "H": H, "D": D}
    for kind in ("split", "mbflash", "mbattention"):
        if kind == "split":
            ops = [{"name": "s", "kernel": "attscore", "constants": {**base, "SCALE": 0.3, "ROWS": B * L}, "bind": ["qkv", "ki", "sc"], "dispatch": [1, "rows32"]},
                   {"name": "p", "kernel": "attsoftmax", "constants": {"L": L, "H": H, "WINDOW": window}, "bind": ["mask", "sc"], "dispatch": [H, "rows"]},
                   {"name": "v", "kernel": "attpv", "constants": {**base, "ROWS": B * L}, "bind": ["sc", "qkv", "mask", "ki", "ctx"], "dispatch": [1, "rows32"]}]
        else:
            ops = [{"name": "a", "kernel": kind, "constants": {**base, "SCALE": 0.3, "WINDOW": window, "ROWS": B * L},
                    "bind": ["qkv", "mask", "ctx"], "dispatch": [H, "rows"]}]
        p = mini(L, {"mask": B * L, "qkv": B * L * 3 * hd, "ki": 2 * B, "sc": B * L * H * L, "ctx": B * L * hd}, ops,
                 "ctx", batch=B)
        p.view("qkv")[:] = qkv.reshape(-1)
        p.view("mask")[:] = mask
        p.run(rows)
        got = p.view("ctx")[:rows * hd].reshape(rows, hd)
        valid = mask[:rows] > 0.5
        close(got[valid], want[valid], kind)
        assert np.all(got[~valid] == 0), f"{kind}: masked query rows must be zero"


@pytest.mark.parametrize("L,D,lens", [(7, 5, [5]), (9, 6, [4, 9]), (12, 8, [12])])
def test_relative_attention_split_and_fused(L, D, lens):
    B, H = len(lens), 2
    hd = H * D
    rows = lens[0] if B == 1 else B * L
    qkv = R.arr(B * L * 3 * hd, 2).reshape(B * L, 3 * hd)
    mask = prefix_mask(L, lens)
    qkv[mask == 0] = np.nan
    idx = rel_table(L)
    pk = R.arr(2 * SPAN * hd).reshape(2 * SPAN, hd)
    pq = R.arr(2 * SPAN * hd).reshape(2 * SPAN, hd)
    scale = math.sqrt(3 * D)
    want = attention_ref(qkv, mask, L, B, H, D, scale, 0, rows, (idx, pk.astype(np.float64), pq.astype(np.float64)))
    moff = int(idx[L - 1])
    nm = int(idx[(L - 1) * L]) - moff + 1
    relc = {"H": H, "D": D, "ROWS": B * L, "NM": nm, "MOFF": moff, "L": L}
    for fused in (False, True):
        if fused:
            ops = [{"name": "a", "kernel": "attention", "constants": {"L": L, "H": H, "D": D, "SCALE": scale},
                    "bind": ["qkv", "w:pk", "w:pq", "ri", "mask", "ctx"], "dispatch": [H, "rows"]}]
        else:
            ops = [{"name": "c", "kernel": "attrel", "constants": {**relc, "PART": 0}, "bind": ["qkv", "w:pk", "ki", "ri", "c2p"], "dispatch": [1, "rows32"]},
                   {"name": "p", "kernel": "attrel", "constants": {**relc, "PART": 1}, "bind": ["qkv", "w:pq", "ki", "ri", "p2c"], "dispatch": [1, "rows32"]},
                   {"name": "s", "kernel": "attscore", "constants": {"L": L, "H": H, "D": D, "SCALE": 1 / scale, "ROWS": B * L}, "bind": ["qkv", "ki", "sc"], "dispatch": [1, "rows32"]},
                   {"name": "sr", "kernel": "attsoftrel", "constants": {"L": L, "H": H, "NM": nm, "MOFF": moff, "INVSCALE": 1 / scale}, "bind": ["mask", "ri", "c2p", "p2c", "sc"], "dispatch": [H, "rows"]},
                   {"name": "v", "kernel": "attpv", "constants": {"L": L, "H": H, "D": D, "ROWS": B * L}, "bind": ["sc", "qkv", "mask", "ki", "ctx"], "dispatch": [1, "rows32"]}]
        p = mini(L, {"mask": B * L, "qkv": B * L * 3 * hd, "ki": 2 * B, "ri": idx, "sc": B * L * H * L,
                     "c2p": B * L * H * nm, "p2c": B * L * H * nm, "ctx": B * L * hd}, ops, "ctx",
                 {"pk": pk, "pq": pq}, batch=B)
        p.view("qkv")[:] = qkv.reshape(-1)
        p.view("mask")[:] = mask
        p.run(rows)
        got = p.view("ctx")[:rows * hd].reshape(rows, hd)
        valid = mask[:rows] > 0.5
        close(got[valid], want[valid], "fused" if fused else "split")
        assert np.all(got[~valid] == 0)


# ---- mask sentinel (tests/mask_sentinel.test.ts:36-60) ---------------------------------------

def softmax(scores, keep, dense=False):
    lib = O.lib()
    lib.kho_softmax_row.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                    ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_float]
    p = np.asarray(scores, dtype=np.float32).copy()
    m = np.asarray(keep, dtype=np.float32)
    lib.kho_softmax_row(p.ctypes.data, len(p), m.ctypes.data, 0, 0, 0, 1, int(dense), 1.0)
    return p


def test_masked_keys_get_zero_weight_below_minus_1e4():
    w = softmax([-31000, -30500, -24000, -29000, -2, -2, -2, -2], [1, 1, 1, 1, 0, 0, 0, 0])
    assert w[4:].sum() == 0
    assert abs(w[:4].sum() - 1) < 1e-6


def test_masked_keys_get_zero_weight_below_minus_1e30():
    w = softmax([-1e31, -2e31, 9, 9], [1, 1, 0, 0])
    assert w[2] + w[3] == 0
    assert w[0] == 1


def test_usual_scores_keep_their_order_and_no_key_gives_zeros():
    w = softmax([-13.4, -1.6, -5, -2, 0, 0], [1, 1, 1, 1, 0, 0])
    assert w[4] == 0 and w[5] == 0
    assert w[1] > w[3] > w[2] > w[0]
    assert np.all(softmax([1, 2, 3, 4], [0, 0, 0, 0]) == 0)


def test_dense_softmax_equals_general_path():
    s = R.arr(37, 8)
    a = softmax(s, np.ones(37), dense=True)
    b = softmax(s, np.ones(37), dense=False)
    close(a, b, "dense vs general", 1e-6)


# ---- closed forms ----------------------------------------------------------------------------

def test_vexp_and_gelu_closed_forms():
    lib = O.lib()
    xs = np.linspace(-87, 88, 20001).astype(np.float32)
    ve = np.array([lib.kho_vexp(float(x)) for x in xs[::10]])
    ref = np.exp(xs[::10].astype(np.float64))
    assert np.max(np.abs(ve - ref) / ref) < 3e-7  # Cephes expf: about 1 ulp
    gs = np.linspace(-8, 8, 4001).astype(np.float32)
    exact = gelu(gs.astype(np.float64))
    for name in ("kho_gelu", "kho_vgelu"):
        f = getattr(lib, name)
        got = np.array([f(float(x)) for x in gs])
        assert np.max(np.abs(got - exact)) < 3e-7 * 8, name  # A&S 7.1.26: |erf error| <= 1.5e-7
    # GELU odd symmetry of the erf part: gelu(x) - gelu(-x) = x
    g = np.array([lib.kho_gelu(float(x)) for x in gs]) - np.array([lib.kho_gelu(float(-x)) for x in gs])
    assert np.max(np.abs(g - gs)) < 1e-5


def test_relative_bucket_table_pins():
    """DeBERTa buckets: double-precision table of the plan builder equals the float32 HF formula
    for every offset at span 256 / max 512 (src/plan/build.ts:22-45); L = 512 gives MOFF 1, NM 511."""
    t = rel_pos_table(512, 256, 512).reshape(512, 512)
    rel = np.arange(-511, 512)
    mid = 128
    sign = np.sign(rel)
    abs_pos = np.where((rel < mid) & (rel > -mid), mid - 1, np.abs(rel)).astype(np.float32)
    log_pos = np.ceil(np.log(abs_pos / mid) / np.log(np.float32((512 - 1) / mid)) * (mid - 1)).astype(np.float32) + mid
    hf = np.where(abs_pos <= mid, rel, log_pos * sign).astype(np.int64) + 256
    hf = np.clip(hf, 0, 511)
    mine = np.array([t[d, 0] if d >= 0 else t[0, -d] for d in rel])
    assert np.array_equal(mine, hf)
    assert t[0, 511] == 1 and t[511, 0] - t[0, 511] + 1 == 511


# ---- invariances -----------------------------------------------------------------------------

def test_thread_count_and_batch_invariance():
    w = configs.c2(4)
    spec = dict(w.spec, layers=2, vocab=3000)
    ids = [x % 3000 for x in w.ids()]
    case = Case(spec, w.head, ids, 128)
    one = oracle_outputs(case, threads=1)
    four = oracle_outputs(case, threads=4)
    assert np.array_equal(one, four)
    # a batch plan (padded rows computed, masked out by attention) equals the single plans
    from kleinhirn_amd import inputs
    from kleinhirn_amd.plan.build import build_plan
    plan = build_plan(spec, w.head, 128, len(ids), False)
    p = O.OracleRuntime(case.weights, [plan]).plan(plan, threads=4)
    ri = inputs.run_input(spec, case.weights["embeddings.word.weight"], ids, 128)
    p.upload(ri["embeddings"], ri["mask"], ri["typeIds"])
    p.run(128 * len(ids))
    close(p.read_output().reshape(len(ids), -1), one, "batch vs single", 1e-6)
