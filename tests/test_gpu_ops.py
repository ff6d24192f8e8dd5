"""Op-level parity of the HIP kernels through the C ABI: one-op plans (the way the reference's
tests/wasm_plan.test.ts checks each WASM computation) against f64 numpy restatements, on ragged
prefix masks, odd widths and both storage types. The input of each plan is its 'emb' buffer, so
the rows go through the same packing (cu_seqlens) as a model run."""
from __future__ import annotations

import math

import numpy as np
import pytest

from kleinhirn_amd.plan.build import rel_pos_table

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(12345)


def _backend(weights):
    from kleinhirn_amd.backend import HipBackend
    return HipBackend(weights)


def mini_plan(f16, L, B, E, ops, buffers, out, out_cols, inputs_extra=None):
    es = 2 if f16 else 4
    bufs = [{"id": "emb", "bytes": L * B * E * es, "usage": "rw"},
            {"id": "mask", "bytes": L * B * 4, "usage": "rw"}]
    for bid, elems in buffers.items():
        if isinstance(elems, np.ndarray):
            bufs.append({"id": bid, "bytes": elems.nbytes, "usage": "rw", "init": elems})
        else:
            bufs.append({"id": bid, "bytes": int(math.ceil(elems * es / 4) * 4), "usage": "rw"})
    inputs = {"embeddings": "emb", "mask": "mask"}
    inputs.update(inputs_extra or {})
    return {"f16": f16, "length": L, "batch": B, "markers": 0, "embeddingSize": E, "buffers": bufs,
            "segments": [{"name": "s", "prefix": "", "ops": ops}], "inputs": inputs,
            "output": {"buffer": out, "bytes": L * B * out_cols * es, "dtype": "storage",
                       "rows": L * B, "cols": out_cols},
            "captureSlots": 0, "captureSlotBytes": 0}


def prefix_mask(L, lens):
    m = np.zeros(L * len(lens), dtype=np.float32)
    for b, n in enumerate(lens):
        m[b * L:b * L + n] = 1
    return m


def run_plan(plan, weights, emb, mask, rows, type_ids=None):
    be = _backend(weights)
    try:
        be.check(plan)
        r = be.runner(plan)
        r.upload({"embeddings": emb, "mask": mask, "typeIds": type_ids})
        r.run(rows)
        out = r.read_output()
        r.destroy()
        return out
    finally:
        be.dispose()


def gelu(v):
    from scipy.special import erf
    return 0.5 * v * (1 + erf(v / math.sqrt(2)))


ACTS = [lambda v: v, lambda v: np.maximum(v, 0), gelu, np.tanh, lambda v: v / (1 + np.exp(-v))]


def close(got, want, tol, what):
    scale = max(1.0, float(np.abs(want).max()))
    err = float(np.abs(got - want).max())
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    assert err <= tol * scale, f"{what}: max error {err} (scale {scale}, tol {tol})"


@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("N,K,lens", [(384, 768, [5, 130]), (2304, 768, [257]), (37, 64, [7, 3]),
                                      (3, 768, [1, 4]), (1536, 384, [64, 64, 1]), (200, 136, [129]),
                                      (768, 3072, [300, 77]), (3072, 768, [193]), (768, 768, [1]),
                                      (2, 768, [3, 1]), (3, 40, [2]), (200, 768, [129]), (264, 512, [70, 3])])
def test_matmul_against_f64(f16, N, K, lens):
    L = max(lens)
    B = len(lens)
    dt = np.float16 if f16 else np.float32
    W = (RNG.standard_normal((N, K)) * 0.05).astype(dt)
    bias = (RNG.standard_normal(N) * 0.1).astype(dt)
    A = (RNG.standard_normal((L * B, K))).astype(dt)
    mask = prefix_mask(L, lens)
    for act in range(5):
        op = {"name": "mm", "kernel": "mmtile", "constants": {"M": L * B, "N": N, "K": K, "ACT": act},
              "bind": ["emb", "w:w", "w:b", "c"], "dispatch": [math.ceil(N / 64), "rows32"]}
        plan = mini_plan(f16, L, B, K, [op], {"c": L * B * N}, "c", N)
        out = run_plan(plan, {"w": W, "b": bias}, A, mask, L * B).reshape(L * B, N)
        valid = mask > 0.5
        want = ACTS[act](A.astype(np.float64) @ W.astype(np.float64).T + bias.astype(np.float64))
        close(out[valid], want[valid], 5e-3 if f16 else 2e-5, f"act {act} f16 {f16}")
        assert np.all(out[~valid] == 0), "padding rows must read back as zero"


@pytest.mark.parametrize("N,K", [(768, 1536), (200, 768)])
@pytest.mark.parametrize("tile", list(range(15)))
def test_matmul_every_tile_configuration(tile, N, K, monkeypatch):
    """Each GEMM tile configuration (forced through KH_GEMM_TILE) on a ragged f16 batch whose rows
    end inside a tile, against f64; N = 200 also ends inside a column tile of every width (the
    columns past N, whose bias reads are not used, are never stored)."""
    monkeypatch.setenv("KH_GEMM_TILE", str(tile))
    lens = [211, 5, 64]
    L, B = max(lens), len(lens)
    W = (RNG.standard_normal((N, K)) * 0.05).astype(np.float16)
    bias = (RNG.standard_normal(N) * 0.1).astype(np.float16)
    A = RNG.standard_normal((L * B, K)).astype(np.float16)
    mask = prefix_mask(L, lens)
    for act in (0, 2):
        op = {"name": "mm", "kernel": "mmtile", "constants": {"M": L * B, "N": N, "K": K, "ACT": act},
              "bind": ["emb", "w:w", "w:b", "c"], "dispatch": [math.ceil(N / 64), "rows32"]}
        plan = mini_plan(True, L, B, K, [op], {"c": L * B * N}, "c", N)
        out = run_plan(plan, {"w": W, "b": bias}, A, mask, L * B).reshape(L * B, N)
        valid = mask > 0.5
        want = ACTS[act](A.astype(np.float64) @ W.astype(np.float64).T + bias.astype(np.float64))
        close(out[valid], want[valid], 5e-3, f"tile {tile} act {act}")


@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("N", [384, 768, 40])
def test_layernorm_modes_and_embln(f16, N):
    """384 and 768: several rows per wavefront (lane groups); 40: one wavefront per row."""
    L, lens = 9, [4, 9]
    B = len(lens)
    dt = np.float16 if f16 else np.float32
    w = (1 + 0.1 * RNG.standard_normal(N)).astype(dt)
    bias = (0.1 * RNG.standard_normal(N)).astype(dt)
    a = (3 * RNG.standard_normal((L * B, N))).astype(dt)
    mask = prefix_mask(L, lens)
    valid = mask > 0.5

    def ref(v, eps):
        v = v.astype(np.float64)
        mean = v.mean(1, keepdims=True)
        var = ((v - mean) ** 2).mean(1, keepdims=True)
        return (v - mean) / np.sqrt(var + eps) * w.astype(np.float64) + bias.astype(np.float64)

    for mode in (0, 1):
        op = {"name": "ln", "kernel": "layernorm", "constants": {"N": N, "MODE": mode, "EPS": 1e-5},
              "bind": ["emb", "dummy", "w:w", "w:bias", "mask", "o"], "dispatch": ["rows", 1]}
        plan = mini_plan(f16, L, B, N, [op], {"o": L * B * N, "dummy": 1}, "o", N)
        out = run_plan(plan, {"w": w, "bias": bias}, a, mask, L * B).reshape(L * B, N)
        close(out[valid], ref(a, 1e-5)[valid], 1e-2 if f16 else 2e-5, f"mode {mode}")
    # MODE 2: LN(a + W a) through a matmul-produced second operand
    Wm = (0.05 * RNG.standard_normal((N, N))).astype(dt)
    ops = [{"name": "mm", "kernel": "mmtile", "constants": {"M": L * B, "N": N, "K": N, "ACT": 0},
            "bind": ["emb", "w:m", "zero", "y"], "dispatch": [6, "rows32"]},
           {"name": "ln", "kernel": "layernorm", "constants": {"N": N, "MODE": 2, "EPS": 1e-7},
            "bind": ["emb", "y", "w:w", "w:bias", "mask", "o"], "dispatch": ["rows", 1]}]
    plan = mini_plan(f16, L, B, N, ops, {"y": L * B * N, "o": L * B * N, "zero": np.zeros(N * 4, np.uint8)}, "o", N)
    out = run_plan(plan, {"w": w, "bias": bias, "m": Wm}, a, mask, L * B).reshape(L * B, N)
    y = a.astype(np.float64) @ Wm.astype(np.float64).T
    if f16:
        y = y.astype(np.float16).astype(np.float64)
    close(out[valid], ref(a.astype(np.float64) + y, 1e-7)[valid], 1e-2 if f16 else 2e-5, "mode 2")

    # embln: offset 2, 9 position rows, 3 types, POSIDS in the high bits
    P = 9
    pos = RNG.standard_normal((P, N)).astype(dt)
    typ = RNG.standard_normal((3, N)).astype(dt)
    for posids in (0, 1):
        tt = np.array([(i % 3) | ((((i * 5) % P) << 16) if posids else 0) for i in range(L * B)], dtype=np.uint32)
        op = {"name": "e", "kernel": "embln",
              "constants": {"N": N, "L": L, "OFFSET": 2, "MAXPOS": P, "EPS": 1e-5, "MASKMUL": 0, "POSIDS": posids},
              "bind": ["emb", "w:pos", "w:typ", "typeIds", "w:w", "w:bias", "mask", "o"], "dispatch": ["rows", 1]}
        plan = mini_plan(f16, L, B, N, [op], {"typeIds": L * B * (2 if f16 else 1), "o": L * B * N}, "o", N,
                         {"typeIds": "typeIds"})
        out = run_plan(plan, {"w": w, "bias": bias, "pos": pos, "typ": typ}, a, mask, L * B, tt).reshape(L * B, N)
        r = np.arange(L * B)
        prow = np.minimum((tt >> 16).astype(np.int64) if posids else (r % L) + 2, P - 1)
        v = a.astype(np.float64) + pos.astype(np.float64)[prow] + typ.astype(np.float64)[(tt & 0xFFFF).astype(np.int64)]
        close(out[valid], ref(v, 1e-5)[valid], 1e-2 if f16 else 2e-5, f"embln posids {posids}")


def attention_ref(qkv, lens, L, H, D, scale, window=0, rel=None):
    """f64 attention over packed sequences (tests/wasm_plan.test.ts:297-334 restated)."""
    hd = H * D
    out = np.zeros((L * len(lens), hd))
    q64 = qkv.astype(np.float64)
    for b, n in enumerate(lens):
        rows = q64[b * L:b * L + n]
        for h in range(H):
            q = rows[:, h * D:(h + 1) * D]
            k = rows[:, (H + h) * D:(H + h + 1) * D]
            v = rows[:, (2 * H + h) * D:(2 * H + h + 1) * D]
            s = q @ k.T
            if rel is not None:
                idx, pk, pq = rel
                i = np.arange(n)[:, None]
                j = np.arange(n)[None, :]
                p = idx[i * L + j]
                s = s + np.einsum("id,ijd->ij", q, pk[p][:, :, h * D:(h + 1) * D]) \
                      + np.einsum("jd,ijd->ij", k, pq[p][:, :, h * D:(h + 1) * D])
                s = s / scale
            else:
                s = s * scale
            if window:
                i = np.arange(n)[:, None]
                j = np.arange(n)[None, :]
                s = np.where(np.abs(i - j) <= window, s, -np.inf)
            s = s - s.max(1, keepdims=True)
            e = np.exp(s)
            pm = e / e.sum(1, keepdims=True)
            out[b * L:b * L + n, h * D:(h + 1) * D] = pm @ v
    return out


@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("D,lens,window,split", [(64, [5, 70], 0, True), (32, [128], 0, False), (64, [200, 3], 2, True),
                                                 (64, [300], 64, False), (32, [1, 65, 64], 0, True),
                                                 (50, [5, 70], 0, True), (20, [33, 1], 0, False),
                                                 (40, [150], 64, False)])
def test_standard_attention(f16, D, lens, window, split):
    """Head dimensions 32 and 64, and others (50 as polyBERT's, 20, 40) padded inside the kernel."""
    H = 3
    L = max(lens)
    L = ((L + 31) // 32) * 32
    B = len(lens)
    hd = H * D
    dt = np.float16 if f16 else np.float32
    qkv = (RNG.standard_normal((L * B, 3 * hd)) * 1.5).astype(dt)
    mask = prefix_mask(L, lens)
    scale = D ** -0.5
    base = {"L": L, "H": H, "D": D}
    if split:
        ops = [{"name": "s", "kernel": "attscore", "constants": {**base, "SCALE": scale, "ROWS": L * B},
                "bind": ["emb", "kinfo", "scores"], "dispatch": [H, "rows32"]},
               {"name": "p", "kernel": "attsoftmax", "constants": {"L": L, "H": H, "WINDOW": window},
                "bind": ["mask", "scores"], "dispatch": [H, "rows"]},
               {"name": "v", "kernel": "attpv", "constants": {**base, "ROWS": L * B},
                "bind": ["scores", "emb", "mask", "kinfo", "ctx"], "dispatch": [H, "rows32"]}]
        extra = {"kinfo": 2 * B * (2 if f16 else 1), "scores": L * B * H * L * (2 if f16 else 1), "ctx": L * B * hd}
    else:
        ops = [{"name": "a", "kernel": "mbflash", "constants": {**base, "SCALE": scale, "WINDOW": window, "ROWS": L * B},
                "bind": ["emb", "mask", "ctx"], "dispatch": [H, "rows32"]}]
        extra = {"ctx": L * B * hd}
    plan = mini_plan(f16, L, B, 3 * hd, ops, extra, "ctx", hd)
    out = run_plan(plan, {}, qkv, mask, L * B).reshape(L * B, hd)
    want = attention_ref(qkv, lens, L, H, D, scale, window)
    valid = mask > 0.5
    close(out[valid], want[valid], 1e-2 if f16 else 1e-5, f"attention D {D} window {window}")


@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("D,lens,split", [(64, [7], False), (64, [40, 129], True), (64, [200], False),
                                          (50, [90, 33], False), (50, [70], True)])
def test_relative_attention(f16, D, lens, split):
    H = 2
    L = 256
    B = len(lens)
    hd = H * D
    span, maxpos = 32, 64  # log buckets beyond |i - j| > 16
    dt = np.float16 if f16 else np.float32
    qkv = (RNG.standard_normal((L * B, 3 * hd))).astype(dt)
    pk = RNG.standard_normal((2 * span, hd)).astype(dt)
    pq = RNG.standard_normal((2 * span, hd)).astype(dt)
    idx = rel_pos_table(L, span, maxpos)
    mask = prefix_mask(L, lens)
    scale = math.sqrt(3 * D)
    moff = int(idx[L - 1])
    nm = int(idx[(L - 1) * L]) - moff + 1
    if split:
        relc = {"H": H, "D": D, "ROWS": L * B, "NM": nm, "MOFF": moff, "L": L}
        ops = [{"name": "c", "kernel": "attrel", "constants": {**relc, "PART": 0}, "bind": ["emb", "w:pk", "kinfo", "relidx", "c2p"], "dispatch": [1, "rows32"]},
               {"name": "p", "kernel": "attrel", "constants": {**relc, "PART": 1}, "bind": ["emb", "w:pq", "kinfo", "relidx", "p2c"], "dispatch": [1, "rows32"]},
               {"name": "s", "kernel": "attscore", "constants": {"L": L, "H": H, "D": D, "SCALE": 1 / scale, "ROWS": L * B}, "bind": ["emb", "kinfo", "scores"], "dispatch": [1, "rows32"]},
               {"name": "sr", "kernel": "attsoftrel", "constants": {"L": L, "H": H, "NM": nm, "MOFF": moff, "INVSCALE": 1 / scale}, "bind": ["mask", "relidx", "c2p", "p2c", "scores"], "dispatch": [H, "rows"]},
               {"name": "v", "kernel": "attpv", "constants": {"L": L, "H": H, "D": D, "ROWS": L * B}, "bind": ["scores", "emb", "mask", "kinfo", "ctx"], "dispatch": [1, "rows32"]}]
        extra = {"kinfo": 4 * B, "relidx": idx, "scores": 2 * L * B * H * L, "c2p": 2 * L * B * H * nm,
                 "p2c": 2 * L * B * H * nm, "ctx": L * B * hd}
    else:
        ops = [{"name": "a", "kernel": "attention", "constants": {"L": L, "H": H, "D": D, "SCALE": scale},
                "bind": ["emb", "w:pk", "w:pq", "relidx", "mask", "ctx"], "dispatch": [H, "rows"]}]
        extra = {"relidx": idx, "ctx": L * B * hd}
    plan = mini_plan(f16, L, B, 3 * hd, ops, extra, "ctx", hd)
    out = run_plan(plan, {"pk": pk, "pq": pq}, qkv, mask, L * B).reshape(L * B, hd)
    want = attention_ref(qkv, lens, L, H, D, scale, 0, (idx, pk.astype(np.float64), pq.astype(np.float64)))
    valid = mask > 0.5
    close(out[valid], want[valid], 1e-2 if f16 else 1e-5, f"relative attention {lens}")


def rel_attention_ref_rows(qkv, lens, L, H, D, scale, idx, pk, pq, chunk=64):
    """The relative attention of attention_ref, a block of query rows at a time (a 1280-row
    sequence's [n, n, D] position gathers would not fit in memory at once)."""
    hd = H * D
    out = np.zeros((L * len(lens), hd))
    q64 = qkv.astype(np.float64)
    for b, n in enumerate(lens):
        rows = q64[b * L:b * L + n]
        j = np.arange(n)
        for h in range(H):
            k = rows[:, (H + h) * D:(H + h + 1) * D]
            v = rows[:, (2 * H + h) * D:(2 * H + h + 1) * D]
            pkh, pqh = pk[:, h * D:(h + 1) * D], pq[:, h * D:(h + 1) * D]
            for i0 in range(0, n, chunk):
                i = np.arange(i0, min(n, i0 + chunk))
                q = rows[i, h * D:(h + 1) * D]
                p = idx[i[:, None] * L + j[None, :]]
                s = q @ k.T + (q @ pkh.T)[np.arange(len(i))[:, None], p] + (k @ pqh.T)[j[None, :], p]
                s = s / scale
                s = s - s.max(1, keepdims=True)
                e = np.exp(s)
                out[b * L + i, h * D:(h + 1) * D] = (e / e.sum(1, keepdims=True)) @ v
    return out


@pytest.mark.parametrize("f16", [False, True])
def test_relative_attention_long_plan(f16):
    """GLiNER-base length (L = 1280, the reference's tests/helpers/plan-trace.ts:50) with its
    bucket table (256 log buckets, max distance 512): one full sequence and one of 700 rows, the
    fused DeBERTa attention against float64."""
    H, D = 2, 64
    L, lens = 1280, [1280, 700]
    B = len(lens)
    hd = H * D
    span, maxpos = 256, 512
    dt = np.float16 if f16 else np.float32
    qkv = (RNG.standard_normal((L * B, 3 * hd)) * 0.5).astype(dt)
    pk = (RNG.standard_normal((2 * span, hd)) * 0.5).astype(dt)
    pq = (RNG.standard_normal((2 * span, hd)) * 0.5).astype(dt)
    idx = rel_pos_table(L, span, maxpos)
    mask = prefix_mask(L, lens)
    scale = math.sqrt(3 * D)
    ops = [{"name": "a", "kernel": "attention", "constants": {"L": L, "H": H, "D": D, "SCALE": scale},
            "bind": ["emb", "w:pk", "w:pq", "relidx", "mask", "ctx"], "dispatch": [H, "rows"]}]
    plan = mini_plan(f16, L, B, 3 * hd, ops, {"relidx": idx, "ctx": L * B * hd}, "ctx", hd)
    out = run_plan(plan, {"pk": pk, "pq": pq}, qkv, mask, L * B).reshape(L * B, hd)
    want = rel_attention_ref_rows(qkv, lens, L, H, D, scale, idx, pk.astype(np.float64), pq.astype(np.float64))
    valid = mask > 0.5
    close(out[valid], want[valid], 1e-2 if f16 else 1e-5, f"relative attention L {L}")


@pytest.mark.parametrize("f16", [False, True])
def test_add_geglu_rope_pool_gather(f16):
    L, lens = 7, [3, 7]
    B = len(lens)
    H, D = 2, 6
    N = 3 * H * D
    dt = np.float16 if f16 else np.float32
    x = RNG.standard_normal((L * B, N)).astype(dt)
    mask = prefix_mask(L, lens)
    valid = mask > 0.5
    tol = 1e-2 if f16 else 2e-5
    # rope on q and k (table [L][cos D | sin D])
    table = np.zeros((L, 2 * D), np.float32)
    for i in range(L):
        for d in range(D // 2):
            f = i * 10000 ** (-(2 * d) / D)
            table[i, d] = math.cos(f)
            table[i, D + d] = math.sin(f)
    # identity matmul copies emb into a writable buffer first
    eye = np.eye(N, dtype=dt)
    ops = [{"name": "cp", "kernel": "matmul", "constants": {"M": L * B, "N": N, "K": N, "ACT": 0},
            "bind": ["emb", "w:eye", "zero", "qkv"], "dispatch": [3, "rows16"]},
           {"name": "r", "kernel": "rope", "constants": {"L": L, "H": H, "D": D}, "bind": ["qkv", "cs"], "dispatch": ["rows", 2 * H]}]
    plan = mini_plan(f16, L, B, N, ops, {"qkv": L * B * N, "cs": table.reshape(-1), "zero": np.zeros(4 * N, np.uint8)}, "qkv", N)
    out = run_plan(plan, {"eye": eye}, x, mask, L * B).reshape(L * B, N)
    want = x.astype(np.float64).copy()
    for r in range(L * B):
        il = r % L
        for s in range(2 * H):
            for d in range(D // 2):
                a, b = x[r, s * D + d], x[r, s * D + d + D // 2]
                c, sn = table[il, d], table[il, D + d]
                want[r, s * D + d] = a * c - b * sn
                want[r, s * D + d + D // 2] = b * c + a * sn
    close(out[valid], want[valid], tol, "rope")
    # add MODE 0 and geglu
    I = N // 2
    ops = [{"name": "cp", "kernel": "matmul", "constants": {"M": L * B, "N": N, "K": N, "ACT": 0},
            "bind": ["emb", "w:eye", "zero", "y"], "dispatch": [3, "rows16"]},
           {"name": "a", "kernel": "add", "constants": {"TOTAL": L * B * N, "N": N, "MODE": 0, "L": L}, "bind": ["y", "emb"], "dispatch": [1, 1]},
           {"name": "g", "kernel": "geglu", "constants": {"I": I}, "bind": ["y", "gate"], "dispatch": ["rows", 1]}]
    plan = mini_plan(f16, L, B, N, ops, {"y": L * B * N, "gate": L * B * I, "zero": np.zeros(4 * N, np.uint8)}, "gate", I)
    out = run_plan(plan, {"eye": eye}, x, mask, L * B).reshape(L * B, I)
    y = 2 * x.astype(np.float64)
    if f16:
        y = y.astype(np.float16).astype(np.float64)
    want = gelu(y[:, :I]) * y[:, I:]
    close(out[valid], want[valid], tol, "add + geglu")
    # pool mean / max and CLS gather -> [B, N] rows
    for kind in ("mean", "max", "first"):
        if kind == "first":
            op = {"name": "g", "kernel": "gather", "constants": {"K": 1, "D": N, "L": L}, "bind": ["first", "emb", "st"], "dispatch": [1, 1]}
            extra = {"first": np.zeros(3 * B, np.uint32), "st": B * N}
        else:
            op = {"name": "p", "kernel": "pool", "constants": {"L": L, "N": N, "MODE": 0 if kind == "mean" else 1},
                  "bind": ["emb", "mask", "st"], "dispatch": [1, B]}
            extra = {"st": B * N}
        plan = mini_plan(f16, L, B, N, [op], extra, "st", N)
        plan["output"]["rows"] = B
        out = run_plan(plan, {}, x, mask, L * B).reshape(B, N)
        x64 = x.astype(np.float64)
        for b, n in enumerate(lens):
            seq = x64[b * L:b * L + n]
            want = seq.mean(0) if kind == "mean" else seq.max(0) if kind == "max" else seq[0]
            close(out[b], want, tol, f"pool {kind}")


def attention_ref_masked(qkv, mask, L, H, D, scale, window=0, rel=None):
    """f64 attention with the reference's general masking (src/wasm/plan.ts:573-582, 652-661):
    keys count where the mask exceeds 0.5, a query row whose mask does not is zero, every other
    query attends over the counted keys (and its window)."""
    hd = H * D
    B = len(mask) // L
    out = np.zeros((L * B, hd))
    q64 = qkv.astype(np.float64)
    for b in range(B):
        m = mask[b * L:(b + 1) * L]
        keys = np.nonzero(m > 0.5)[0]
        for i in np.nonzero(m > 0.5)[0]:
            row = q64[b * L + i]
            for h in range(H):
                q = row[h * D:(h + 1) * D]
                ks = keys if not window else keys[np.abs(keys - i) <= window]
                k = q64[b * L + ks][:, (H + h) * D:(H + h + 1) * D]
                v = q64[b * L + ks][:, (2 * H + h) * D:(2 * H + h + 1) * D]
                s = k @ q
                if rel is not None:
                    idx, pk, pq = rel
                    p = idx[i * L + ks]
                    s = (s + pk[p][:, h * D:(h + 1) * D] @ q + np.einsum("jd,jd->j", k, pq[p][:, h * D:(h + 1) * D])) / scale
                else:
                    s = s * scale
                e = np.exp(s - s.max())
                out[b * L + i, h * D:(h + 1) * D] = (e / e.sum()) @ v
    return out


def holed_mask(L, lens, seed):
    """Prefix masks with holes (0 inside), fractional values (0.7 counts as a key, 0.3 does not),
    a masked first row, and a trailing row of 0.4 past the last key."""
    rng = np.random.default_rng(seed)
    m = np.zeros(L * len(lens), dtype=np.float32)
    for b, n in enumerate(lens):
        v = np.ones(n, dtype=np.float32)
        if n > 8:
            for i in rng.choice(np.arange(1, n - 1), size=max(1, n // 8), replace=False):
                v[i] = rng.choice([0.0, 0.7, 0.3])
        if b == 1:
            v[0] = 0.0
        m[b * L:b * L + n] = v
        if n < L:
            m[b * L + n] = 0.4
    return m


@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("kind", ["standard", "window", "relative"])
def test_attention_with_general_masks(f16, kind):
    """Masks with holes and fractional values: the kernels' key test and zeroed query rows
    against the reference's rule in f64."""
    H, D = 2, 64
    lens = [150, 70, 9]
    L = 160
    B = len(lens)
    hd = H * D
    dt = np.float16 if f16 else np.float32
    qkv = RNG.standard_normal((L * B, 3 * hd)).astype(dt)
    mask = holed_mask(L, lens, 3)
    window = 16 if kind == "window" else 0
    rel = None
    weights = {}
    if kind == "relative":
        span, maxpos = 32, 64
        pk = RNG.standard_normal((2 * span, hd)).astype(dt)
        pq = RNG.standard_normal((2 * span, hd)).astype(dt)
        idx = rel_pos_table(L, span, maxpos)
        scale = math.sqrt(3 * D)
        ops = [{"name": "a", "kernel": "attention", "constants": {"L": L, "H": H, "D": D, "SCALE": scale},
                "bind": ["emb", "w:pk", "w:pq", "relidx", "mask", "ctx"], "dispatch": [H, "rows"]}]
        extra = {"relidx": idx, "ctx": L * B * hd}
        weights = {"pk": pk, "pq": pq}
        rel = (idx, pk.astype(np.float64), pq.astype(np.float64))
    else:
        scale = D ** -0.5
        ops = [{"name": "a", "kernel": "mbflash", "constants": {"L": L, "H": H, "D": D, "SCALE": scale,
                                                               "WINDOW": window, "ROWS": L * B},
                "bind": ["emb", "mask", "ctx"], "dispatch": [H, "rows32"]}]
        extra = {"ctx": L * B * hd}
    plan = mini_plan(f16, L, B, 3 * hd, ops, extra, "ctx", hd)
    out = run_plan(plan, weights, qkv, mask, L * B).reshape(L * B, hd)
    want = attention_ref_masked(qkv, mask, L, H, D, scale, window, rel)
    keep = mask > 0.5
    close(out[keep], want[keep], 1e-2 if f16 else 1e-5, f"{kind} attention, general masks")
    masked_rows = (mask != 0) & ~keep  # computed rows whose mask does not count them: zeros
    assert np.all(out[masked_rows] == 0)
