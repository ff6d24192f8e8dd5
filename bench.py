"""Throughput of the encoder hot path on one MI355X: sequences/s and tokens/s of a ragged batch.

A step is one forward of the whole batch plan (embedding + LayerNorm, 12 post-LN layers, CLS head)
over inputs already resident in HBM. The default workload is BASELINE.json's headline config
(RoBERTa-base shape, f16 storage / f32 accumulate, 256 sequences with lognormal lengths, median
45, packed without padding); --workload picks another benchmark config.

The timed steps run as the library runs them: a batch with fewer than 400,000 valid rows goes as two
halves on two streams (`streams` in the line). After them the bench times, per launch, the same
steps with the whole batch on one stream and a HIP event pair around every launch on that stream
(kh_trace): events around each launch would serialise the two streams, so the split run cannot be
timed per launch without changing it. That pass gives the dominant kernel's roofline, for the
kernels at the workload's full size (`roofline.mode`). The bench also times the CPU oracle (f32
restatement of the reference's WASM executor) on a bounded sample of the same batch.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK = {"f16_mfma_tflops": 2500.0, "f32_mfma_tflops": 157.3, "hbm_gbs": 8000.0}

# HBM bytes per launch of a workload's dominant kernel family, from two rocprofv3 --pmc runs of this
# bench (FETCH_SIZE, then WRITE_SIZE; KiB per dispatch averaged over the family), each counter scaled
# by what it reads for a plain device copy of 1 GiB (python3 -m kleinhirn_amd.profiling copy 1024:
# FETCH_SIZE reads 0.5 GiB -> x2.0, WRITE_SIZE reads 1.0 GiB -> x1.0). Summaries with the commands:
# profiles/gemm_mfma_c2_roberta_base_ragged256_traffic.md, gemm_mfma_c5_xlmr_minilm_l12_pairs4096_traffic.md and
# layernorm_c4_modernbert_small_b64_traffic.md.
# Re-measured whenever the kernel changes (an entry whose source digest differs is not reported).
FETCH_SCALE, WRITE_SCALE = 2.0, 1.0
TRAFFIC_KIB = {  # (workload, family): (FETCH_SIZE KiB, WRITE_SIZE KiB) per dispatch, kernel source sha256[:16]
    ("c2-roberta-base-f16-ragged256", "gemm_mfma"): (50725.5, 40025.3, "eff3a2d673240c43"),
    ("c5-xlmr-minilm-l12-f16-pairs4096", "gemm_mfma"): (1104903.2, 1894393.1, "eff3a2d673240c43"),
    ("c4-modernbert-small-f16-b64", "layernorm"): (93671.2, 187261.4, "4da9f9850653c494"),
}
# the source file of each kernel family (a counter figure measured on other code is not reported)
FAMILY_SOURCE = {"gemm_mfma": "gemm.hip", "attention": "attention.hip", "layernorm": "rowops.hip",
                 "embln": "rowops.hip"}


def source_digest(family: str) -> str | None:
    import hashlib
    f = FAMILY_SOURCE.get(family)
    if not f:
        return None
    with open(os.path.join(ROOT, "kleinhirn_amd", "csrc", f), "rb") as fh:
        return hashlib.sha256(fh.read()).hexdigest()[:16]


def physical_cores(cpus) -> int:
    """Distinct (package, core) pairs among the CPUs this process may run on."""
    seen, cur = set(), {}
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh.read().split("\n") + [""]:
                if not line.strip():
                    if cur.get("processor") in cpus:
                        seen.add((cur.get("physical id"), cur.get("core id")))
                    cur = {}
                    continue
                k, _, v = line.partition(":")
                k, v = k.strip(), v.strip()
                cur[k] = int(v) if k == "processor" else v
    except OSError:
        return len(cpus)
    return len(seen) or len(cpus)


def run_facts() -> dict:
    """BASELINE.md section 7's record fields: commit, ROCm version, device name and clock."""
    import ctypes
    facts = {}
    try:
        with open(os.path.join(ROOT, "kleinhirn_amd", "build_info.json")) as fh:
            facts.update(json.load(fh))
    except (OSError, ValueError):
        facts["commit"] = None
    try:
        with open("/opt/rocm/.info/version") as fh:
            facts["rocm"] = fh.read().strip()
    except OSError:
        facts["rocm"] = None
    try:
        import torch
        props = torch.cuda.get_device_properties(0)
        facts["device"] = f"{props.name} ({getattr(props, 'gcnArchName', '?')}, {props.multi_processor_count} CUs)"
        hip = ctypes.CDLL("libamdhip64.so")
        v = ctypes.c_int(0)
        if hip.hipDeviceGetAttribute(ctypes.byref(v), 5, 0) == 0:  # hipDeviceAttributeClockRate (kHz, peak)
            facts["clock_mhz"] = v.value // 1000
    except Exception:
        pass
    return facts


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def cpu_baseline(w, weights, seconds: float = 12.0, threads: int | None = None) -> tuple[dict, np.ndarray]:
    """The oracle on the host cores, the reference's WASM schedule (one sequence at a time on the
    bucket plan, real rows only), over as many sequences of the batch as fit ~`seconds`; threads
    default to min(cores, 8), the reference's 'auto' (src/wasm-plan-host.ts:35-49). Returns the
    figure and the oracle's outputs for the sequences it ran (the parity check's reference)."""
    from kleinhirn_amd import inputs
    from kleinhirn_amd.plan.build import build_plan
    from oracle.oracle import OracleRuntime
    cpus = sorted(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else list(range(os.cpu_count() or 1))
    phys = physical_cores(set(cpus))
    threads = threads or max(1, min(len(cpus), 8))
    plan = build_plan(w.spec, w.head, w.length, 1, False)
    rt = OracleRuntime(weights, [plan])
    p = rt.plan(plan, threads=threads)
    table = weights["embeddings.word.weight"]
    ids = w.ids()
    done = toks = 0
    outs = []
    t0 = time.perf_counter()
    for seq in ids:
        ri = inputs.run_input(w.spec, table, [seq], w.length)
        p.upload(ri["embeddings"], ri["mask"], ri["typeIds"])
        p.run(len(seq))
        outs.append(p.read_output())
        done += 1
        toks += len(seq)
        if time.perf_counter() - t0 > seconds:
            break
    dt = time.perf_counter() - t0
    fig = {"value": round(done / dt, 3), "unit": "sequences/s", "cores": threads, "kind": "port",
           "tokens_per_s": round(toks / dt, 1),
           "sample": f"first {done} of {len(ids)} sequences ({toks} tokens), one B=1 bucket plan "
                     f"(L={w.length}) per sequence, f32, {threads} OpenMP threads; the process may run on "
                     f"{len(cpus)} CPUs ({phys} physical cores)"}
    return fig, np.stack(outs)


def parity(ref: np.ndarray, got: np.ndarray, embedding: bool) -> dict:
    """The reference's whole-run gate (bench/kbench/runner-lib.mjs:171-195,
    convert/k28_close_calls.py:1-8): largest logit deviation, decisions that agree, decisions
    excluded because their f32 top-2 gap is under twice that deviation, exact argmax identity, and
    the smallest row cosine."""
    ref = ref.astype(np.float64)
    got = got.astype(np.float64)
    delta = float(np.abs(ref - got).max())
    cos = (ref * got).sum(1) / np.maximum(np.linalg.norm(ref, axis=1) * np.linalg.norm(got, axis=1), 1e-30)
    out = {"n": int(len(ref)), "max_dlogit": round(delta, 6), "min_cosine": round(float(cos.min()), 6)}
    if ref.shape[1] > 1 and not embedding:
        top2 = np.sort(ref, axis=1)[:, -2:]
        flippable = (top2[:, 1] - top2[:, 0]) < 2 * delta
        same = ref.argmax(1) == got.argmax(1)
        out.update(agree=int((same | flippable).sum()), excluded=int(flippable.sum()),
                   identical=int(same.sum()), mismatched=int((~same & ~flippable).sum()))
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="c2", choices=["c1", "c2", "c3a", "c3b", "c4", "c5"])
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--ids", action="store_true", help="device word gather (token ids) instead of host rows")
    ap.add_argument("--no-trace", action="store_true",
                    help="time the steps without per-launch events (no roofline; checks the events' cost)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build runs the path on a single MI355X (no sharding, "
              f"no collectives); --gpus {args.gpus} is not supported", file=sys.stderr)
        return 2

    import torch  # device plumbing only: the hot path is libkh_hip.so
    from kleinhirn_amd import configs, inputs, synth
    from kleinhirn_amd.backend import HipBackend
    from kleinhirn_amd.plan.build import build_plan

    assert torch.cuda.is_available(), "bench needs the GPU"
    w = configs.ALL[args.workload]()
    f16 = w.f16
    t0 = time.perf_counter()
    weights = configs.make_weights(w.spec, w.head)
    W = configs.storage(weights, f16)
    log(f"weights {time.perf_counter() - t0:.1f}s")
    be = HipBackend(W)
    plan = build_plan(w.spec, w.head, w.length, w.batch, f16)
    be.check(plan)
    r = be.runner(plan)
    ids = w.ids()
    rows = w.length * w.batch
    if args.ids:
        be.set_words(W["embeddings.word.weight"])
        mask, tt = inputs.mask_and_types(w.spec, ids, w.length)
        flat = np.zeros(rows, dtype=np.int32)
        for b, seq in enumerate(ids):
            flat[b * w.length:b * w.length + len(seq)] = seq
        r.upload_ids(flat, mask, tt)
    else:
        run_input = inputs.run_input(w.spec, W["embeddings.word.weight"], ids, w.length)
        r.upload(run_input)
    # boundary time of the first call: packing + H2D of the valid rows + forward + readback
    t0 = time.perf_counter()
    r.run(rows)
    out = r.read_output()
    boundary_ms = (time.perf_counter() - t0) * 1e3
    assert np.isfinite(out).all()
    out = out.reshape(w.batch, -1)
    T = r.packed_rows()
    for _ in range(args.warmup):
        r.run(rows)
    r.sync()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        r.run(rows)
    r.sync()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / max(1, args.steps)
    streams = int(r.info.streams)
    seq_s = w.batch / dt
    tok_s = T / dt
    # steady-state boundary: host RunInput -> upload -> run -> host f32 output, one call after the other
    bts = []
    for _ in range(max(3, min(10, args.steps))):
        t0 = time.perf_counter()
        if args.ids:
            r.upload_ids(flat, mask, tt)
        else:
            r.upload(run_input)
        r.run(rows)
        r.read_output()
        bts.append(time.perf_counter() - t0)
    bts.sort()
    bdt = bts[len(bts) // 2]
    if args.no_trace:
        print(json.dumps({"metric": "sequences/sec", "value": round(seq_s, 1), "ms_per_step": round(dt * 1e3, 4),
                          "streams": streams}), flush=True)
        return 0

    # per-launch pass: the same steps, the whole batch on one stream, an event pair around each launch
    saved = os.environ.get("KH_NO_SPLIT")
    os.environ["KH_NO_SPLIT"] = "1"
    r.run(rows)
    r.sync()
    r.trace(True)
    for _ in range(args.steps):
        r.run(rows)
    prof = r.trace_read()
    r.trace(False)
    if saved is None:
        os.environ.pop("KH_NO_SPLIT")
    else:
        os.environ["KH_NO_SPLIT"] = saved

    # the timed steps' launches by kernel family, and the dominant kernel's roofline
    by_kernel: dict[str, dict] = {}
    for p in prof:
        k = by_kernel.setdefault(p["kernel"], {"ms": 0.0, "flops": 0.0, "bytes": 0.0, "launches": 0})
        k["ms"] += p["ms"]
        k["flops"] += p["flops"]
        k["bytes"] += p["bytes"]
        k["launches"] += 1
    total_ms = sum(k["ms"] for k in by_kernel.values()) / max(1, args.steps)  # per step
    for k in by_kernel.values():
        k["ms"] /= max(1, args.steps)
        k["flops"] /= max(1, args.steps)
        k["bytes"] /= max(1, args.steps)
        k["launches"] = int(round(k["launches"] / max(1, args.steps)))
    for name, k in sorted(by_kernel.items(), key=lambda kv: -kv[1]["ms"]):
        tf = k["flops"] / (k["ms"] * 1e-3) / 1e12 if k["ms"] else 0
        gb = k["bytes"] / (k["ms"] * 1e-3) / 1e9 if k["ms"] else 0
        log(f"  {name:16s} {k['launches']:4d} launches {k['ms']:8.3f} ms ({100 * k['ms'] / total_ms:5.1f} %) "
            f"{tf:8.1f} TFLOP/s {gb:8.1f} GB/s")
    dom_name, dom = max(by_kernel.items(), key=lambda kv: kv[1]["ms"])
    # MFMA-bound: the tile GEMMs and attention; the wavefront-per-output dot products read memory
    mfma = dom_name != "gemm_rowdot" and (dom_name.startswith("gemm") or dom_name.startswith("attention"))
    avg_ms = dom["ms"] / dom["launches"]
    if mfma:
        achieved = dom["flops"] / dom["launches"] / (avg_ms * 1e-3) / 1e12
        peak = PEAK["f16_mfma_tflops"] if f16 else PEAK["f32_mfma_tflops"]
        roof = {"bound": "mfma", "achieved": round(achieved, 1), "peak": peak, "unit": "TFLOP/s"}
    else:
        achieved = dom["bytes"] / dom["launches"] / (avg_ms * 1e-3) / 1e9
        roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK["hbm_gbs"], "unit": "GB/s"}
    roof["frac"] = round(roof["achieved"] / roof["peak"], 4)
    kib = TRAFFIC_KIB.get((w.name, dom_name))
    # a counter figure holds only for the kernel source it was measured on
    current = kib is not None and kib[2] == source_digest(dom_name)
    roof["traffic"] = round((kib[0] * FETCH_SCALE + kib[1] * WRITE_SCALE) * 1024) if current else None
    roof["traffic_unit"] = "bytes/launch (rocprofv3 --pmc FETCH_SIZE + WRITE_SIZE, copy-calibrated)"
    if kib is not None and not current:
        roof["traffic_note"] = "counters measured on another revision of the kernel source: not reported"
    roof["algorithmic_bytes"] = round(dom["bytes"] / dom["launches"])
    roof["kernel"] = dom_name
    roof["avg_launch_ms"] = round(avg_ms, 4)
    roof["launches"] = int(round(dom["launches"]))  # per step
    roof["mode"] = "per launch: the timed steps re-run with the whole batch on one stream, HIP events around each launch"

    cpu = cpu_all = None
    checks = []
    embedding = w.head.get("type") == "embed"
    if not args.no_cpu:
        cpu, ref = cpu_baseline(w, weights, args.cpu_seconds)
        checks.append(dict(parity(ref, out[:len(ref)], embedding), reference="oracle on this host, the CPU sample"))
        cpus = sorted(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else [0]
        allc = physical_cores(set(cpus))
        if allc != cpu["cores"]:
            cpu_all, _ = cpu_baseline(w, weights, args.cpu_seconds, threads=allc)
    # the whole batch against the committed oracle outputs of the same seeded batch
    gold = os.path.join(ROOT, "tests", "golden", f"oracle_{args.workload}_full.npz")
    if os.path.exists(gold):
        import hashlib
        g = np.load(gold)
        n = len(g["out"])
        ids_ok = hashlib.sha256(np.concatenate(ids[:n]).astype(np.int32).tobytes()).hexdigest() == str(g["ids_sha256"])
        if ids_ok and np.array_equal(np.array([len(x) for x in ids[:n]]), g["lengths"]):
            checks.append(dict(parity(g["out"], out[:n], embedding),
                               reference="committed oracle outputs (tests/golden) of the same sequences"))

    line = {
        "metric": "sequences/sec + tokens/sec, BERT-base f16 ragged batch; % MFMA / HBM peak",
        "value": round(seq_s, 1), "unit": "sequences/s", "tokens_per_s": round(tok_s, 1),
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(dt * 1e3, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f16" if f16 else "f32", "data": "synthetic (seeded LCG ids and N(0,0.02) weights)",
        "config": {"workload": w.name, "global_batch": w.batch, "tokens": T, "bucket_length": w.length,
                   "layers": w.spec["layers"], "hidden": w.spec["hidden"], "packed": True,
                   "word_rows": "device gather" if args.ids else "host gather, uploaded once"},
        "roofline": roof,
        "cpu_baseline": cpu,
        "cpu_baseline_all_cores": cpu_all,
        "parity": checks,
        "gpu_kernel_ms": round(total_ms, 4), "streams": streams,
        "first_call_boundary_ms": round(boundary_ms, 2),
        "boundary": {"value": round(w.batch / bdt, 1), "unit": "sequences/s", "ms_per_call": round(bdt * 1e3, 3),
                     "mode": "host RunInput -> kh_upload -> kh_run -> kh_read_output (f32), calls back to back, "
                             "median"},
        "seed": synth.SEED,
        **run_facts(),
    }
    print(json.dumps(line), flush=True)
    r.destroy()
    be.dispose()
    return 0


if __name__ == "__main__":
    sys.exit(main())
