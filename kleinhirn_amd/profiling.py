"""rocprofv3 output -> short text summaries, grouped into the kernel families libkh_hip.so's own
per-launch profile (kh_profile) reports, so a kernel trace can be checked against bench.py's
HIP-event timings and PMC byte counters can be set against a launch's algorithmic bytes.

    python3 -m kleinhirn_amd.profiling copy <MiB>            plain device copy (counter calibration)
    python3 -m kleinhirn_amd.profiling trace <rocprof dir>   kernel-trace summary by family and by kernel (markdown)
    python3 -m kleinhirn_amd.profiling pmc <rocprof dir> ... counter sums per family (markdown)
    python3 -m kleinhirn_amd.profiling clock <rocprof dir>   shader clock per kernel of a --pmc GRBM_COUNT run (markdown)

The copy mode is the calibration workload: FETCH_SIZE and WRITE_SIZE of one copy of N bytes should
read N bytes each; the ratio is the scale applied to the same counters of the encoder's kernels.
"""
from __future__ import annotations

import collections
import csv
import glob
import os
import re
import sqlite3
import sys

# mangled kernel name fragment -> kh_profile family
FAMILIES = [
    ("gemm_lean_kernel", "gemm_mfma"),
    ("gemm_dma_kernel", "gemm_mfma"),
    ("gemm_persist_kernel", "gemm_mfma"),
    ("gemm_reg_kernel", "gemm_mfma"),
    ("gemm_small_f32_kernel", "gemm_mfma"),
    ("gemm_rowdot_kernel", "gemm_rowdot"),
    ("attn_kernel", "attention"),
    ("embln_kernel", "embln"),
    ("layernorm_kernel", "layernorm"),
    ("layernorm_rows_kernel", "layernorm"),
    ("add_vec_kernel", "add"),
    ("add_kernel", "add"),
    ("geglu_kernel", "geglu"),
    ("rope_kernel", "rope"),
    ("pool_kernel", "pool"),
    ("gather_kernel", "gather"),
    ("first_rows_kernel", "compact"),
    ("prefetch_kernel", "prefetch"),
    ("to_f32_kernel", "to_f32"),
    ("elementwise_kernel", "probe_copy"),
    ("copyBuffer", "runtime_copy"),
    ("fillBuffer", "runtime_fill"),
]


def family(name: str) -> str:
    for frag, fam in FAMILIES:
        if frag in name:
            return fam
    return "other:" + name[:40]


def _csv_rows(d: str, suffix: str) -> list[dict]:
    files = sorted(glob.glob(os.path.join(d, "**", f"*{suffix}"), recursive=True))
    if not files:
        raise FileNotFoundError(f"no *{suffix} under {d}")
    rows = []
    for f in files:
        with open(f, newline="") as fh:
            rows.extend(csv.DictReader(fh))
    return rows


def kernel_durations(d: str) -> list[tuple[str, float]]:
    """(kernel name, duration ns) per dispatch from a --kernel-trace run (csv or rocpd database)."""
    dbs = sorted(glob.glob(os.path.join(d, "**", "*.db"), recursive=True))
    if dbs:
        out = []
        for db in dbs:
            c = sqlite3.connect(db)
            out.extend((n, float(t)) for n, t in c.execute("select name, duration from kernels"))
        return out
    return [(r["Kernel_Name"], float(r["End_Timestamp"]) - float(r["Start_Timestamp"]))
            for r in _csv_rows(d, "kernel_trace.csv")]


def trace_summary(d: str) -> str:
    per = collections.defaultdict(list)
    names = collections.defaultdict(set)
    for name, ns in kernel_durations(d):
        fam = family(name)
        per[fam].append(ns)
        names[fam].add(name)
    total = sum(sum(v) for v in per.values())
    lines = ["| family | launches | avg us | total ms | % | kernels |", "|---|---|---|---|---|---|"]
    for fam, v in sorted(per.items(), key=lambda kv: -sum(kv[1])):
        lines.append(f"| {fam} | {len(v)} | {sum(v) / len(v) / 1e3:.2f} | {sum(v) / 1e6:.3f} | "
                     f"{100 * sum(v) / total:.1f} | {len(names[fam])} |")
    return "\n".join(lines)


def short_name(name: str) -> str:
    """Demangled-looking kernel name without namespaces and argument lists."""
    n = re.sub(r"kh::(\(anonymous namespace\)::)?", "", name)
    n = re.sub(r"\([^()]*\)$", "", n.strip())
    return n.replace("void ", "").strip()[:90]


def kernel_table(d: str, top: int = 16) -> str:
    """The `top` kernels (template instance and grid) by total time of a --kernel-trace run."""
    per = collections.defaultdict(list)
    for name, grid, ns in kernel_grids(d):
        per[(short_name(name), grid)].append(ns)
    total = sum(sum(v) for v in per.values())
    lines = ["| kernel | grid (work-items) | launches | avg us | total ms | % |", "|---|---|---|---|---|---|"]
    for (name, grid), v in sorted(per.items(), key=lambda kv: -sum(kv[1]))[:top]:
        lines.append(f"| {name} | {grid} | {len(v)} | {sum(v) / len(v) / 1e3:.2f} | {sum(v) / 1e6:.3f} | "
                     f"{100 * sum(v) / total:.1f} |")
    return "\n".join(lines)


def kernel_grids(d: str) -> list[tuple[str, str, float]]:
    return [(r["Kernel_Name"], "x".join(r.get(f"Grid_Size_{a}", "?") for a in "XYZ").replace("x1x1", ""),
             float(r["End_Timestamp"]) - float(r["Start_Timestamp"]))
            for r in _csv_rows(d, "kernel_trace.csv")]


def pmc_sums(d: str) -> dict[str, dict[str, float]]:
    """family -> {counter: summed value, 'dispatches': n} from a --pmc run (csv output)."""
    acc: dict = collections.defaultdict(lambda: collections.defaultdict(float))
    seen = collections.defaultdict(set)
    for r in _csv_rows(d, "counter_collection.csv"):
        fam = family(r["Kernel_Name"])
        acc[fam][r["Counter_Name"]] += float(r["Counter_Value"])
        seen[fam].add(r.get("Dispatch_Id") or r.get("Correlation_Id"))
    for fam in acc:
        acc[fam]["dispatches"] = len(seen[fam])
    return acc


def pmc_summary(dirs: list[str]) -> str:
    merged: dict = collections.defaultdict(dict)
    for d in dirs:
        for fam, c in pmc_sums(d).items():
            merged[fam].update(c)
    counters = sorted({k for c in merged.values() for k in c if k != "dispatches"})
    lines = ["| family | dispatches | " + " | ".join(f"{k} KiB/dispatch" for k in counters) + " |",
             "|---|---|" + "---|" * len(counters)]
    for fam, c in sorted(merged.items(), key=lambda kv: -sum(v for k, v in kv[1].items() if k != "dispatches")):
        n = max(1, int(c.get("dispatches", 1)))
        lines.append(f"| {fam} | {n} | " + " | ".join(f"{c.get(k, 0) / n:.1f}" for k in counters) + " |")
    return "\n".join(lines)


def clock_table(d: str, xcds: int = 8, top: int = 12) -> str:
    """Shader clock per kernel (template instance and grid) from a `--pmc GRBM_COUNT` run. The
    counter sums the GPU clock over the XCDs for the dispatch's sampling window, which is longer
    than the kernel's timestamps by a fixed amount; the window of the runtime's 2 us copy kernels
    (median) estimates it. GHz = (count - that) / duration / XCDs: a kernel's average clock while it
    ran, meaningful where the kernel is long against the correction (median over its dispatches)."""
    rows = [r for r in _csv_rows(d, "counter_collection.csv") if r["Counter_Name"] == "GRBM_COUNT"]
    base = sorted(float(r["Counter_Value"]) for r in rows if "copyBuffer" in r["Kernel_Name"])
    fixed = base[len(base) // 2] if base else 0.0
    per = collections.defaultdict(list)
    for r in rows:
        ns = float(r["End_Timestamp"]) - float(r["Start_Timestamp"])
        if ns <= 0 or "rocclr" in r["Kernel_Name"]:
            continue
        grid = r.get("Grid_Size") or "x".join(r.get(f"Grid_Size_{a}", "?") for a in "XYZ")
        per[(short_name(r["Kernel_Name"]), grid)].append((ns, (float(r["Counter_Value"]) - fixed) / ns / xcds))
    lines = [f"window correction: {fixed:.0f} counts (median of the runtime copy kernels)", "",
             "| kernel | grid (work-items) | dispatches | median us | median GHz |", "|---|---|---|---|---|"]
    for (name, grid), v in sorted(per.items(), key=lambda kv: -sum(x[0] for x in kv[1]))[:top]:
        ns = sorted(x[0] for x in v)[len(v) // 2]
        ghz = sorted(x[1] for x in v)[len(v) // 2]
        lines.append(f"| {name} | {grid} | {len(v)} | {ns / 1e3:.1f} | {ghz:.2f} |")
    return "\n".join(lines)


def copy_probe(mib: int, reps: int = 3) -> None:
    import torch
    n = mib << 20
    # uninitialised on purpose: a fill would be a second elementwise kernel in the counters
    src = torch.empty(n // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(reps):
        torch.neg(src, out=dst)  # one elementwise kernel: reads n bytes, writes n bytes
    torch.cuda.synchronize()
    print(f"copied {reps} x {n} bytes", flush=True)


def main(argv: list[str]) -> int:
    if len(argv) >= 2 and argv[0] == "copy":
        copy_probe(int(argv[1]))
    elif len(argv) >= 2 and argv[0] == "trace":
        print(trace_summary(argv[1]))
        print()
        print(kernel_table(argv[1]))
    elif len(argv) >= 2 and argv[0] == "pmc":
        print(pmc_summary(argv[1:]))
    elif len(argv) >= 2 and argv[0] == "clock":
        print(clock_table(argv[1]))
    else:
        print(__doc__, file=sys.stderr)
        return 2
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
