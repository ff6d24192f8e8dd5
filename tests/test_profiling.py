"""The rocprofv3 summaries of kleinhirn_amd.profiling on small synthetic csv outputs: family grouping
of a kernel trace, counter sums per dispatch, and the GRBM_COUNT clock with its window correction."""
from __future__ import annotations

import csv
import os

from kleinhirn_amd import profiling as P

TRACE_COLS = ["Kernel_Name", "Start_Timestamp", "End_Timestamp", "Grid_Size_X", "Grid_Size_Y", "Grid_Size_Z"]
PMC_COLS = ["Dispatch_Id", "Kernel_Name", "Grid_Size", "Counter_Name", "Counter_Value", "Start_Timestamp",
            "End_Timestamp"]


def _write(d, name, cols, rows):
    os.makedirs(d, exist_ok=True)
    with open(os.path.join(d, name), "w", newline="") as fh:
        w = csv.DictWriter(fh, fieldnames=cols)
        w.writeheader()
        for r in rows:
            w.writerow(r)


def test_trace_summary_groups_kernels_into_families(tmp_path):
    rows = [
        {"Kernel_Name": "void kh::gemm_lean_kernel<192, 128, 2, 2, 0, 0, 2>(kh::GemmArgs, int, int)",
         "Start_Timestamp": 0, "End_Timestamp": 3000, "Grid_Size_X": 256, "Grid_Size_Y": 1, "Grid_Size_Z": 1},
        {"Kernel_Name": "void kh::gemm_lean_kernel<192, 128, 2, 2, 0, 0, 2>(kh::GemmArgs, int, int)",
         "Start_Timestamp": 5000, "End_Timestamp": 6000, "Grid_Size_X": 256, "Grid_Size_Y": 1, "Grid_Size_Z": 1},
        {"Kernel_Name": "_ZN2kh12_GLOBAL__N_121layernorm_rows_kernelIDF16_Li32ELi3EE",
         "Start_Timestamp": 7000, "End_Timestamp": 8000, "Grid_Size_X": 64, "Grid_Size_Y": 1, "Grid_Size_Z": 1},
    ]
    d = str(tmp_path / "t")
    _write(d, "x_kernel_trace.csv", TRACE_COLS, rows)
    s = P.trace_summary(d)
    lines = s.splitlines()
    # gemm: 2 launches, 2 us average, 4 of the 5 us
    assert lines[2] == "| gemm_mfma | 2 | 2.00 | 0.004 | 80.0 | 1 |", lines[2]
    assert lines[3] == "| layernorm | 1 | 1.00 | 0.001 | 20.0 | 1 |", lines[3]


def test_pmc_summary_averages_per_dispatch(tmp_path):
    rows = []
    for i, v in enumerate([100.0, 300.0]):
        rows.append({"Dispatch_Id": i, "Kernel_Name": "gemm_lean_kernel<64, 64>", "Grid_Size": 64,
                     "Counter_Name": "FETCH_SIZE", "Counter_Value": v, "Start_Timestamp": 0, "End_Timestamp": 1})
    d = str(tmp_path / "p")
    _write(d, "x_counter_collection.csv", PMC_COLS, rows)
    s = P.pmc_summary([d]).splitlines()
    assert s[2] == "| gemm_mfma | 2 | 200.0 |", s[2]


def test_clock_table_subtracts_the_window_of_the_copy_kernels(tmp_path):
    # window: 8000 counts; a 1 ms kernel that counted 8000 + 8 XCDs x 2.0 GHz x 1e6 ns
    rows = [{"Dispatch_Id": 0, "Kernel_Name": "__amd_rocclr_copyBuffer", "Grid_Size": 512, "Counter_Name": "GRBM_COUNT",
             "Counter_Value": 8000.0, "Start_Timestamp": 0, "End_Timestamp": 2000}]
    for i in range(3):
        rows.append({"Dispatch_Id": i + 1, "Kernel_Name": "void kh::gemm_lean_kernel<256, 256, 2, 4, 0, 0, 2>()",
                     "Grid_Size": 4096, "Counter_Name": "GRBM_COUNT", "Counter_Value": 8000.0 + 8 * 2.0 * 1e6,
                     "Start_Timestamp": 10_000_000 * i, "End_Timestamp": 10_000_000 * i + 1_000_000})
    d = str(tmp_path / "c")
    _write(d, "x_counter_collection.csv", PMC_COLS, rows)
    s = P.clock_table(d).splitlines()
    assert s[0].startswith("window correction: 8000 counts")
    row = [l for l in s if "gemm_lean_kernel" in l][0]
    assert row.endswith("| 3 | 1000.0 | 2.00 |"), row
