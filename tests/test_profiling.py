"""The rocprofv3 summaries (moe_dispatch/profiling.py) on small synthetic CSVs."""

import csv

from moe_dispatch import profiling


def _write(path, header, rows):
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(header)
        w.writerows(rows)


def test_counter_runs_split_at_other_kernels_and_normalise(tmp_path):
    header = ["Dispatch_Id", "Kernel_Name", "Start_Timestamp", "End_Timestamp", "Counter_Name", "Counter_Value"]
    rows = []
    # Two runs of kernel A (two launches, then one) with kernel B between them.
    for d, (name, us) in enumerate([("A", 10), ("A", 10), ("B", 1), ("A", 20)]):
        cycles = us * 1000 * 2  # 2 GHz per XCD
        rows += [[d, name, 0, us * 1000, "GRBM_GUI_ACTIVE", cycles * profiling.XCDS],
                 [d, name, 0, us * 1000, "SQ_VALU_MFMA_BUSY_CYCLES", cycles * profiling.SIMDS // 2],
                 [d, name, 0, us * 1000, "SQ_WAIT_ANY", cycles * profiling.SIMDS // 4 // 10],
                 [d, name, 0, us * 1000, "TCP_TCC_READ_REQ_sum", 100],
                 [d, name, 0, us * 1000, "TCP_TCC_READ_REQ_LATENCY_sum", 35000]]
    path = tmp_path / "run_counter_collection.csv"
    _write(path, header, rows)
    got = profiling.runs(profiling.launches(path), keep="^A$")
    assert [(r["launches"], round(r["us"])) for r in got] == [(2, 10), (1, 20)]
    r = got[0]
    assert abs(r["clock_ghz"] - 2.0) < 1e-9 and abs(r["mfma_busy"] - 0.5) < 1e-9
    assert abs(r["raw"]["SQ_WAIT_ANY/cyc"] - 0.1) < 1e-9  # quad-cycles x 4 over SIMD cycles
    assert r["raw"]["TCC_READ_LATENCY_cyc"] == 350.0
    table = profiling.markdown(got, raw=True)
    assert "SQ_WAIT_ANY/cyc" in table and table.count("\n") == 3


def test_trace_steady_state_uses_the_last_launches(tmp_path):
    header = ["Dispatch_Id", "Kernel_Name", "Start_Timestamp", "End_Timestamp"]
    durs = [50, 40] + [10] * 10
    rows = [[i, "void moe::k<1>(int)", 0, d * 1000] for i, d in enumerate(durs)]
    rows.append([len(durs), "other", 0, 3000])
    path = tmp_path / "run_kernel_trace.csv"
    _write(path, header, rows)
    got = profiling.steady_state(profiling.trace_launches(path), last=10)
    assert got[0] == {"kernel": "moe::k<1>", "launches": 12, "mean_us": 10.0, "min_us": 10.0}
    assert got[1]["kernel"] == "other" and got[1]["launches"] == 1
    stats = tmp_path / "run_kernel_stats.csv"
    _write(stats, ["Name", "Calls", "TotalDurationNs", "AverageNs", "Percentage", "MinNs", "MaxNs"],
           [["void moe::k<1>(int)", 12, 190000, 15833, 98.4, 10000, 50000], ["other", 1, 3000, 3000, 1.6, 3000, 3000]])
    table = profiling.stats_table(stats)
    assert table.splitlines()[2].startswith("| `moe::k<1>` | 12 | 15.83 | 10.00 | 50.00 | 98.40 |")
