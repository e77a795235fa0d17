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


def test_trace_steady_state_uses_the_longest_back_to_back_run(tmp_path):
    header = ["Dispatch_Id", "Kernel_Name", "Start_Timestamp", "End_Timestamp"]
    # Two forwards (k, other), a timed replay of 12 back-to-back k calls, then three
    # more forwards whose k launches must not enter the steady state.
    names = ["k", "other"] * 2 + ["k"] * 12 + ["other", "k"] * 3
    durs = [70, 3, 60, 3] + [50, 40] + [10] * 10 + [3, 90] * 3
    rows = [[i, "void moe::k<1>(int)" if n == "k" else "other", 0, d * 1000]
            for i, (n, d) in enumerate(zip(names, durs))]
    path = tmp_path / "run_kernel_trace.csv"
    _write(path, header, rows)
    got = profiling.steady_state(profiling.trace_launches(path), last=10)
    assert got[0] == {"kernel": "moe::k<1>", "launches": 17, "run": 12, "mean_us": 10.0, "min_us": 10.0}
    # A kernel never launched twice in a row averages its last launches.
    assert got[1] == {"kernel": "other", "launches": 5, "run": 1, "mean_us": 3.0, "min_us": 3.0}
    # Two equally long runs: the later one.
    again = profiling.steady_state([("a", 5.0), ("a", 5.0), ("b", 1.0), ("a", 7.0), ("a", 9.0)], last=10)
    assert again[0]["mean_us"] == 8.0 and again[0]["run"] == 2
    # Kernels filtered out by `keep` still cut runs.
    cut = profiling.steady_state([("a", 5.0), ("b", 1.0), ("a", 7.0)], last=10, keep="^a$")
    assert cut[0]["run"] == 1 and cut[0]["mean_us"] == 6.0
    table = profiling.trace_markdown(got)
    assert table.splitlines()[2] == "| `moe::k<1>` | 17 | 12 | 10.00 | 10.00 |"
    stats = tmp_path / "run_kernel_stats.csv"
    _write(stats, ["Name", "Calls", "TotalDurationNs", "AverageNs", "Percentage", "MinNs", "MaxNs"],
           [["void moe::k<1>(int)", 12, 190000, 15833, 98.4, 10000, 50000], ["other", 1, 3000, 3000, 1.6, 3000, 3000]])
    table = profiling.stats_table(stats)
    assert table.splitlines()[2].startswith("| `moe::k<1>` | 12 | 15.83 | 10.00 | 50.00 | 98.40 |")
