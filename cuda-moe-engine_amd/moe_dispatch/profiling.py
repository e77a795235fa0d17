"""Summaries of rocprofv3 output: counter collections for the expert GEMMs
(MFMA utilisation, clock, stalls, memory) and kernel traces (steady-state
launch times).

``python -m moe_dispatch.profiling <dir>/run_counter_collection.csv`` prints a
markdown table with one line per run of consecutive launches of one kernel
(the order the program launched them), with:

* the mean launch duration from the dispatch timestamps;
* the clock: ``GRBM_GUI_ACTIVE`` counts GPU-busy cycles summed over the XCDs
  (8 on MI355X), so cycles per XCD / duration;
* MFMA busy: ``SQ_VALU_MFMA_BUSY_CYCLES`` is summed over every SIMD (1024 on
  MI355X: 256 CUs x 4), so busy / (SIMDs x cycles);
* the MFMA work executed: ``SQ_INSTS_VALU_MFMA_MOPS_BF16`` counts units of 512
  FLOP, padding rows included (the algorithmic FLOP excludes them);
* the fraction of CU cycles with a wave resident (``SQ_BUSY_CU_CYCLES``).

Each counter appears only if it was collected; ``--raw`` adds every other
collected counter, normalised where its unit is known (quad-cycle wave
counters and per-SIMD busy counters over SIMD cycles, per-CU LDS and TA stall
counters over CU cycles, ``TCP_TCC_READ_REQ_LATENCY`` as cycles per request).

``python -m moe_dispatch.profiling --trace <dir>/run_kernel_trace.csv`` prints,
per kernel, the mean and minimum duration of the last N launches of its longest
run of back-to-back launches (the steady state of a timed replay of repeated
calls) and, with ``--stats <dir>/run_kernel_stats.csv``, rocprofv3's table of
all launches. Standard library only.
"""

from __future__ import annotations

import argparse
import csv
import re
from collections import OrderedDict

XCDS = 8
SIMDS = 1024
CUS = 256


def _short(name):
    name = re.sub(r"^void ", "", name)
    name = name.split("(")[0] if name.startswith("moe::") else name
    return name[:70]


def launches(path):
    """Launches in dispatch order: [(kernel, duration_us, {counter: value})]."""
    by_dispatch = OrderedDict()
    with open(path, newline="") as f:
        for rec in csv.DictReader(f):
            key = int(rec["Dispatch_Id"])
            entry = by_dispatch.get(key)
            if entry is None:
                dur = (int(rec["End_Timestamp"]) - int(rec["Start_Timestamp"])) / 1000.0
                entry = by_dispatch[key] = (_short(rec["Kernel_Name"]), dur, {})
            entry[2][rec["Counter_Name"]] = float(rec["Counter_Value"])
    return [by_dispatch[k] for k in sorted(by_dispatch)]


def runs(items, keep=None, last=None):
    """Group consecutive launches of one kernel; optionally keep kernels matching `keep` and
    average only the last `last` launches of each run (the steady state)."""
    groups = []
    for name, dur, counters in items:
        # Runs are cut by any other kernel, kept or not: two runs of one kernel
        # with other work between them stay apart.
        if groups and groups[-1][0] == name:
            groups[-1][1].append((dur, counters))
        else:
            groups.append((name, [(dur, counters)]))
    out = []
    for name, members in groups:
        if keep and not re.search(keep, name):
            continue
        chosen = members[-last:] if last else members
        n = len(chosen)
        dur = sum(d for d, _ in chosen) / n
        mean = {}
        for _, counters in chosen:
            for c, v in counters.items():
                mean[c] = mean.get(c, 0.0) + v / n
        row = {"kernel": name, "launches": len(members), "averaged": n, "us": dur}
        gui = mean.get("GRBM_GUI_ACTIVE")
        if gui:
            cycles = gui / XCDS
            row["clock_ghz"] = cycles / (dur * 1e3)
            if "SQ_VALU_MFMA_BUSY_CYCLES" in mean:
                row["mfma_busy"] = mean["SQ_VALU_MFMA_BUSY_CYCLES"] / (SIMDS * cycles)
            if "SQ_BUSY_CU_CYCLES" in mean:
                row["cu_busy"] = mean["SQ_BUSY_CU_CYCLES"] / (CUS * cycles)
        if "SQ_INSTS_VALU_MFMA_MOPS_BF16" in mean:
            row["mfma_flop"] = mean["SQ_INSTS_VALU_MFMA_MOPS_BF16"] * 512
        row["raw"] = _normalised(mean, gui / XCDS if gui else None)
        out.append(row)
    return out


# Wave counters in quad-cycles summed over the SIMDs; per-SIMD busy counters;
# per-CU counters.
_QUAD_SIMD = ("SQ_WAVE_CYCLES", "SQ_WAIT_ANY", "SQ_WAIT_INST_ANY", "SQ_WAIT_INST_LDS", "SQ_ACTIVE_INST_ANY",
              "SQ_ACTIVE_INST_LDS", "SQ_ACTIVE_INST_VMEM", "SQ_ACTIVE_INST_VALU")
_PER_CU = ("SQ_LDS_IDX_ACTIVE", "SQ_LDS_BANK_CONFLICT", "SQ_LDS_DATA_FIFO_FULL", "SQ_LDS_CMD_FIFO_FULL",
           "SQ_VMEM_TA_ADDR_FIFO_FULL", "SQ_VMEM_TA_CMD_FIFO_FULL")
_SKIP = ("GRBM_GUI_ACTIVE", "SQ_VALU_MFMA_BUSY_CYCLES", "SQ_BUSY_CU_CYCLES", "SQ_INSTS_VALU_MFMA_MOPS_BF16")


def _normalised(mean, cycles):
    out = {}
    for name, value in mean.items():
        if name in _SKIP:
            continue
        key = name[:-4] if name.endswith("_sum") else name
        if cycles and name in _QUAD_SIMD:
            out[key + "/cyc"] = value * 4 / (SIMDS * cycles)
        elif cycles and name in _PER_CU:
            out[key + "/cyc"] = value / (CUS * cycles)
        elif key == "TCP_TCC_READ_REQ_LATENCY":
            req = mean.get("TCP_TCC_READ_REQ_sum", mean.get("TCP_TCC_READ_REQ"))
            out["TCC_READ_LATENCY_cyc"] = value / req if req else float("nan")
        else:
            out[key] = value
    return out


def trace_launches(path):
    """(kernel, duration_us) in dispatch order from a rocprofv3 kernel-trace CSV."""
    rows = []
    with open(path, newline="") as f:
        for rec in csv.DictReader(f):
            dur = (int(rec["End_Timestamp"]) - int(rec["Start_Timestamp"])) / 1000.0
            rows.append((int(rec.get("Dispatch_Id", len(rows))), _short(rec["Kernel_Name"]), dur))
    rows.sort()
    return [(name, dur) for _, name, dur in rows]


def steady_state(items, last=10, keep=None):
    """Per kernel (first-launch order): its launches, the length of its longest run of
    back-to-back launches (no other kernel between them: a call replayed from a graph of
    repeated calls), and the mean and min of the last `last` launches of that run (the
    last such run where several are equally long). Launches after the run (a later
    forward) do not enter the mean. A kernel never launched twice in a row averages its
    last `last` launches."""
    by = OrderedDict()
    prev = None
    for name, dur in items:
        if keep and not re.search(keep, name):
            prev = name
            continue
        entry = by.setdefault(name, {"launches": 0, "runs": []})
        entry["launches"] += 1
        if prev == name:
            entry["runs"][-1].append(dur)
        else:
            entry["runs"].append([dur])
        prev = name
    out = []
    for name, entry in by.items():
        longest = max(len(r) for r in entry["runs"])
        if longest > 1:
            chosen = [r for r in entry["runs"] if len(r) == longest][-1]
        else:
            chosen = [r[0] for r in entry["runs"]]
        tail = chosen[-last:]
        out.append({"kernel": name, "launches": entry["launches"], "run": longest,
                    "mean_us": sum(tail) / len(tail), "min_us": min(tail)})
    return out


def stats_table(path, top=15):
    """rocprofv3's kernel stats CSV as a markdown table (the `top` kernels by time)."""
    with open(path, newline="") as f:
        recs = list(csv.DictReader(f))
    recs.sort(key=lambda r: -float(r["TotalDurationNs"]))
    lines = ["| kernel | calls | avg us | min us | max us | % of GPU time |", "|---|---|---|---|---|---|"]
    for r in recs[:top]:
        lines.append("| `{}` | {} | {:.2f} | {:.2f} | {:.2f} | {:.2f} |".format(
            _short(r["Name"])[:90], r["Calls"], float(r["AverageNs"]) / 1000, float(r["MinNs"]) / 1000,
            float(r["MaxNs"]) / 1000, float(r["Percentage"])))
    return "\n".join(lines)


def markdown(rows, raw=False):
    cols = [("kernel", "{}"), ("launches", "{}"), ("averaged", "{}"), ("us", "{:.1f}"), ("clock_ghz", "{:.3f}"),
            ("mfma_busy", "{:.3f}"), ("cu_busy", "{:.3f}"), ("mfma_flop", "{:.4g}")]
    present = [(c, f) for c, f in cols if any(c in r for r in rows)]
    extra = sorted({k for r in rows for k in r.get("raw", {})}) if raw else []
    lines = ["| " + " | ".join([c for c, _ in present] + extra) + " |", "|" + "---|" * (len(present) + len(extra))]
    for r in rows:
        cells = [f.format(r[c]) if c in r else "" for c, f in present]
        cells += ["{:.4g}".format(r["raw"][k]) if k in r.get("raw", {}) else "" for k in extra]
        lines.append("| " + " | ".join(cells) + " |")
    return "\n".join(lines)


def trace_markdown(rows):
    lines = ["| kernel | launches | longest back-to-back run | mean us (its last N) | min us (its last N) |",
             "|---|---|---|---|---|"]
    for r in rows:
        lines.append("| `{}` | {} | {} | {:.2f} | {:.2f} |".format(r["kernel"], r["launches"], r["run"], r["mean_us"],
                                                                    r["min_us"]))
    return "\n".join(lines)


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("csv", help="rocprofv3 run_counter_collection.csv (or, with --trace, run_kernel_trace.csv)")
    ap.add_argument("--keep", default=None, help="regex of kernel names to keep")
    ap.add_argument("--last", type=int, default=None,
                    help="average the last N launches of each run (with --trace: of each kernel's longest run)")
    ap.add_argument("--raw", action="store_true", help="also every other collected counter, normalised")
    ap.add_argument("--trace", action="store_true", help="the csv is a kernel trace: steady-state launch times")
    ap.add_argument("--stats", default=None, help="with --trace: run_kernel_stats.csv for the all-launches table")
    args = ap.parse_args(argv)
    if args.trace:
        print(trace_markdown(steady_state(trace_launches(args.csv), args.last or 10, args.keep)))
        if args.stats:
            print()
            print(stats_table(args.stats))
        return 0
    print(markdown(runs(launches(args.csv), args.keep, args.last), args.raw))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
