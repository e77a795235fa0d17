"""Summaries of rocprofv3 counter collections for the expert GEMMs (MFMA utilisation, clock).

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

Each counter appears only if it was collected. Standard library only.
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
        if keep and not re.search(keep, name):
            continue
        if groups and groups[-1][0] == name:
            groups[-1][1].append((dur, counters))
        else:
            groups.append((name, [(dur, counters)]))
    out = []
    for name, members in groups:
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
        out.append(row)
    return out


def markdown(rows):
    cols = [("kernel", "{}"), ("launches", "{}"), ("averaged", "{}"), ("us", "{:.1f}"), ("clock_ghz", "{:.3f}"),
            ("mfma_busy", "{:.3f}"), ("cu_busy", "{:.3f}"), ("mfma_flop", "{:.4g}")]
    present = [(c, f) for c, f in cols if any(c in r for r in rows)]
    lines = ["| " + " | ".join(c for c, _ in present) + " |", "|" + "---|" * len(present)]
    for r in rows:
        lines.append("| " + " | ".join(f.format(r[c]) if c in r else "" for c, f in present) + " |")
    return "\n".join(lines)


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("csv", help="rocprofv3 run_counter_collection.csv")
    ap.add_argument("--keep", default=None, help="regex of kernel names to keep")
    ap.add_argument("--last", type=int, default=None, help="average the last N launches of each run")
    args = ap.parse_args(argv)
    print(markdown(runs(launches(args.csv), args.keep, args.last)))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
