"""Benchmark evidence records and their verifier (standard library only, no torch).

A benchmark run stores every raw timing sample next to the statistics derived
from it, the sha256 of every source that was measured, the hardware, the
correctness checks that gated the run and the routed expert counts. A
``manifest.json`` of sha256 hashes seals a directory of such files. ``verify``
recomputes every statistic from the raw samples and rejects a record whose
stored median / p95 / min differ from them, whose sample counts differ from
the stated repeats, whose routed tokens are not conserved, whose forward
validation failed or is missing, whose graph timings are not backed by a
passed replay check, or whose source hashes differ from this checkout.

Record layouts follow the reference so its readers apply unchanged: the
transport record ``results.json`` of ``src/moe_dispatch/cli.py:113-143`` checked
as in ``src/moe_dispatch/evidence.py:10-61``, and the block record
``block_results.json`` of ``src/moe_dispatch/block_benchmark.py:186-210`` checked
as in ``scripts/verify_release.py:16-125``. Implementation labels are the
reference's API names ("CUDA vectorized" is this package's vectorized HIP path,
``implementation="cuda_fused"`` its fused HIP block).

Command line: ``python -m moe_dispatch.evidence DIRECTORY [--seal] [--output FILE]``
verifies every record in DIRECTORY (``--seal`` first writes its manifest).
"""

from __future__ import annotations

import argparse
import hashlib
import json
import math
from pathlib import Path
import statistics
import sys

TRANSPORT_IMPLEMENTATIONS = ("PyTorch reference", "CUDA scalar", "CUDA vectorized")
TRANSPORT_STAGES = ("dispatch", "combine", "dispatch+combine")
BLOCK_IMPLEMENTATIONS = ("torch", "cuda", "cuda_fused")
BLOCK_STAGES = ("router", "dispatch", "experts", "combine", "forward")

PACKAGE_DIR = Path(__file__).resolve().parent
CSRC_DIR = PACKAGE_DIR.parent / "csrc"
HEADER = PACKAGE_DIR.parents[1] / "include" / "moe_hip.h"


def percentile(values, fraction):
    """Linear interpolation between closest ranks (the reference's ``benchmark.py:15-22``)."""
    ordered = sorted(values)
    if not ordered:
        return 0.0
    position = (len(ordered) - 1) * fraction
    lower, upper = math.floor(position), math.ceil(position)
    return ordered[lower] + (ordered[upper] - ordered[lower]) * (position - lower)


def sample_statistics(samples):
    return {"median_us": statistics.median(samples), "p95_us": percentile(samples, 0.95),
            "min_us": min(samples)}


# Package modules that never run inside a measurement: profiling.py summarises
# profiler output files afterwards.
OFFLINE_MODULES = ("profiling.py",)


def source_files():
    """What a measurement depends on: kernel sources, the ABI header and the package modules."""
    files = sorted(CSRC_DIR.glob("*.hip")) + sorted(CSRC_DIR.glob("*.h"))
    if HEADER.is_file():
        files.append(HEADER)
    files += sorted(f for f in PACKAGE_DIR.glob("*.py") if f.name not in OFFLINE_MODULES)
    return [f for f in files if f.is_file()]


def source_hashes():
    return {f.name: hashlib.sha256(f.read_bytes()).hexdigest() for f in source_files()}


def _check_samples(row, repeats, fields=("median_us", "p95_us", "min_us")):
    samples = row["samples_us"]
    if not samples or len(samples) != repeats:
        raise ValueError("raw-sample count differs from the stated repeats")
    if any(not isinstance(v, (int, float)) or not math.isfinite(v) or v <= 0 for v in samples):
        raise ValueError("timings must be finite and positive")
    recomputed = sample_statistics(samples)
    for field in fields:
        if not math.isclose(row[field], recomputed[field], rel_tol=1e-9):
            raise ValueError(f"stored {field} differs from the raw samples")


def _check_counts(case):
    counts = case["expert_counts"]
    if len(counts) != case["experts"] or any(c < 0 for c in counts):
        raise ValueError("incorrect expert-count vector")
    if sum(counts) != case["tokens"] * case["topk"]:
        raise ValueError("expert counts do not conserve routed tokens")


def _cases(configurations):
    cases = {c["case_id"]: c for c in configurations}
    if not cases or len(cases) != len(configurations):
        raise ValueError("empty or duplicate configuration IDs")
    return cases


def read_results(path):
    """Load and check a transport record (``results.json``)."""
    result = json.loads(Path(path).read_text())
    configurations = result.get("configurations", [])
    rows = result.get("benchmarks", [])
    expected_rows = len(TRANSPORT_IMPLEMENTATIONS) * len(TRANSPORT_STAGES)
    if not configurations or len(rows) != len(configurations) * expected_rows:
        raise ValueError("expected three implementations and three stages per configuration")
    if not result.get("block_demo", {}).get("passed"):
        raise ValueError("MoE block validation is missing or failed")
    if result.get("correctness", {}).get("failed") != 0:
        raise ValueError("correctness failed or was not recorded")
    cases = _cases(configurations)
    seen = set()
    for row in rows:
        key = (row["case_id"], row["implementation"], row["stage"])
        if key in seen or row["case_id"] not in cases:
            raise ValueError("duplicate or unknown benchmark row")
        seen.add(key)
        if row["implementation"] not in TRANSPORT_IMPLEMENTATIONS or row["stage"] not in TRANSPORT_STAGES:
            raise ValueError("unknown implementation/stage")
        case = cases[row["case_id"]]
        for field in ("tokens", "hidden", "experts", "topk", "pattern", "dtype"):
            if row[field] != case[field]:
                raise ValueError(f"row/configuration mismatch: {field}")
        _check_samples(row, result["method"]["repeats"], ("median_us", "p95_us"))
        if row["workspace_bytes"] <= 0:
            raise ValueError("workspace bytes must be positive")
    for case in configurations:
        _check_counts(case)
    return result


def summarize(result):
    """Per-stage speedups of the vectorized path over the PyTorch variant and the scalar path."""
    rows = {(r["case_id"], r["implementation"], r["stage"]): r for r in result["benchmarks"]}
    summary = {"gpu": result["hardware"]["gpu"], "configurations": len(result["configurations"]),
               "correctness_checks": result["correctness"]["passed"],
               "method": result["method"]["timing"], "stages": {}}
    for stage in TRANSPORT_STAGES:
        speedups, vs_scalar, memory = [], [], []
        for case in result["configurations"]:
            cid = case["case_id"]
            torch_row = rows[cid, "PyTorch reference", stage]
            scalar = rows[cid, "CUDA scalar", stage]
            vector = rows[cid, "CUDA vectorized", stage]
            speedups.append(torch_row["median_us"] / vector["median_us"])
            vs_scalar.append(1 - vector["median_us"] / scalar["median_us"])
            memory.append(1 - vector["workspace_bytes"] / torch_row["workspace_bytes"])
        summary["stages"][stage] = {
            "median_per_configuration_speedup": statistics.median(speedups),
            "minimum_speedup": min(speedups),
            "maximum_speedup": max(speedups),
            "maximum_latency_reduction_vs_scalar_cuda": max(vs_scalar),
            "minimum_persistent_workspace_reduction": min(memory),
            "maximum_persistent_workspace_reduction": max(memory),
        }
    return summary


def validate_block(data, hashes=None):
    """Check a block record (``block_results.json``); returns its summary.

    ``hashes`` (default: this checkout's ``source_hashes()``) must equal the
    record's ``source_hashes``.
    """
    if data.get("kind") != "moe_block_benchmark":
        raise ValueError("not a block benchmark")
    method = data["method"]
    cases = _cases(data["configurations"])
    for case in cases.values():
        _check_counts(case)
        if case["expert_backend"] != method["expert_backend"]:
            raise ValueError("expert backend mismatch")
    expected_validation = {(c, i) for c in cases for i in BLOCK_IMPLEMENTATIONS}
    validated = set()
    for v in data["validation"]:
        key = (v["case_id"], v["implementation"])
        if key in validated or key not in expected_validation or v["passed"] is not True:
            raise ValueError("duplicate, unknown or failed forward validation")
        validated.add(key)
        for field in ("max_absolute_error", "relative_l2_error"):
            if not math.isfinite(v[field]) or v[field] < 0:
                raise ValueError("invalid correctness error")
        if v["relative_l2_error"] > v["relative_l2_limit"]:
            raise ValueError("relative error exceeds threshold")
    if validated != expected_validation:
        raise ValueError("missing forward validation")
    expected = {(c, i, s) for c in cases for i in BLOCK_IMPLEMENTATIONS for s in BLOCK_STAGES}
    seen, rows = set(), {}
    for r in data["benchmarks"]:
        key = (r["case_id"], r["implementation"], r["stage"])
        if key in seen:
            raise ValueError("duplicate benchmark row")
        seen.add(key)
        graph_row = (key[0] in cases and key[1] in BLOCK_IMPLEMENTATIONS and key[2] == "forward_graph"
                     and method.get("graphs_requested"))
        if key not in expected and not graph_row:
            raise ValueError("unknown benchmark row")
        _check_samples(r, method["repeats"])
        if r["persistent_workspace_bytes"] <= 0:
            raise ValueError("invalid workspace bytes")
        rows[key] = r
    if not expected <= seen:
        raise ValueError("missing benchmark row")
    graph_passed = set()
    if method.get("graphs_requested"):
        for v in data["validation"]:
            if v.get("graph_status") == "passed":
                graph_passed.add((v["case_id"], v["implementation"], "forward_graph"))
            elif v.get("graph_status") != "unsupported" or not v.get("graph_error"):
                raise ValueError("graph validation status is missing or invalid")
        if {k for k in seen if k[2] == "forward_graph"} != graph_passed:
            raise ValueError("graph timings do not match successful replay validation")
    actual = source_hashes() if hashes is None else hashes
    if actual != data["source_hashes"]:
        raise ValueError("measured source hashes differ from this checkout")
    ratios = [rows[c, "torch", "forward"]["median_us"] / rows[c, "cuda_fused", "forward"]["median_us"]
              for c in cases]
    summary = {
        "gpu": data["hardware"]["gpu"],
        "configurations": len(cases),
        "forward_comparisons_passed": len(validated),
        "source_hashes_verified": len(actual),
        "timing_rows_verified": len(seen),
        "median_forward_ratio": statistics.median(ratios),
        "min_forward_ratio": min(ratios),
        "max_forward_ratio": max(ratios),
        "max_absolute_error": max(v["max_absolute_error"] for v in data["validation"]),
        "max_relative_l2_error": max(v["relative_l2_error"] for v in data["validation"]),
        "expert_backend": method["expert_backend"],
        "graphs_requested": bool(method.get("graphs_requested")),
    }
    if method.get("graphs_requested"):
        complete = [c for c in cases if all((c, i, "forward_graph") in rows for i in BLOCK_IMPLEMENTATIONS)]
        summary["graph_replay_checks_passed"] = len(graph_passed)
        summary["complete_graph_comparison_cases"] = len(complete)
        graph_ratios = [rows[c, "torch", "forward_graph"]["median_us"]
                        / rows[c, "cuda_fused", "forward_graph"]["median_us"] for c in complete]
        if graph_ratios:
            summary.update(median_graph_ratio=statistics.median(graph_ratios),
                           min_graph_ratio=min(graph_ratios), max_graph_ratio=max(graph_ratios))
    return summary


def write_manifest(directory):
    """Seal every file under ``directory`` (except the manifest) with its sha256."""
    directory = Path(directory)
    hashes = {}
    for path in sorted(p for p in directory.rglob("*") if p.is_file() and p.name != "manifest.json"):
        hashes[path.relative_to(directory).as_posix()] = hashlib.sha256(path.read_bytes()).hexdigest()
    manifest = {"sha256": hashes}
    (directory / "manifest.json").write_text(json.dumps(manifest, indent=2) + "\n")
    return manifest


def check_manifest(directory):
    directory = Path(directory).resolve()
    manifest = json.loads((directory / "manifest.json").read_text())
    for relative, expected in manifest["sha256"].items():
        resolved = (directory / relative).resolve()
        if not resolved.is_relative_to(directory):
            raise ValueError("manifest path escapes the evidence directory")
        if hashlib.sha256(resolved.read_bytes()).hexdigest() != expected:
            raise ValueError(f"evidence hash mismatch: {relative}")
    return manifest


def verify(directory, hashes=None):
    """Check every record under ``directory``; returns a summary per record file."""
    directory = Path(directory)
    summary = {}
    if (directory / "manifest.json").exists():
        summary["manifest_files"] = len(check_manifest(directory)["sha256"])
    records = sorted(directory.rglob("block_results.json")) + sorted(directory.rglob("results.json"))
    if not records:
        raise ValueError("no block_results.json or results.json under the directory")
    for path in records:
        key = path.relative_to(directory).as_posix()
        if path.name == "block_results.json":
            summary[key] = validate_block(json.loads(path.read_text()), hashes)
        else:
            summary[key] = summarize(read_results(path))
    return summary


def main(argv=None):
    parser = argparse.ArgumentParser(description="Verify benchmark evidence records.")
    parser.add_argument("directory", type=Path)
    parser.add_argument("--seal", action="store_true", help="write manifest.json before verifying")
    parser.add_argument("--output", type=Path, help="also write the summary here")
    args = parser.parse_args(argv)
    try:
        if args.seal:
            write_manifest(args.directory)
        content = json.dumps(verify(args.directory), indent=2) + "\n"
    except (ValueError, KeyError, OSError) as error:
        print(f"evidence: {error}", file=sys.stderr)
        return 1
    if args.output:
        args.output.write_text(content)
    print(content, end="")
    return 0


if __name__ == "__main__":
    sys.exit(main())
