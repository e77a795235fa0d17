"""The evidence verifier on synthetic records (CPU, no torch in the verifier).

A consistent record passes; each single tampering a verifier must catch
(a stored statistic that does not follow from the raw samples, a wrong sample
count, a non-positive sample, routed tokens not conserved, a failed or missing
forward validation, a missing or unknown timing row, a graph timing without a
passed replay check, a source-hash mismatch, a sealed file changed after
sealing) is rejected.
"""

import copy
import json
import random

import pytest

from moe_dispatch import evidence

REPEATS = 7


def _timed(rng):
    samples = [rng.uniform(5.0, 50.0) for _ in range(REPEATS)]
    return {**evidence.sample_statistics(samples), "samples_us": samples}


def block_record(graphs=True, seed=0):
    rng = random.Random(seed)
    configurations = [
        {"case_id": 0, "tokens": 128, "hidden": 512, "intermediate": 1024, "experts": 8, "topk": 2,
         "alignment": 8, "pattern": "balanced", "dtype": "bfloat16", "expert_backend": "grouped_mm",
         "expert_counts": [32] * 8},
        {"case_id": 1, "tokens": 16, "hidden": 512, "intermediate": 1024, "experts": 8, "topk": 2,
         "alignment": 8, "pattern": "skewed", "dtype": "bfloat16", "expert_backend": "grouped_mm",
         "expert_counts": [16, 16, 0, 0, 0, 0, 0, 0]},
    ]
    validation, rows = [], []
    for case in configurations:
        for impl in evidence.BLOCK_IMPLEMENTATIONS:
            v = {"case_id": case["case_id"], "implementation": impl, "passed": True,
                 "max_absolute_error": 1e-3, "relative_l2_error": 2e-4, "rtol": 0.03, "atol": 0.03,
                 "relative_l2_limit": 0.02}
            if graphs:
                v["graph_status"] = "passed"
            validation.append(v)
            stages = evidence.BLOCK_STAGES + (("forward_graph",) if graphs else ())
            for stage in stages:
                rows.append({"case_id": case["case_id"], "implementation": impl, "stage": stage,
                             "persistent_workspace_bytes": 1 << 20, **_timed(rng)})
    return {"kind": "moe_block_benchmark", "hardware": {"gpu": "AMD Instinct MI355X"},
            "source_hashes": {"gemm.hip": "ab" * 32}, "configurations": configurations,
            "validation": validation, "benchmarks": rows,
            "method": {"suite": "smoke", "warmup": 1, "repeats": REPEATS, "expert_backend": "grouped_mm",
                       "graphs_requested": graphs}}


def transport_record(seed=0):
    rng = random.Random(seed)
    configurations = [{"case_id": 0, "tokens": 128, "hidden": 512, "experts": 8, "topk": 2,
                       "pattern": "balanced", "dtype": "float16", "expert_counts": [32] * 8}]
    rows = []
    for case in configurations:
        for impl in evidence.TRANSPORT_IMPLEMENTATIONS:
            for stage in evidence.TRANSPORT_STAGES:
                rows.append({**{k: case[k] for k in ("case_id", "tokens", "hidden", "experts", "topk",
                                                     "pattern", "dtype")},
                             "implementation": impl, "stage": stage, "workspace_bytes": 4096, **_timed(rng)})
    return {"kind": "transport_benchmark", "hardware": {"gpu": "AMD Instinct MI355X"},
            "correctness": {"passed": 36, "failed": 0}, "block_demo": {"passed": True},
            "configurations": configurations, "benchmarks": rows, "source_hashes": {},
            "method": {"suite": "smoke", "warmup": 1, "repeats": REPEATS, "timing": "events"}}


def _validate(record):
    return evidence.validate_block(record, hashes=record["source_hashes"])


def test_consistent_block_record_passes_and_summarises():
    record = block_record()
    summary = _validate(record)
    assert summary["forward_comparisons_passed"] == 6
    assert summary["timing_rows_verified"] == 36
    assert summary["graph_replay_checks_passed"] == 6
    assert summary["complete_graph_comparison_cases"] == 2
    rows = {(r["case_id"], r["implementation"], r["stage"]): r for r in record["benchmarks"]}
    ratio0 = rows[0, "torch", "forward"]["median_us"] / rows[0, "cuda_fused", "forward"]["median_us"]
    ratio1 = rows[1, "torch", "forward"]["median_us"] / rows[1, "cuda_fused", "forward"]["median_us"]
    assert summary["min_forward_ratio"] == pytest.approx(min(ratio0, ratio1))
    assert _validate(block_record(graphs=False))["graphs_requested"] is False


def _tamper(mutate):
    record = block_record()
    mutate(record)
    return record


BLOCK_TAMPERING = {
    "median": lambda r: r["benchmarks"][3].__setitem__("median_us", r["benchmarks"][3]["median_us"] * 1.01),
    "p95": lambda r: r["benchmarks"][0].__setitem__("p95_us", r["benchmarks"][0]["p95_us"] + 0.5),
    "min": lambda r: r["benchmarks"][5].__setitem__("min_us", r["benchmarks"][5]["min_us"] - 0.5),
    "sample count": lambda r: r["benchmarks"][2]["samples_us"].pop(),
    "non-positive sample": lambda r: r["benchmarks"][1]["samples_us"].__setitem__(0, 0.0),
    "not conserved": lambda r: r["configurations"][1]["expert_counts"].__setitem__(0, 17),
    "count vector length": lambda r: r["configurations"][0]["expert_counts"].append(0),
    "failed validation": lambda r: r["validation"][4].__setitem__("passed", False),
    "missing validation": lambda r: r["validation"].pop(),
    "error above limit": lambda r: r["validation"][0].__setitem__("relative_l2_error", 0.5),
    "missing row": lambda r: r["benchmarks"].pop(0),
    "duplicate row": lambda r: r["benchmarks"].append(copy.deepcopy(r["benchmarks"][0])),
    "unknown stage": lambda r: r["benchmarks"][0].__setitem__("stage", "softmax"),
    "graph row without replay": lambda r: r["validation"][2].__setitem__("graph_status", "unsupported"),
    "graph status missing": lambda r: r["validation"][2].pop("graph_status"),
    "backend mismatch": lambda r: r["configurations"][0].__setitem__("expert_backend", "triton"),
    "workspace bytes": lambda r: r["benchmarks"][7].__setitem__("persistent_workspace_bytes", 0),
}


@pytest.mark.parametrize("name", sorted(BLOCK_TAMPERING))
def test_block_tampering_is_rejected(name):
    with pytest.raises(ValueError):
        _validate(_tamper(BLOCK_TAMPERING[name]))


def test_graph_rows_need_graphs_requested():
    record = block_record()
    record["method"]["graphs_requested"] = False
    for v in record["validation"]:
        v.pop("graph_status")
    with pytest.raises(ValueError, match="unknown benchmark row"):
        _validate(record)


def test_unsupported_graph_with_error_and_no_row_passes():
    record = block_record()
    record["validation"][0]["graph_status"] = "unsupported"
    record["validation"][0]["graph_error"] = "capture failed"
    record["benchmarks"] = [r for r in record["benchmarks"]
                            if not (r["case_id"] == 0 and r["implementation"] == "torch"
                                    and r["stage"] == "forward_graph")]
    summary = _validate(record)
    assert summary["graph_replay_checks_passed"] == 5
    assert summary["complete_graph_comparison_cases"] == 1


def test_source_hashes_must_match_the_checkout():
    with pytest.raises(ValueError, match="source hashes"):
        evidence.validate_block(block_record())  # synthetic hashes vs this checkout
    record = block_record()
    record["source_hashes"] = evidence.source_hashes()
    assert evidence.validate_block(record)["source_hashes_verified"] == len(record["source_hashes"])


def test_source_hashes_cover_kernels_header_and_modules():
    hashes = evidence.source_hashes()
    assert {"gemm.hip", "dispatch.hip", "router.hip", "abi.hip", "moe_common.h", "moe_hip.h",
            "evidence.py", "layer.py"} <= set(hashes)
    assert "profiling.py" not in hashes  # summarises profiler output after a run
    assert all(len(v) == 64 for v in hashes.values())


def test_transport_record_reads_and_summarises(tmp_path):
    record = transport_record()
    (tmp_path / "results.json").write_text(json.dumps(record))
    summary = evidence.summarize(evidence.read_results(tmp_path / "results.json"))
    rows = {(r["implementation"], r["stage"]): r for r in record["benchmarks"]}
    speedup = rows["PyTorch reference", "dispatch"]["median_us"] / rows["CUDA vectorized", "dispatch"]["median_us"]
    assert summary["stages"]["dispatch"]["median_per_configuration_speedup"] == pytest.approx(speedup)
    assert summary["correctness_checks"] == 36


TRANSPORT_TAMPERING = {
    "median": lambda r: r["benchmarks"][4].__setitem__("median_us", 1.0),
    "no demo": lambda r: r.pop("block_demo"),
    "correctness failed": lambda r: r["correctness"].__setitem__("failed", 1),
    "row mismatch": lambda r: r["benchmarks"][0].__setitem__("hidden", 1024),
    "workspace": lambda r: r["benchmarks"][0].__setitem__("workspace_bytes", 0),
    "missing row": lambda r: r["benchmarks"].pop(),
    "counts": lambda r: r["configurations"][0]["expert_counts"].__setitem__(0, 0),
}


@pytest.mark.parametrize("name", sorted(TRANSPORT_TAMPERING))
def test_transport_tampering_is_rejected(tmp_path, name):
    record = transport_record()
    TRANSPORT_TAMPERING[name](record)
    (tmp_path / "results.json").write_text(json.dumps(record))
    with pytest.raises((ValueError, KeyError)):
        evidence.read_results(tmp_path / "results.json")


def test_manifest_seals_a_directory(tmp_path):
    (tmp_path / "results.json").write_text(json.dumps(transport_record()))
    (tmp_path / "sub").mkdir()
    (tmp_path / "sub" / "notes.txt").write_text("run log")
    manifest = evidence.write_manifest(tmp_path)
    assert set(manifest["sha256"]) == {"results.json", "sub/notes.txt"}
    assert evidence.verify(tmp_path)["manifest_files"] == 2
    (tmp_path / "sub" / "notes.txt").write_text("edited")
    with pytest.raises(ValueError, match="hash mismatch"):
        evidence.check_manifest(tmp_path)


def test_manifest_paths_cannot_escape(tmp_path):
    (tmp_path / "outside.txt").write_text("x")
    inner = tmp_path / "evidence"
    inner.mkdir()
    (inner / "manifest.json").write_text(json.dumps({"sha256": {"../outside.txt": "00"}}))
    with pytest.raises(ValueError, match="escapes"):
        evidence.check_manifest(inner)


def test_command_line_seals_and_verifies(tmp_path, capsys):
    (tmp_path / "results.json").write_text(json.dumps(transport_record()))
    assert evidence.main([str(tmp_path), "--seal", "--output", str(tmp_path / "summary.txt")]) == 0
    out = json.loads(capsys.readouterr().out)
    assert out["manifest_files"] == 1 and "results.json" in out
    bad = transport_record()
    bad["benchmarks"][0]["median_us"] += 1.0
    (tmp_path / "results.json").write_text(json.dumps(bad))
    assert evidence.main([str(tmp_path)]) == 1  # the manifest (and the record) no longer verify


def test_verifier_does_not_need_torch():
    import subprocess
    import sys
    from pathlib import Path

    package = Path(evidence.__file__).resolve().parents[1]
    code = ("import sys; sys.modules['torch'] = None; sys.path.insert(0, %r); "
            "from moe_dispatch import evidence; print(len(evidence.source_hashes()))" % str(package))
    proc = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=60)
    assert proc.returncode == 0, proc.stderr


def test_committed_bundle_is_internally_consistent():
    """profiles/evidence: the manifest holds, every statistic follows from its raw
    samples and every validation passed. (Whether its source hashes match the
    checkout is what ``verify`` adds; a later source change ends that match.)"""
    from pathlib import Path

    directory = Path(__file__).resolve().parents[1] / "profiles" / "evidence"
    if not (directory / "manifest.json").exists():
        pytest.skip("no committed evidence bundle")
    assert {"block_results.json", "results.json"} <= set(evidence.check_manifest(directory)["sha256"])
    block = json.loads((directory / "block_results.json").read_text())
    summary = evidence.validate_block(block, hashes=block["source_hashes"])
    assert summary["forward_comparisons_passed"] == 15 and summary["graph_replay_checks_passed"] == 15
    assert summary["max_relative_l2_error"] < 5e-4
    transport = evidence.summarize(evidence.read_results(directory / "results.json"))
    assert transport["correctness_checks"] == 36 and transport["configurations"] == 12
