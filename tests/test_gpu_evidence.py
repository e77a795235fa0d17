"""Evidence records written by real runs on the GPU verify end to end.

The smoke suites (reference ``block_benchmark.py:15-17`` and ``benchmark.py:49-50``)
are run with a few repeats, written to disk, sealed with a manifest and
verified by ``moe_dispatch.evidence.verify`` against this checkout's source
hashes. The block record must show every forward validation passed and the
fused HIP block faster than the PyTorch variant on every case.
"""

import json

import pytest

from moe_dispatch import evidence
from tests._helpers import gpu

pytestmark = gpu


def test_block_record_from_a_real_run_verifies(tmp_path):
    from moe_dispatch.block_benchmark import run_block_benchmark

    result = run_block_benchmark(suite="smoke", warmup=1, repeats=5, output=tmp_path, graphs=True)
    assert {v["implementation"] for v in result["validation"]} == set(evidence.BLOCK_IMPLEMENTATIONS)
    fused = [v for v in result["validation"] if v["implementation"] == "cuda_fused"]
    assert all(v["graph_status"] == "passed" for v in fused)
    evidence.write_manifest(tmp_path)
    summary = evidence.verify(tmp_path)["block_results.json"]
    assert summary["forward_comparisons_passed"] == 6
    assert summary["timing_rows_verified"] >= 30
    assert summary["min_forward_ratio"] > 1.0, summary
    assert summary["max_relative_l2_error"] < 5e-3


def test_transport_record_from_a_real_run_verifies(tmp_path):
    from moe_dispatch.benchmark import run_transport_benchmark

    run_transport_benchmark(tmp_path, suite="smoke", warmup=1, repeats=5)
    record = json.loads((tmp_path / "results.json").read_text())
    assert record["correctness"]["failed"] == 0 and record["correctness"]["passed"] == 36
    assert record["block_demo"]["passed"]
    summary = evidence.verify(tmp_path)["results.json"]
    assert summary["configurations"] == 2
    assert set(summary["stages"]) == set(evidence.TRANSPORT_STAGES)


def test_tampered_real_record_is_rejected(tmp_path):
    from moe_dispatch.block_benchmark import run_block_benchmark

    run_block_benchmark(suite="smoke", warmup=1, repeats=5, output=tmp_path, graphs=False)
    path = tmp_path / "block_results.json"
    record = json.loads(path.read_text())
    record["benchmarks"][0]["median_us"] *= 0.5
    with pytest.raises(ValueError, match="median"):
        evidence.validate_block(record)
