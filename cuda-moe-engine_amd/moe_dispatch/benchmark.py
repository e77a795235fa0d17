"""Timing helpers and the seeded transport benchmark with raw samples.

``measure`` reports the reference's statistics (``src/moe_dispatch/benchmark.py:15-45``:
median, p95 by linear interpolation, min and the raw samples) from events on
the current stream. ``benchmark``
runs the reference's transport suites (``benchmark.py:48-130``): per case, the
PyTorch transport and the scalar and vectorized HIP paths are validated first,
then dispatch, combine and both together are timed in an order rotated per
case. ``run_transport_benchmark`` writes the ``results.json`` record that
``moe_dispatch.evidence.read_results`` checks.
"""

import json
import math
import platform
import statistics
import time
from pathlib import Path

import torch

from .evidence import percentile, read_results, sample_statistics, source_hashes

__all__ = ["percentile", "sample_statistics", "measure", "hardware_metadata", "benchmark", "transport_moe_check",
           "run_transport_benchmark"]


@torch.inference_mode()
def measure(function, warmup, repeats):
    """Time ``repeats`` calls of ``function`` (µs each) after ``warmup`` untimed ones.

    Same statistics as the reference's ``measure`` (``benchmark.py:25-45``).
    The calls run back to back on the current stream, separated by repeats + 1
    recorded events: sample i is the time between boundary i and i + 1, so
    each sample is one call's device time, launch gaps included, and no event
    pair is recorded twice around the same gap.
    """
    for _ in range(warmup):
        function()
    torch.cuda.synchronize()
    marks = [torch.cuda.Event(enable_timing=True) for _ in range(repeats + 1)]
    marks[0].record()
    for mark in marks[1:]:
        function()
        mark.record()
    torch.cuda.synchronize()
    values_us = [a.elapsed_time(b) * 1000.0 for a, b in zip(marks, marks[1:])]
    return {**sample_statistics(values_us), "samples_us": values_us}


def hardware_metadata():
    """GPU, ROCm and host software the numbers were measured on."""
    properties = torch.cuda.get_device_properties(0)
    return {
        "gpu": properties.name,
        "gcn_arch": getattr(properties, "gcnArchName", "unknown"),
        "compute_units": properties.multi_processor_count,
        "gpu_memory_bytes": properties.total_memory,
        "torch_version": torch.__version__,
        "torch_hip": torch.version.hip,
        "python": platform.python_version(),
        "host": platform.node(),
        "utc_run_time": time.strftime("%Y-%m-%dT%H:%M:%SZ", time.gmtime()),
    }


def transport_cases(suite):
    """(tokens, hidden, experts, pattern) per case, the reference's three suites."""
    if suite == "smoke":
        return [(128, 512, 8, "balanced"), (2048, 1024, 16, "skewed")]
    if suite == "quick":
        return [(t, h, e, p) for t in (128, 2048, 8192) for h, e in ((512, 8), (1024, 16))
                for p in ("balanced", "skewed")]
    if suite == "full":
        return [(t, h, e, p) for t in (128, 512, 2048, 8192) for h in (512, 1024) for e in (8, 16)
                for p in ("balanced", "skewed")]
    raise ValueError("suite must be smoke, quick or full")


@torch.inference_mode()
def benchmark(extension, suite, warmup, repeats):
    """Validated, rotated timings of the three transport paths; returns (configurations, rows)."""
    from .reference import TorchWorkspace
    from .routing import make_case
    from .validation import validate_case
    from .workspace import CudaWorkspace

    configurations, records = [], []
    cases = transport_cases(suite)
    for case_id, (tokens, hidden, experts, pattern) in enumerate(cases):
        seed = 100 + case_id
        x, ids32, ids64, weights = make_case(tokens, hidden, experts, 2, torch.float16, pattern, seed)
        workspaces = {
            "PyTorch reference": TorchWorkspace(tokens, hidden, experts, 2, x.dtype),
            "CUDA scalar": CudaWorkspace(tokens, hidden, experts, 2, x.dtype, vectorized=False,
                                         extension=extension),
            "CUDA vectorized": CudaWorkspace(tokens, hidden, experts, 2, x.dtype, vectorized=True,
                                             extension=extension),
        }
        counts = torch.bincount(ids64.reshape(-1), minlength=experts).cpu().tolist()
        configurations.append({"case_id": case_id, "tokens": tokens, "hidden": hidden, "experts": experts,
                               "topk": 2, "pattern": pattern, "dtype": "float16", "expert_counts": counts})
        for workspace in workspaces.values():  # every path is validated before it is timed
            validate_case(workspace, x, ids32, ids64, weights, experts, seed)
        names = list(workspaces)
        names = names[case_id % 3:] + names[: case_id % 3]
        for name in names:
            workspace = workspaces[name]
            workspace.dispatch(x, ids32, ids64)

            def dispatch():
                workspace.dispatch(x, ids32, ids64)

            def combine():
                workspace.combine(workspace.packed, weights)

            def both():
                workspace.dispatch(x, ids32, ids64)
                workspace.combine(workspace.packed, weights)

            for stage, function in (("dispatch", dispatch), ("combine", combine), ("dispatch+combine", both)):
                records.append({"case_id": case_id, "tokens": tokens, "hidden": hidden, "experts": experts,
                                "topk": 2, "pattern": pattern, "dtype": "float16", "implementation": name,
                                "stage": stage, "workspace_bytes": workspace.workspace_bytes,
                                **measure(function, warmup, repeats)})
        print(f"Benchmarked {case_id + 1}/{len(cases)}: T={tokens}, H={hidden}, E={experts}, {pattern}",
              flush=True)
    return configurations, records


@torch.inference_mode()
def transport_moe_check(extension):
    """A SwiGLU top-2 MoE feed-forward behind the HIP transport, checked two ways.

    Experts run with torch matmuls on the packed rows behind the PyTorch
    transport and behind the HIP transport (vectorized, alignment 8, bf16
    rows); the HIP result must match the PyTorch-transport result, and a
    token-major evaluation that uses no transport at all. It is stored as the
    record's ``block_demo`` entry (a functional gate, no speed claim).
    """
    from .reference import TorchWorkspace
    from .workspace import CudaWorkspace

    tokens, hidden, inter, experts, topk = 96, 256, 384, 8, 2
    g = torch.Generator(device="cuda").manual_seed(11)
    x = torch.randn(tokens, hidden, device="cuda", generator=g).bfloat16()
    logits = torch.randn(tokens, experts, device="cuda", generator=g)
    top, ids64 = torch.topk(logits, topk, dim=-1)
    weights = torch.softmax(top, dim=-1).contiguous()
    ids32 = ids64.to(torch.int32).contiguous()
    gate_up = (torch.randn(experts, 2 * inter, hidden, device="cuda", generator=g) / hidden**0.5).bfloat16()
    down = (torch.randn(experts, hidden, inter, device="cuda", generator=g) / inter**0.5).bfloat16()

    def expert(e, rows):
        projection = (rows.float() @ gate_up[e].float().t()).bfloat16().float()
        activation = (torch.nn.functional.silu(projection[:, :inter]) * projection[:, inter:]).bfloat16()
        return (activation.float() @ down[e].float().t()).bfloat16()

    def through(workspace):
        workspace.dispatch(x, ids32, ids64)
        out = torch.zeros_like(workspace.packed)
        starts = workspace.offsets.cpu().tolist()  # host read: functional check only
        counts = workspace.counts.cpu().tolist()
        for e in range(experts):
            if counts[e]:
                rows = slice(starts[e], starts[e] + counts[e])
                out[rows] = expert(e, workspace.packed[rows])
        workspace.combine(out, weights)
        return workspace.output.float().clone()

    via_torch = through(TorchWorkspace(tokens, hidden, experts, topk, x.dtype, alignment=8))
    via_hip = through(CudaWorkspace(tokens, hidden, experts, topk, x.dtype, extension=extension, alignment=8))
    torch.testing.assert_close(via_hip, via_torch, atol=0, rtol=0)
    token_major = torch.zeros(tokens, hidden, device="cuda")
    for e in range(experts):
        share = (weights * (ids64 == e)).sum(1, keepdim=True)
        token_major += expert(e, x).float() * share
    torch.testing.assert_close(via_hip, token_major, atol=2e-2, rtol=2e-2)
    return {"passed": True, "tokens": tokens, "hidden": hidden, "intermediate": inter, "experts": experts,
            "topk": topk, "output_shape": list(via_hip.shape),
            "max_absolute_error": float((via_hip - token_major).abs().max()),
            "benchmark_note": "functional SwiGLU MoE behind the transport; no block/model speedup claimed"}


def run_transport_benchmark(output, suite="smoke", warmup=10, repeats=40, extension=None):
    """Correctness suite, demo block, then the timed suite; writes and re-checks ``results.json``."""
    if warmup < 1 or repeats < 5:
        raise ValueError("use warmup>=1 and repeats>=5")
    from ._extension import get_extension
    from .validation import run_tests

    extension = extension or get_extension()
    correctness = run_tests(extension)
    demo = transport_moe_check(extension)
    configurations, records = benchmark(extension, suite, warmup, repeats)
    result = {
        "kind": "transport_benchmark",
        "hardware": hardware_metadata(),
        "correctness": correctness,
        "block_demo": demo,
        "configurations": configurations,
        "benchmarks": records,
        "source_hashes": source_hashes(),
        "method": {
            "suite": suite, "warmup": warmup, "repeats": repeats, "seed": 100,
            "timing": "hipEvent elapsed time on the launch stream; one sample per call after warmup; "
                      "workspaces reused; the count/offset pass is inside every dispatch sample. Input "
                      "generation and validation are excluded. Small cases include launch gaps.",
            "scope": "Dispatch/combine transport only: FP16 rows, FP32 weighted accumulation. The PyTorch "
                     "transport is compared with the scalar and vectorized HIP paths.",
        },
    }
    output = Path(output)
    output.mkdir(parents=True, exist_ok=True)
    (output / "results.json").write_text(json.dumps(result, indent=2))
    read_results(output / "results.json")
    return result
