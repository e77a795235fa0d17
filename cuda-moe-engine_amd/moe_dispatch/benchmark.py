"""Timing helpers: hipEvent timing on the current stream and linear-interpolation percentiles.

Restates ``percentile`` and ``measure`` (reference ``src/moe_dispatch/benchmark.py:15-45``).
"""

import math
import statistics

import torch


def percentile(values, fraction):
    ordered = sorted(values)
    if not ordered:
        return 0.0
    position = (len(ordered) - 1) * fraction
    lower, upper = math.floor(position), math.ceil(position)
    return ordered[lower] + (ordered[upper] - ordered[lower]) * (position - lower)


@torch.inference_mode()
def measure(function, warmup, repeats):
    """Warm up, then time each call with a pair of events on the current stream (µs)."""
    for _ in range(warmup):
        function()
    torch.cuda.synchronize()
    events = [
        (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
        for _ in range(repeats)
    ]
    for start, end in events:
        start.record()
        function()
        end.record()
    torch.cuda.synchronize()
    values_us = [start.elapsed_time(end) * 1000.0 for start, end in events]
    return {
        "median_us": statistics.median(values_us),
        "p95_us": percentile(values_us, 0.95),
        "min_us": min(values_us),
        "samples_us": values_us,
    }
