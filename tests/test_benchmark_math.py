"""Sample statistics of the timing records (median, p95 by linear interpolation, min)."""

import statistics

import pytest

from moe_dispatch.benchmark import percentile, sample_statistics


def test_percentile_interpolates_between_closest_ranks():
    # 11 evenly spaced samples: rank (n-1)*q lands exactly on a sample
    samples = [float(v) for v in range(100, 0, -10)] + [0.0]
    assert percentile(samples, 0.5) == pytest.approx(50.0)
    assert percentile(samples, 0.95) == pytest.approx(95.0)  # halfway between 90 and 100
    assert percentile(samples, 0.0) == 0.0 and percentile(samples, 1.0) == 100.0
    # two samples: the fraction itself interpolates
    assert percentile([2.0, 6.0], 0.25) == pytest.approx(3.0)


def test_percentile_of_degenerate_inputs():
    assert percentile([3.5], 0.95) == 3.5
    assert percentile([], 0.5) == 0.0
    assert percentile([5, 5, 5], 0.95) == 5


def test_sample_statistics_agree_with_the_standard_library():
    samples = [12.0, 9.5, 30.25, 11.0, 10.5, 9.75]
    stats = sample_statistics(samples)
    assert stats["median_us"] == statistics.median(samples)
    assert stats["min_us"] == 9.5
    ordered = sorted(samples)
    rank = 0.95 * (len(samples) - 1)  # 4.75: between the 5th and 6th smallest
    assert stats["p95_us"] == pytest.approx(ordered[4] + 0.75 * (ordered[5] - ordered[4]))
