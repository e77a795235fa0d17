"""bench.py on the CPU: it imports, refuses more than one GPU, and reads counter traffic."""

import json
import subprocess
import sys
from pathlib import Path

import bench

ROOT = Path(__file__).resolve().parents[1]


def test_bench_refuses_multi_gpu():
    proc = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True,
                          text=True, timeout=120)
    assert proc.returncode == 2
    assert "one GPU" in json.loads(proc.stdout.strip())["error"]


def test_bench_configs_and_defaults():
    args = bench.parse_args([])
    assert args.gpus == 1 and args.config == "c4_t4096"
    assert bench.CONFIGS["c4_t4096"][:5] == (4096, 4096, 14336, 8, 2)
    assert bench.TRANSPORT_CONFIGS["c2_transport"] == (4096, 2048, 8, 2, 1)
    assert bench.parse_args(["--config", "c2_transport"]).config == "c2_transport"


def test_measured_traffic_sums_kernels(tmp_path, monkeypatch):
    table = {"cfg": {"a": {"fetch_bytes": 10, "write_bytes": 5}, "b": {"fetch_bytes": 1, "write_bytes": 2}}}
    path = tmp_path / "traffic.json"
    path.write_text(json.dumps(table))
    monkeypatch.setattr(bench, "TRAFFIC_FILE", path)
    assert bench.measured_traffic("cfg", ("a",)) == 15
    assert bench.measured_traffic("cfg", ("a", "b")) == 18
    assert bench.measured_traffic("cfg", ("missing",)) is None
    assert bench.measured_traffic("other", ("a",)) is None


def test_committed_traffic_table_covers_the_bench_kernels():
    table = json.loads((ROOT / "profiles" / "hbm_traffic.json").read_text())
    assert "grouped_gemm_persistent_kernel<true, false>" in table["c4_t4096"]
    assert {"count_rank_kernel", "pack_kernel<16, false, false>"} <= set(table["c2_transport"])


def test_gateup_roofline_picks_the_bound_by_intensity():
    import numpy as np

    h, i = 4096, 14336
    # Decode: one token on two experts streams 2 x (2I x H) bf16 weights for 4*2*H*I flop.
    dec = bench.gateup_roofline("none", np.array([1, 0, 0, 0, 0, 1, 0, 0]), 58, h, i, 2, 4.0 * 2 * h * i, 100.0)
    weights = 2 * 2 * (2 * i * h)
    assert dec["bound"] == "hbm" and dec["unit"] == "GB/s" and dec["peak"] == bench.HBM_PEAK_GBS
    assert dec["kernel"].startswith("grouped_gemm_decode_kernel<true, 64, false>")
    assert weights < dec["bytes_per_launch"] < weights * 1.001
    assert abs(dec["achieved"] - dec["bytes_per_launch"] / 100e-6 / 1e9) < 0.1
    # Prefill: 8192 assignments over 8 experts is far past the ridge point.
    pre = bench.gateup_roofline("none", np.array([1024] * 8), 8248, h, i, 8192, 4.0 * 8192 * h * i, 1000.0)
    assert pre["bound"] == "mfma" and pre["unit"] == "TFLOP/s"
    assert pre["kernel"].startswith("grouped_gemm_persistent_kernel<true, false>")
    gathered = bench.gateup_roofline("none", np.array([1024] * 8), 8248, h, i, 8192, 1.0, 1.0, gathered=True)
    assert gathered["kernel"].startswith("grouped_gemm_persistent_kernel<true, true>")
    assert abs(pre["achieved"] - 4.0 * 8192 * h * i / 1e-3 / 1e12) < 0.1
    assert list(pre)[0] == "bound"
    # 320 rows over 8 experts (T=128, H=512, I=1024): 64 wide tiles for 256 CUs, so
    # the launcher takes the weight-streaming kernel; with 32 CUs the wide one.
    c1 = (np.array([32] * 8), 320, 512, 1024, 256, 4.0 * 256 * 512 * 1024, 10.0)
    assert bench.gateup_roofline("none", *c1, cus=256)["kernel"].startswith("grouped_gemm_decode_kernel<true, 128, ")
    assert bench.gateup_roofline("none", *c1, cus=32)["kernel"].startswith("grouped_gemm_persistent_kernel<true, ")


def test_byte_models_and_workload_bias_equal_the_oracle():
    """bench.py's own byte models and the Zipf bias generator (product side) equal the oracle's."""
    import numpy as np

    from moe_dispatch.routing import zipf_bias
    from oracle import moe_oracle as oracle

    for args in ((4096, 2048, 2, 0), (4096, 4096, 2, 64), (8192, 2048, 6, 456), (1, 4096, 2, 14)):
        assert bench.dispatch_bytes(*args) == oracle.dispatch_bytes(*args)
        assert bench.combine_bytes(*args[:3]) == oracle.combine_bytes(*args[:3])
    for experts in (8, 64):
        np.testing.assert_array_equal(zipf_bias(experts).numpy(), oracle.zipf_bias(experts))


def test_cpu_baseline_times_the_torch_variant_at_config_1(monkeypatch):
    """The CPU baseline leg runs the PyTorch variant at benchmark config 1 (T=128, H=512; shortened here)."""
    import torch

    calls = []
    real = bench._time_cpu

    def quick(fn, warmup, samples):
        calls.append((warmup, samples))
        return real(fn, 1, 2)

    monkeypatch.setattr(bench, "_time_cpu", quick)
    threads = torch.get_num_threads()
    out = bench.cpu_baseline()
    assert torch.get_num_threads() == threads  # restored
    assert calls == [(10, 40), (10, 40)]
    assert out["kind"] == "port" and out["unit"] == "us" and out["value"] == out["all_cores"]["median_us"]
    assert out["one_thread"]["threads"] == 1 and out["cores"] == out["all_cores"]["threads"] >= 1
    assert out["config"] == {"tokens": 128, "hidden": 512, "intermediate": 1024, "experts": 8, "topk": 2,
                             "dtype": "bf16"}
    assert out["cpu_model"] and out["torch_version"] == torch.__version__
