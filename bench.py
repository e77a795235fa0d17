"""MoE block forward benchmark on one MI355X (implementation="cuda_fused").

Workload (the headline metric's configuration): H=4096, I=14336, E=8, top-2,
T=4096 tokens, bf16 x ~ N(0,1), random-init weights of that architecture
(router fp32 ~ N(0,1/H), gate_up/down bf16 ~ N(0,1/fan_in)), zero router bias.
Inputs and weights are resident in HBM before timing starts.

Prints ONE JSON line: value = mean forward latency (us) over the timed steps,
plus per-stage latencies, expert-GEMM TFLOP/s, dispatch/combine GB/s, the
roofline of the dominant kernel (gate/up GEMM with the SwiGLU epilogue, timed
with events on the stream it is launched on), the PyTorch variant on the same
GPU, and a CPU baseline: the same PyTorch variant on the host CPU at the
reference's CPU-runnable configuration (T=128, H=512, I=1024, E=8, top-2; all
cores and one thread), plus a token sample of this workload.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT / "cuda-moe-engine_amd", ROOT):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0

CONFIGS = {
    # name: (tokens, hidden, intermediate, experts, topk, pattern)
    "c4_t4096": (4096, 4096, 14336, 8, 2, "balanced"),
    "c4_t16": (16, 4096, 14336, 8, 2, "balanced"),
    "c4_t1": (1, 4096, 14336, 8, 2, "balanced"),
    "c1": (128, 512, 1024, 8, 2, "balanced"),
    "c3_t4096": (4096, 1024, 2048, 16, 2, "balanced"),
    "c5": (8192, 2048, 1408, 64, 6, "zipf"),
}
# Standalone transport (dispatch + combine only): tokens, hidden, experts, topk, alignment.
TRANSPORT_CONFIGS = {"c2_transport": (4096, 2048, 8, 2, 1)}
# HBM bytes per launch from rocprofv3 FETCH_SIZE / WRITE_SIZE runs, scaled by the
# same counters read on a copy of known size (written next to the kernel summaries).
TRAFFIC_FILE = ROOT / "profiles" / "hbm_traffic.json"


def dispatch_bytes(tokens, hidden, topk, padding_rows, elem=2):
    """Algorithmic dispatch bytes: x read once, each assignment's row and the
    padding rows written once, the ids read and the inverse map written (4 B each)."""
    n = tokens * topk
    return (tokens + n + padding_rows) * hidden * elem + n * 8


def combine_bytes(tokens, hidden, topk, elem=2):
    """Algorithmic combine bytes: K rows gathered per token, one row written, the
    inverse map and the weights read (4 B each)."""
    n = tokens * topk
    return (n + tokens) * hidden * elem + n * 8


def parse_args(argv=None):
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    # The GPU's clock settles over its first ~15 GEMM launches (the second is the
    # slowest, about 35% above the steady state); 15 untimed forwards pass that.
    ap.add_argument("--warmup", type=int, default=15)
    ap.add_argument("--config", default="c4_t4096", choices=sorted(CONFIGS) + sorted(TRANSPORT_CONFIGS))
    ap.add_argument("--copy-calibration", action="store_true",
                    help="time a 1 GiB device-to-device copy (the counter scale for traffic)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-torch-variant", action="store_true")
    ap.add_argument("--no-graph", action="store_true", help="skip the hipGraph replay timing")
    ap.add_argument("--gemm-study", action="store_true",
                    help="time the expert GEMMs beside hipBLASLt, a dense one-expert problem and zero weights")
    ap.add_argument("--cpu-sample-tokens", type=int, default=64,
                    help="tokens of the benchmark workload the CPU variant also runs (0: config 1 only)")
    return ap.parse_args(argv)


def _events(n):
    import torch

    return [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]


def time_loop(fn, steps, warmup):
    """Mean time of one call (us): `steps` back-to-back calls between two events on the
    current stream (the stream every kernel of this package is launched on)."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(steps):
        fn()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) * 1000.0 / steps


def time_graph(fn, reps, warmup):
    """Mean GPU time of one fn() call: `reps` back-to-back calls captured in a
    HIP graph and replayed (no host launch overhead in the measurement)."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            for _ in range(reps):
                fn()
    torch.cuda.current_stream().wait_stream(stream)
    graph.replay()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    graph.replay()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) * 1000.0 / reps


def time_stages(block, x, steps, warmup):
    """Per-stage GPU time: the forward's own C-ABI calls (the block's pre-bound
    launches, router split already done), each repeated back to back in a graph
    (every stage is idempotent given the previous stage's outputs)."""
    import torch

    with torch.inference_mode():
        block(x)  # a validated forward binds the launches; the next ones reuse them
        launches = block._launches[(x.shape[0], x.device)]
        assert launches.still_valid(block)
        stages = launches.stage_calls(x)
        return {name: {"mean_us": time_graph(fn, steps, warmup)} for name, fn in stages.items()}


def _cpu_model():
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:  # pragma: no cover
        pass
    import platform

    return platform.processor() or "unknown"


def _host_threads():
    """CPUs this process may run on (the box's share, not the whole host), capped by OMP_NUM_THREADS."""
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        avail = os.cpu_count() or 1
    cap = os.environ.get("OMP_NUM_THREADS")
    return min(avail, int(cap)) if cap and cap.isdigit() and int(cap) > 0 else avail


def _time_cpu(fn, warmup, samples):
    """perf_counter_ns around each call after `warmup` untimed calls: median/p95/min in us."""
    from moe_dispatch.evidence import percentile

    for _ in range(warmup):
        fn()
    values = []
    for _ in range(samples):
        t0 = time.perf_counter_ns()
        fn()
        values.append((time.perf_counter_ns() - t0) / 1000.0)
    return {"median_us": round(statistics.median(values), 2), "p95_us": round(percentile(values, 0.95), 2),
            "min_us": round(min(values), 2), "samples": samples, "warmup": warmup}


def cpu_baseline(gpu_block=None, gpu_x=None, c4_sample_tokens=64):
    """The PyTorch variant (implementation="torch", F.grouped_mm) on the host CPU.

    Main figure: the reference's CPU-runnable configuration (T=128, H=512, I=1024, E=8, top-2, bf16, seed 0),
    every token, 10 warm-ups + 40 perf_counter_ns samples, with all the CPUs this
    process may use and again with 1 thread. When the benchmark's own block is
    given, the same variant also runs on its first `c4_sample_tokens` tokens with
    its weights (copied to the host), reported per token and scaled to the full
    token count (labelled as such: the weights are streamed once per call, so a
    small sample over-weights that cost).
    """
    import torch

    from moe_dispatch.layer import MoEBlock, MoEConfig, make_weights

    threads_before = torch.get_num_threads()
    threads = _host_threads()
    cfg = MoEConfig(512, 1024, 8, 2)
    weights = make_weights(cfg, "cpu", torch.bfloat16, seed=0)
    block = MoEBlock(cfg, device="cpu", dtype=torch.bfloat16, implementation="torch", weights=weights)
    x = torch.randn(128, 512, generator=torch.Generator().manual_seed(0)).bfloat16()
    runs = {}
    try:
        for label, n in (("all_cores", threads), ("one_thread", 1)):
            torch.set_num_threads(n)
            runs[label] = {"threads": n, **_time_cpu(lambda: block(x), 10, 40)}
        result = {
            "value": runs["all_cores"]["median_us"],
            "unit": "us",
            "cores": threads,
            "kind": "port",
            "workload": "c1_t128",
            "sample": "C1 (T=128 H=512 I=1024 E=8 top-2 bf16), not the bench workload: this repo's PyTorch "
                      "variant of the reference block (implementation='torch': topk/softmax router, stable-sort "
                      "transport, F.grouped_mm experts, fp32 combine), seed 0, all 128 tokens, no scaling; median "
                      "of 40 perf_counter_ns samples after 10 warm-ups",
            "config": {"tokens": 128, "hidden": 512, "intermediate": 1024, "experts": 8, "topk": 2,
                       "dtype": "bf16"},
            "all_cores": runs["all_cores"],
            "one_thread": runs["one_thread"],
            "cpu_model": _cpu_model(),
            "host_cpu_count": os.cpu_count(),
            "torch_version": torch.__version__,
        }
        if gpu_block is not None and c4_sample_tokens > 0:
            torch.set_num_threads(threads)
            bcfg = gpu_block.config
            host_w = type(weights)(gpu_block.router_weight.cpu(), gpu_block.gate_up_weight.cpu(),
                                   gpu_block.down_weight.cpu())
            host = MoEBlock(bcfg, device="cpu", dtype=torch.bfloat16, implementation="torch", weights=host_w)
            host.routing_bias.copy_(gpu_block.routing_bias.cpu())
            xs = gpu_x[:c4_sample_tokens].cpu()
            timing = _time_cpu(lambda: host(xs), 1, 3)
            total = gpu_x.shape[0]
            result["bench_workload_sample"] = {
                "tokens": c4_sample_tokens, "of_tokens": total, "threads": threads, **timing,
                "scaled_us": round(timing["median_us"] * total / c4_sample_tokens, 1),
                "note": "same variant on the first tokens of the benchmark workload, median scaled linearly "
                        "to the full token count",
            }
            del host, host_w
        return result
    finally:
        torch.set_num_threads(threads_before)


def torch_variant_gpu(cfg, weights, x, steps, warmup):
    import torch

    from moe_dispatch.benchmark import measure
    from moe_dispatch.experts import backend_label, torch_backend_calls
    from moe_dispatch.layer import MoEBlock

    block = MoEBlock(cfg, device=x.device, implementation="torch", expert_backend="torch", weights=weights)
    before = torch_backend_calls.copy()
    stats = measure(lambda: block(x), warmup, steps)
    # The path of the timed calls themselves (warm-up and timed forwards).
    kind = backend_label(before, torch_backend_calls)
    del block
    torch.cuda.empty_cache()
    return {"median_us": stats["median_us"], "min_us": stats["min_us"], "gemm_backend": kind}


def measured_traffic(config, kernels):
    """Scaled HBM bytes per launch of `kernels` at `config`, if a counter run recorded them."""
    try:
        table = json.loads(TRAFFIC_FILE.read_text())
    except (OSError, ValueError):
        return None
    total = 0
    for kernel in kernels:
        entry = table.get(config, {}).get(kernel)
        if not entry:
            return None
        total += entry.get("fetch_bytes", 0) + entry.get("write_bytes", 0)
    return total


def gateup_roofline(config, counts, packed_rows, hidden, inter, n_assign, flop, launch_us, cus=None,
                    gathered=False):
    """Roofline entry for the gate/up GEMM + SwiGLU launch.

    Algorithmic bytes per launch: the weights of the experts that hold rows
    (2I x H bf16 each), the packed activations read once (rows x H bf16) and the
    activated output written once (assignments x I bf16). When flop/byte is below
    the MI355X ridge point (2500 TFLOP/s / 8 TB/s = 312.5) the launch is bound by
    HBM and the entry is in GB/s; otherwise by the bf16 MFMA peak, in TFLOP/s.
    The kernel is the one the launcher picks (``launch_gemm_t`` in
    ``csrc/gemm.hip``): the weight-streaming (decode) kernel when the buffer
    has at most 128 rows, or at most 128 per expert while the 256 x 256 tiles
    (rows spread evenly over the experts) would number fewer than the CUs
    (``cus``; default: the current GPU's, 256 without one). ``gathered``: the
    forward's gate/up GEMM read its rows from x through the row table (the
    kernels' GATHER instances).
    """
    import torch

    def ceil_div(a, b):
        return -(-a // b)

    experts = len(counts)
    active = int((counts > 0).sum())
    byte = 2.0 * (active * 2 * inter * hidden + n_assign * hidden + n_assign * inter)
    if cus is None:
        cus = torch.cuda.get_device_properties(0).multi_processor_count if torch.cuda.is_available() else 256
    wide_tiles = experts * ceil_div(ceil_div(packed_rows, experts), 256) * ceil_div(inter, 128)
    decode = hidden % 64 == 0 and (packed_rows <= 128 or (packed_rows <= 128 * experts and wide_tiles < cus))
    g = "true" if gathered else "false"
    if decode:
        kernel = f"grouped_gemm_decode_kernel<true, {64 if packed_rows <= 64 else 128}, {g}>"
    else:
        kernel = f"grouped_gemm_persistent_kernel<true, {g}>"
    entry = {"kernel": kernel + " (gate/up GEMM + SwiGLU epilogue)"}
    if flop / byte < BF16_PEAK_TFLOPS * 1e12 / (HBM_PEAK_GBS * 1e9):
        achieved = byte / (launch_us * 1e-6) / 1e9
        entry.update(bound="hbm", achieved=round(achieved, 1), peak=HBM_PEAK_GBS, unit="GB/s",
                     frac=round(achieved / HBM_PEAK_GBS, 4))
    else:
        achieved = flop / (launch_us * 1e-6) / 1e12
        entry.update(bound="mfma", achieved=round(achieved, 1), peak=BF16_PEAK_TFLOPS, unit="TFLOP/s",
                     frac=round(achieved / BF16_PEAK_TFLOPS, 4))
    entry.update(traffic=measured_traffic(config, (kernel,)), flop_per_launch=flop, bytes_per_launch=byte,
                 avg_launch_us=round(launch_us, 2))
    # "bound" first, as the contract lists it
    return {k: entry[k] for k in ("bound", "kernel", "achieved", "peak", "unit", "frac", "traffic",
                                  "flop_per_launch", "bytes_per_launch", "avg_launch_us")}


def copy_calibration(steps):
    """1 GiB device-to-device copy: reads and writes exactly 2^30 bytes per launch."""
    import torch

    n = 1 << 30
    src = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(2):
        dst.copy_(src)
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(steps):
        dst.copy_(src)
    e.record()
    torch.cuda.synchronize()
    us = s.elapsed_time(e) * 1000.0 / steps
    print(json.dumps({"copy_bytes_each_way": n, "avg_us": round(us, 2),
                      "gbs_read_plus_write": round(2 * n / (us * 1e-6) / 1e9, 1)}), flush=True)
    return 0


def transport_bench(args):
    """Standalone dispatch + combine (ops-level transport) on one GPU."""
    import torch

    from moe_dispatch.routing import make_transport_case
    from moe_dispatch.workspace import CudaWorkspace
    tokens, hidden, experts, topk, alignment = TRANSPORT_CONFIGS[args.config]
    torch.cuda.set_device(0)
    x, ids32, ids64, weights = make_transport_case(tokens, hidden, experts, topk, torch.bfloat16, seed=0)
    ws = CudaWorkspace(tokens, hidden, experts, topk, torch.bfloat16, alignment=alignment)
    y = torch.randn(ws.capacity_rows, hidden, device="cuda",
                    generator=torch.Generator(device="cuda").manual_seed(1)).bfloat16()
    torch.cuda.synchronize()
    # GPU time per call: back-to-back calls replayed from a HIP graph (the host
    # work of a Python call is about as long as these kernels).
    with torch.inference_mode():
        mean_us = time_graph(lambda: (ws.dispatch(x, ids32, ids64), ws.combine(y, weights)), args.steps,
                             max(args.warmup, 1))
        d_us = time_graph(lambda: ws.dispatch(x, ids32, ids64), args.steps, max(args.warmup, 1))
        c_us = time_graph(lambda: ws.combine(y, weights), args.steps, max(args.warmup, 1))
    pad_rows = int(ws.offsets[-1].item()) - tokens * topk
    disp_bytes = dispatch_bytes(tokens, hidden, topk, pad_rows)
    comb_bytes = combine_bytes(tokens, hidden, topk)
    d_gbs = disp_bytes / (d_us * 1e-6) / 1e9
    c_gbs = comb_bytes / (c_us * 1e-6) / 1e9
    traffic = measured_traffic(args.config, ("count_rank_kernel", "pack_kernel<16, false, false>"))
    result = {
        "metric": "MoE block fwd latency (us) + expert TFLOP/s % bf16 MFMA peak; dispatch GB/s",
        "value": round(mean_us, 2),
        "unit": "us",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(mean_us / 1000.0, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) rows, uniform random expert ids, softmax weights)",
        "config": {"workload": f"standalone dispatch+combine {args.config}: T={tokens} H={hidden} "
                               f"E={experts} top-{topk} alignment={alignment}",
                   "tokens": tokens, "hidden": hidden, "experts": experts, "topk": topk,
                   "alignment": alignment},
        "stages_us": {"dispatch": round(d_us, 2), "combine": round(c_us, 2)},
        "dispatch_gbs": round(d_gbs, 1),
        "combine_gbs": round(c_gbs, 1),
        "roofline": {
            "bound": "hbm",
            "kernel": "count_rank_kernel + pack_kernel (one dispatch call)",
            "achieved": round(d_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(d_gbs / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "bytes_per_launch": disp_bytes,
            "avg_launch_us": round(d_us, 2),
        },
    }
    print(json.dumps(result), flush=True)
    return 0


def gemm_study(block, x, args):
    """Expert GEMMs beside hipBLASLt and the same kernels on a dense problem (one JSON line).

    For the configuration's real routing: the gate/up (+ SwiGLU) and down grouped
    GEMMs (where the forward gathers the gate/up GEMM's rows from x, the packed
    gate/up GEMM on the packed copy of the same rows, then the gathered one);
    torch.matmul (hipBLASLt) on dense bf16 GEMMs of the same total shape
    (M = assignments); this build's kernels on one expert holding all M rows (no
    short row tiles); and the grouped GEMMs again with zero weights, which keeps
    the schedule and the data movement but not the multiplier activity. Run it
    under rocprofv3 --pmc to read the clock (GRBM_GUI_ACTIVE) and MFMA busy
    cycles of each launch; the kernels run in the order listed.
    """
    import torch

    cfg = block.config
    state = block.workspace(x)
    t = state.transport
    ext = block._extension
    n = x.shape[0] * cfg.topk
    h, i = cfg.hidden, cfg.intermediate
    steps, warm = args.steps, max(args.warmup, 3)
    flop_gu, flop_dn = 4.0 * n * h * i, 2.0 * n * h * i
    rows = {}

    def row(name, fn, flop):
        us = time_loop(fn, steps, warm)
        rows[name] = {"us": round(us, 2), "tflops": round(flop / (us * 1e-6) / 1e12, 1),
                      "mfma_frac": round(flop / (us * 1e-6) / 1e12 / BF16_PEAK_TFLOPS, 4)}

    with torch.inference_mode():
        block(x)
        gathered = block._launches[(x.shape[0], x.device)].gathered
        if gathered:
            # The forward wrote the row table only: the packed copy of the same
            # layout (same offsets) for the packed kernel.
            ids32, ids64, _ = block._route_buffers[(x.shape[0], x.device)]
            t.dispatch(x, ids32, ids64)
        row("gateup_swiglu", lambda: ext.gateup_swiglu_out(t.packed, block.gate_up_weight, t.offsets,
                                                           state.activated), flop_gu)
        if gathered:
            row("gateup_swiglu_gathered", lambda: ext.gateup_swiglu_gathered_out(
                x, t.row_src, block.gate_up_weight, t.offsets, state.activated), flop_gu)
        row("down", lambda: ext.grouped_gemm_out(state.activated, block.down_weight, t.offsets,
                                                 state.expert_output), flop_dn)
        gen = torch.Generator(device=x.device).manual_seed(3)
        a = torch.randn(n, h, device=x.device, generator=gen).bfloat16()
        b = torch.randn(2 * i, h, device=x.device, generator=gen).bfloat16()
        row("hipblaslt_gateup_shape", lambda: torch.matmul(a, b.t()), flop_gu)
        del b
        a2 = torch.randn(n, i, device=x.device, generator=gen).bfloat16()
        b2 = torch.randn(h, i, device=x.device, generator=gen).bfloat16()
        row("hipblaslt_down_shape", lambda: torch.matmul(a2, b2.t()), flop_dn)
        del a2, b2
        one = torch.tensor([0, n], device=x.device, dtype=torch.int32)
        act = torch.empty(n, i, device=x.device, dtype=torch.bfloat16)
        out = torch.empty(n, h, device=x.device, dtype=torch.bfloat16)
        gu1 = block.gate_up_weight[:1]
        dn1 = block.down_weight[:1]
        row("gateup_swiglu_one_expert", lambda: ext.gateup_swiglu_out(a, gu1, one, act), flop_gu)
        row("down_one_expert", lambda: ext.grouped_gemm_out(act, dn1, one, out), flop_dn)
        del a, act, out
        zero_gu = torch.zeros_like(block.gate_up_weight)
        row("gateup_swiglu_zero_weights", lambda: ext.gateup_swiglu_out(t.packed, zero_gu, t.offsets,
                                                                        state.activated), flop_gu)
        del zero_gu
        zero_dn = torch.zeros_like(block.down_weight)
        row("down_zero_weights", lambda: ext.grouped_gemm_out(state.activated, zero_dn, t.offsets,
                                                              state.expert_output), flop_dn)
        del zero_dn
    torch.cuda.synchronize()
    print(json.dumps({"gemm_study": args.config, "assignments": n, "hidden": h, "intermediate": i,
                      "experts": cfg.experts, "expert_counts": t.counts.tolist(), "steps": steps,
                      "warmup": warm, "rows": rows}), flush=True)
    return 0


def main(argv=None):
    args = parse_args(argv)
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; multi-GPU runs are out of scope",
                          "n_gpus": args.gpus}))
        return 2
    if args.copy_calibration:
        return copy_calibration(args.steps)
    if args.config in TRANSPORT_CONFIGS:
        return transport_bench(args)
    import numpy as np
    import torch

    from moe_dispatch.layer import MoEBlock, MoEConfig, make_weights
    from moe_dispatch.routing import zipf_bias

    tokens, hidden, inter, experts, topk, pattern = CONFIGS[args.config]
    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    cfg = MoEConfig(hidden, inter, experts, topk)
    weights = make_weights(cfg, device, torch.bfloat16, seed=0)
    block = MoEBlock(cfg, device=device, implementation="cuda_fused", weights=weights)
    if pattern == "zipf":
        block.set_routing_bias(zipf_bias(experts))
    gen = torch.Generator(device=device).manual_seed(0)
    x = torch.randn(tokens, hidden, device=device, generator=gen).bfloat16()
    if args.gemm_study:
        return gemm_study(block, x, args)

    with torch.inference_mode():
        for _ in range(args.warmup):
            block(x)
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        per_step = _events(args.steps)
        start.record()
        for i in range(args.steps):
            per_step[i][0].record()
            block(x)
            per_step[i][1].record()
        end.record()
        torch.cuda.synchronize()
    total_ms = start.elapsed_time(end)
    step_us = [s.elapsed_time(e) * 1000.0 for s, e in per_step]
    mean_us = total_ms * 1000.0 / args.steps

    stages = time_stages(block, x, args.steps, max(min(args.warmup, 3), 1))
    graph_us = None
    if not args.no_graph:
        from moe_dispatch.block_benchmark import capture_forward

        graph = capture_forward(block, x)
        graph_us = time_loop(graph.replay, args.steps, max(args.warmup, 1))
    counts = block.workspace(x).transport.counts.cpu().numpy()
    offsets = block.workspace(x).transport.offsets.cpu().numpy()
    n_assign = tokens * topk
    pad_rows = int(offsets[-1]) - n_assign
    gateup_flop = 4.0 * n_assign * hidden * inter
    down_flop = 2.0 * n_assign * hidden * inter
    t_gu = stages["gateup_swiglu"]["mean_us"]
    t_dn = stages["down"]["mean_us"]
    expert_tflops = (gateup_flop + down_flop) / ((t_gu + t_dn) * 1e-6) / 1e12
    disp_bytes = dispatch_bytes(tokens, hidden, topk, pad_rows)
    comb_bytes = combine_bytes(tokens, hidden, topk)

    result = {
        "metric": "MoE block fwd latency (us) + expert TFLOP/s % bf16 MFMA peak; dispatch GB/s",
        "value": round(mean_us, 2),
        "unit": "us",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(mean_us / 1000.0, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) activations, random-init weights of the named shape)",
        "config": {"workload": f"MoE block fwd {args.config}: T={tokens} H={hidden} I={inter} E={experts} "
                               f"top-{topk} {pattern} routing, implementation=cuda_fused",
                   "tokens": tokens, "hidden": hidden, "intermediate": inter, "experts": experts,
                   "topk": topk, "alignment": cfg.alignment},
        "median_step_us": round(statistics.median(step_us), 2),
        "forward_graph_us": round(graph_us, 2) if graph_us is not None else None,
        "stages_us": {k: round(v["mean_us"], 2) for k, v in stages.items()},
        "expert_tflops": round(expert_tflops, 1),
        "expert_mfma_frac": round(expert_tflops / BF16_PEAK_TFLOPS, 4),
        "dispatch_gbs": round(disp_bytes / (stages["dispatch"]["mean_us"] * 1e-6) / 1e9, 1),
        "combine_gbs": round(comb_bytes / (stages["combine"]["mean_us"] * 1e-6) / 1e9, 1),
        "expert_counts": counts.tolist(),
        "roofline": gateup_roofline(args.config, counts, block.workspace(x).transport.packed.shape[0],
                                    hidden, inter, n_assign, gateup_flop, t_gu,
                                    gathered=block._launches[(x.shape[0], x.device)].gathered),
    }
    if not args.no_torch_variant:
        try:
            result["torch_variant_gpu_us"] = torch_variant_gpu(cfg, weights, x, min(args.steps, 10), 2)
        except RuntimeError as exc:  # e.g. out of memory: report, do not hide
            result["torch_variant_gpu_us"] = {"error": str(exc)[:200]}
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(block, x, args.cpu_sample_tokens)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
