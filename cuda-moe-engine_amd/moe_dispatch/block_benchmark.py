"""Block benchmark driver (raw samples, forward validation) and graph capture of the forward.

``run_block_benchmark`` writes the evidence record ``block_results.json`` checked by
``moe_dispatch.evidence.validate_block``.

Graph capture and replay of the MoE block forward:

Mirrors ``capture_forward`` of the reference (``src/moe_dispatch/block_benchmark.py:48-64``):
warm up on a side stream, capture one ``block(x)`` into a graph (a hipGraph under
ROCm), replay it once and require the replay to reproduce the eager output. The
graph leaves the router weights' split out (see ``ForwardGraph``).
The reference accepts rtol = atol = 3e-2 here; every kernel of this package is
deterministic, so the replay must match the eager forward bit for bit.

Capture is legal because the forward never synchronises the host, never reads
device values on the host, allocates nothing after the first call for a given
token count (workspaces are cached), launches every kernel on the current
stream and records no memset node.
"""

from __future__ import annotations

import torch


class ForwardGraph:
    """A captured ``block(x)``: ``replay()`` runs it again on the current stream.

    For ``cuda_fused`` blocks the graph reads the router weights' bf16 split
    from the block's scratch instead of recomputing it (one kernel fewer per
    replay); ``replay()`` first redoes the split, outside the graph, when the
    router weights were replaced or written in place since the split was
    taken, so every replay routes with the weights as they are. ``graph`` is
    the underlying ``torch.cuda.CUDAGraph`` (the object the reference's
    ``capture_forward`` returns); replaying it directly skips that check, so
    after a router-weight update it routes with the split taken before. The
    graph's own ``reset()``, ``pool()`` and ``enable_debug_mode()`` pass through.
    """

    def __init__(self, block, graph, output):
        self.block = block
        self.graph = graph
        self.output = output

    def reset(self):
        self.graph.reset()

    def pool(self):
        return self.graph.pool()

    def enable_debug_mode(self):
        self.graph.enable_debug_mode()

    def replay(self):
        block = self.block
        if block.implementation == "cuda_fused" and block._router_scratch is not None:
            key = block._router_split_key()
            if not block._same_split(key, block._router_split_of):
                block._extension.router_split_out(block.router_weight, block._router_scratch)
                block._router_split_of = key
        self.graph.replay()


@torch.inference_mode()
def capture_forward(block, x, warmup=3):
    """Capture ``block(x)`` into a graph (a hipGraph under ROCm); raises if the replay differs.

    Returns a ``ForwardGraph``. The graph reads ``x`` and writes
    ``block.workspace(x).transport.output`` (the tensor ``block(x)`` returns);
    keep ``x`` alive and update it in place to feed new tokens of the same shape.
    """
    expected = block(x).clone()
    device = x.device
    stream = torch.cuda.Stream(device=device)
    stream.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(stream):
        for _ in range(warmup):
            block(x)
    torch.cuda.current_stream(device).wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    block._split_in_capture = False
    try:
        with torch.cuda.graph(graph, stream=stream):
            output = block(x)
    finally:
        block._split_in_capture = True
    forward = ForwardGraph(block, graph, output)
    forward.replay()
    torch.cuda.synchronize(device)
    if not torch.equal(output, expected):
        raise RuntimeError("graph replay differs from the eager forward")
    return forward


IMPLEMENTATIONS = ("torch", "cuda", "cuda_fused")


def workload_cases(suite):
    """(tokens, MoEConfig, pattern) per case.

    ``smoke``, ``quick`` and ``model`` are the reference's suites
    (``src/moe_dispatch/block_benchmark.py:15-26``); ``baseline`` adds this
    build's headline shapes: C1, C3 at T=4096, C4 at T = 1, 16 and 4096.
    """
    from .layer import MoEConfig

    if suite == "smoke":
        return [(128, MoEConfig(), pattern) for pattern in ("balanced", "skewed")]
    if suite == "model":
        config = MoEConfig(hidden=4096, intermediate=14336, experts=8, topk=2)
        return [(128, config, "balanced"), (256, config, "skewed")]
    if suite == "quick":
        return [(tokens, config, pattern) for tokens in (128, 2048)
                for config in (MoEConfig(), MoEConfig(1024, 2048, 16, 2))
                for pattern in ("balanced", "skewed")]
    if suite == "baseline":
        c4 = MoEConfig(hidden=4096, intermediate=14336, experts=8, topk=2)
        return [(128, MoEConfig(), "balanced"), (4096, MoEConfig(1024, 2048, 16, 2), "balanced"),
                (1, c4, "balanced"), (16, c4, "balanced"), (4096, c4, "balanced")]
    raise ValueError("suite must be smoke, quick, model or baseline")


@torch.inference_mode()
def check_forward(block, x, rtol=0.03, atol=0.03, relative_l2_limit=0.02):
    """Forward vs the dense token-major evaluation at the reference's gate.

    The gate is the reference's (``block_benchmark.py:29-45``: allclose at
    rtol = atol = 3e-2, relative L2 at most 2e-2); the errors are recorded.
    """
    from .layer import token_major_oracle

    actual = block(x).clone()
    expected = token_major_oracle(block, x)
    torch.testing.assert_close(actual, expected, rtol=rtol, atol=atol)
    difference = actual.float() - expected.float()
    relative = float(difference.norm() / expected.float().norm().clamp_min(1e-8))
    if relative > relative_l2_limit:
        raise AssertionError(f"relative L2 error {relative} exceeds {relative_l2_limit}")
    return {"passed": True, "max_absolute_error": float(difference.abs().max()),
            "relative_l2_error": relative, "rtol": rtol, "atol": atol,
            "relative_l2_limit": relative_l2_limit}


def _persistent_bytes(block, state):
    tensors = [state.projection, state.activated, state.expert_output]
    tensors += [t for buffers in block._route_buffers.values() for t in buffers]
    if block._router_scratch is not None:
        tensors.append(block._router_scratch)
    return state.transport.workspace_bytes + sum(t.numel() * t.element_size() for t in tensors)


@torch.inference_mode()
def run_block_benchmark(suite="smoke", expert_backend="auto", warmup=10, repeats=40, output="runs/block",
                        graphs=False):
    """Validate, then time router / dispatch / experts / combine / forward for every implementation.

    Writes ``block_results.json`` (the reference's record, ``block_benchmark.py:186-210``)
    with raw samples, checks it with ``moe_dispatch.evidence.validate_block`` and
    returns it. Weights use seed 42 + case, activations 100 + case; the order of
    the implementations rotates per case.
    """
    from dataclasses import asdict
    from pathlib import Path
    import json

    from .benchmark import hardware_metadata, measure
    from .evidence import source_hashes, validate_block
    from .layer import MoEBlock, make_weights

    if not torch.cuda.is_available():
        raise RuntimeError("the block benchmark needs an AMD GPU")
    if warmup < 1 or repeats < 5:
        raise ValueError("use warmup>=1 and repeats>=5")
    configurations, validation, records = [], [], []
    backend_used = None
    cases = workload_cases(suite)
    for case_id, (tokens, config, pattern) in enumerate(cases):
        weights = make_weights(config, "cuda", torch.bfloat16, 42 + case_id)
        generator = torch.Generator(device="cuda").manual_seed(100 + case_id)
        x = torch.randn(tokens, config.hidden, device="cuda", generator=generator).bfloat16()
        blocks = {}
        for name in IMPLEMENTATIONS:
            backend = expert_backend if name == "torch" else "hip"
            blocks[name] = MoEBlock(config, device="cuda", implementation=name, expert_backend=backend,
                                    weights=weights)
            blocks[name].set_routing_pattern(pattern)
        backend_used = blocks["torch"].expert_backend
        ids32, ids64, probabilities = blocks["torch"].route(x)
        counts = torch.bincount(ids64.flatten(), minlength=config.experts).cpu().tolist()
        configurations.append({"case_id": case_id, "tokens": tokens, **asdict(config), "pattern": pattern,
                               "dtype": "bfloat16", "expert_backend": backend_used, "expert_counts": counts})
        names = list(IMPLEMENTATIONS)
        names = names[case_id % len(names):] + names[: case_id % len(names)]
        for name in names:
            block = blocks[name]
            checked = check_forward(block, x)
            validation.append({"case_id": case_id, "implementation": name, **checked})
            state = block.workspace(x)
            state.transport.dispatch(x, ids32, ids64)
            block.experts_forward(state)
            stages = (
                ("router", lambda: block.route(x)),
                ("dispatch", lambda: state.transport.dispatch(x, ids32, ids64)),
                ("experts", lambda: block.experts_forward(state)),
                ("combine", lambda: state.transport.combine(state.expert_output, probabilities)),
                ("forward", lambda: block(x)),
            )
            persistent = _persistent_bytes(block, state)
            for stage, function in stages:
                records.append({"case_id": case_id, "implementation": name, "stage": stage,
                                "persistent_workspace_bytes": persistent, **measure(function, warmup, repeats)})
            if graphs:
                try:
                    graph = capture_forward(block, x)
                    records.append({"case_id": case_id, "implementation": name, "stage": "forward_graph",
                                    "persistent_workspace_bytes": persistent,
                                    **measure(graph.replay, warmup, repeats)})
                    checked["graph_status"] = "passed"
                except RuntimeError as error:
                    checked["graph_status"] = "unsupported"
                    checked["graph_error"] = str(error)
                validation[-1].update(checked)
        print(f"MoE block {case_id + 1}/{len(cases)}: T={tokens}, H={config.hidden}, I={config.intermediate}, "
              f"E={config.experts}, K={config.topk}, {pattern}", flush=True)
    result = {
        "kind": "moe_block_benchmark",
        "package_version": "0.1.0",
        "hardware": hardware_metadata(),
        "source_hashes": source_hashes(),
        "configurations": configurations,
        "validation": validation,
        "benchmarks": records,
        "method": {
            "suite": suite, "warmup": warmup, "repeats": repeats, "expert_backend": backend_used,
            "graphs_requested": graphs,
            "scope": "One synthetic MoE feed-forward block: fp32 router, top-k and softmax; bf16 grouped "
                     "gate/up GEMM; SwiGLU in fp32 with one bf16 cast; bf16 grouped down GEMM; fp32 weighted "
                     "combine. The three implementations share weights; expert_backend names the torch "
                     "implementation's GEMM, while cuda and cuda_fused run the HIP grouped GEMMs (cuda_fused "
                     "with SwiGLU in the gate/up epilogue and the fused router). Not a full language model.",
            "timing": "hipEvent elapsed time on the launch stream after warmup, one sample per call. The "
                      "experts stage is both GEMMs and the activation; stages are timed in isolation and "
                      "need not sum to the forward. Validation and compilation are excluded; eager samples "
                      "can include host launch gaps. Graph replay timings are separate rows.",
        },
    }
    output = Path(output)
    output.mkdir(parents=True, exist_ok=True)
    (output / "block_results.json").write_text(json.dumps(result, indent=2))
    validate_block(result)
    print(f"Saved {output}/block_results.json", flush=True)
    return result
