"""Graph capture and replay of the MoE block forward.

Mirrors ``capture_forward`` of the reference (``src/moe_dispatch/block_benchmark.py:48-64``):
warm up on a side stream, capture one ``block(x)`` into a graph (a hipGraph under
ROCm), replay it once and require the replay to reproduce the eager output.
The reference accepts rtol = atol = 3e-2 here; every kernel of this package is
deterministic, so the replay must match the eager forward bit for bit.

Capture is legal because the forward never synchronises the host, never reads
device values on the host, allocates nothing after the first call for a given
token count (workspaces are cached), launches every kernel on the current
stream and records no memset node.
"""

from __future__ import annotations

import torch


@torch.inference_mode()
def capture_forward(block, x, warmup=3):
    """Capture ``block(x)`` into a ``torch.cuda.CUDAGraph``; raises if the replay differs.

    The graph reads ``x`` and writes ``block.workspace(x).transport.output`` (the
    tensor ``block(x)`` returns); keep ``x`` alive and update it in place to feed
    new tokens of the same shape.
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
    with torch.cuda.graph(graph, stream=stream):
        output = block(x)
    graph.replay()
    torch.cuda.synchronize(device)
    if not torch.equal(output, expected):
        raise RuntimeError("graph replay differs from the eager forward")
    return graph
