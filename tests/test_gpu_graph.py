"""hipGraph capture of the block forward (reference block_benchmark.py:48-64).

Every replay must equal the eager forward bit for bit, including replays with
eager work of the same shape (which reuses the same workspace) in between and
a replay after the captured input was updated in place.
"""

import pytest
import torch

from moe_dispatch.block_benchmark import capture_forward
from moe_dispatch.layer import MoEBlock, MoEConfig
from tests._helpers import gpu

pytestmark = gpu


@pytest.mark.parametrize("cfg,tokens", [
    (MoEConfig(512, 1024, 8, 2), 128),      # C1 shape
    (MoEConfig(1024, 2048, 16, 2), 256),    # C3 shape
    (MoEConfig(4096, 14336, 8, 2), 16),     # C4 decode shape
    (MoEConfig(2048, 1408, 64, 6), 600),    # C5 shape (top-6: the row table and the gathered gate/up GEMM)
])
def test_graph_replays_match_eager(cfg, tokens):
    block = MoEBlock(cfg, device="cuda", implementation="cuda_fused", seed=0)
    gen = torch.Generator(device="cuda").manual_seed(1)
    x = torch.randn(tokens, cfg.hidden, device="cuda", generator=gen).bfloat16()
    expected = block(x).clone()
    graph = capture_forward(block, x)
    output = block.workspace(x).transport.output
    other = torch.randn(tokens, cfg.hidden, device="cuda", generator=gen).bfloat16()
    expected_other = block(other).clone()
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(output, expected)
        # Eager work on the same workspace between replays.
        assert torch.equal(block(other), expected_other)
        torch.cuda.synchronize()
    # New tokens through the captured input buffer.
    x.copy_(other)
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(output, expected_other)


def test_graph_replay_reads_router_weights_as_they_are():
    """A captured forward re-splits the router weights on every replay, so an
    in-place update after capture routes the replay with the new weights."""
    cfg = MoEConfig(512, 1024, 8, 2)
    block = MoEBlock(cfg, device="cuda", implementation="cuda_fused", seed=0)
    twin = MoEBlock(cfg, device="cuda", implementation="cuda_fused", seed=0)
    gen = torch.Generator(device="cuda").manual_seed(2)
    x = torch.randn(128, cfg.hidden, device="cuda", generator=gen).bfloat16()
    block(x)  # the split is now held between calls
    graph = capture_forward(block, x)
    output = block.workspace(x).transport.output
    new_w = torch.randn(cfg.experts, cfg.hidden, device="cuda", generator=gen) / cfg.hidden**0.5
    block.router_weight.copy_(new_w)
    twin.router_weight = new_w.clone()
    expected = twin(x).clone()
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(output, expected)


def test_user_captured_graph_records_the_router_split():
    """A graph captured directly with torch.cuda.graph (not capture_forward) keeps the
    router split inside, so replaying it after an in-place router update routes with
    the new weights without any wrapper."""
    cfg = MoEConfig(512, 1024, 8, 2)
    block = MoEBlock(cfg, device="cuda", implementation="cuda_fused", seed=0)
    twin = MoEBlock(cfg, device="cuda", implementation="cuda_fused", seed=0)
    gen = torch.Generator(device="cuda").manual_seed(3)
    x = torch.randn(128, cfg.hidden, device="cuda", generator=gen).bfloat16()
    block(x)
    block(x)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        output = block(x)
    torch.cuda.current_stream().wait_stream(side)
    new_w = torch.randn(cfg.experts, cfg.hidden, device="cuda", generator=gen) / cfg.hidden**0.5
    block.router_weight.copy_(new_w)
    twin.router_weight = new_w.clone()
    expected = twin(x).clone()
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(output, expected)
    # ... and eager forwards afterwards see the same weights.
    assert torch.equal(block(x), expected)


def test_forward_graph_replays_skip_the_split_until_the_weights_change():
    """capture_forward's graph leaves the split out; replay() redoes it only after a change."""
    cfg = MoEConfig(512, 1024, 8, 2)
    block = MoEBlock(cfg, device="cuda", implementation="cuda_fused", seed=0)
    x = torch.randn(128, cfg.hidden, device="cuda").bfloat16()
    graph = capture_forward(block, x)
    calls = []
    real = block._extension.router_split_out
    block._extension.router_split_out = lambda *a: (calls.append(1), real(*a))
    try:
        graph.replay()
        graph.replay()
        assert calls == []
        block.router_weight.mul_(1.0)  # an in-place write bumps the version
        graph.replay()
        graph.replay()
        assert calls == [1]
    finally:
        block._extension.router_split_out = real
    torch.cuda.synchronize()
