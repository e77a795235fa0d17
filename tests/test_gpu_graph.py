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
