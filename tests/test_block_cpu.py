"""MoEBlock(implementation="torch") on CPU against both oracles (reference tests/test_block.py)."""

import numpy as np
import pytest
import torch

from moe_dispatch.layer import MoEBlock, MoEConfig, token_major_oracle
from oracle import moe_oracle as oracle


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("tokens", [0, 1, 13, 33])
@pytest.mark.parametrize("pattern", ["balanced", "skewed"])
@pytest.mark.parametrize("topk", [1, 2])
def test_complete_cpu_block_matches_token_major_oracle(dtype, tokens, pattern, topk):
    cfg = MoEConfig(hidden=32, intermediate=64, experts=8, topk=topk)
    block = MoEBlock(cfg, device="cpu", dtype=dtype, implementation="torch")
    block.set_routing_pattern(pattern)
    x = torch.randn(tokens, 32, generator=torch.Generator().manual_seed(42)).to(dtype)
    actual = block(x).clone()
    expected = token_major_oracle(block, x)
    torch.testing.assert_close(actual, expected, rtol=0.03, atol=0.03)


@pytest.mark.parametrize("topk,experts", [(2, 8), (6, 64)])
def test_cpu_block_matches_numpy_oracle(topk, experts):
    cfg = MoEConfig(hidden=64, intermediate=128, experts=experts, topk=topk)
    block = MoEBlock(cfg, device="cpu", dtype=torch.bfloat16, implementation="torch", seed=1)
    if experts == 64:
        block.set_routing_bias(oracle.zipf_bias(64))
    x = torch.randn(96, 64, generator=torch.Generator().manual_seed(2)).bfloat16()
    actual = block(x).float().numpy()
    ids32, _, weights = block.route(x)
    ref = oracle.block_forward(
        x.float().numpy(), block.router_weight.numpy(), block.routing_bias.numpy(),
        block.gate_up_weight.float().numpy(), block.down_weight.float().numpy(), topk, 8,
        ids=ids32.numpy(), weights=weights.numpy(),
    )
    diff = np.abs(actual - ref["output"])
    assert diff.max() <= 1.6e-2
    assert np.linalg.norm(actual - ref["output"]) / np.linalg.norm(ref["output"]) <= 2e-3


def test_shared_weights_and_workspace_reuse():
    block = MoEBlock(MoEConfig(32, 64, 8, 2), device="cpu", dtype=torch.float32, implementation="torch")
    x = torch.randn(13, 32)
    first = block.workspace(x)
    block(x)
    assert block.workspace(x) is first


def test_set_routing_bias_validates_shape():
    block = MoEBlock(MoEConfig(32, 64, 8, 2), device="cpu", dtype=torch.float32, implementation="torch")
    block.set_routing_bias(torch.arange(8.0))
    assert block.routing_bias.tolist() == list(range(8))
    with pytest.raises(ValueError):
        block.set_routing_bias(torch.zeros(7))
