"""MoEBlock(implementation="torch") on CPU against the token-major evaluation and the numpy oracle.

Covers the contracts of the reference's ``tests/test_block.py`` (block vs
token-major oracle, workspace reuse) with this build's own cases: K up to 6,
E up to 64, an arbitrary router bias, empty batches.
"""

import numpy as np
import pytest
import torch

from moe_dispatch.layer import MoEBlock, MoEConfig, token_major_oracle
from oracle import moe_oracle as oracle


@pytest.mark.parametrize("case", [
    # (tokens, hidden, intermediate, experts, topk, pattern, dtype)
    (0, 16, 24, 4, 2, "balanced", torch.float32),
    (1, 24, 16, 8, 1, "skewed", torch.bfloat16),
    (9, 16, 40, 8, 2, "balanced", torch.bfloat16),
    (40, 32, 16, 8, 2, "skewed", torch.float32),
    (17, 8, 8, 16, 4, "balanced", torch.bfloat16),
])
def test_cpu_block_agrees_with_token_major_evaluation(case):
    """The packed-layout forward and the layout-free token-major evaluation agree."""
    tokens, hidden, inter, experts, topk, pattern, dtype = case
    cfg = MoEConfig(hidden=hidden, intermediate=inter, experts=experts, topk=topk)
    block = MoEBlock(cfg, device="cpu", dtype=dtype, implementation="torch", seed=tokens + 1)
    block.set_routing_pattern(pattern)
    x = torch.randn(tokens, hidden, generator=torch.Generator().manual_seed(3)).to(dtype)
    actual = block(x).clone()
    expected = token_major_oracle(block, x)
    assert actual.shape == expected.shape == (tokens, hidden) and actual.dtype == dtype
    # one output rounding apart at most (bf16: 2^-8 relative), plus fp32 order effects
    tol = 1e-5 if dtype == torch.float32 else 2.0**-7
    torch.testing.assert_close(actual.float(), expected.float(), rtol=tol, atol=tol)
    if pattern == "skewed" and tokens > 8:
        # the bias of +5 on the first K experts routes nearly every assignment there
        ids32, _, _ = block.route(x)
        assert (ids32 < topk).float().mean() > 0.9


def test_token_major_evaluation_matches_the_numpy_oracle():
    """The torch token-major evaluation (bf16 GEMM outputs) agrees with the numpy oracle's."""
    cfg = MoEConfig(hidden=32, intermediate=48, experts=8, topk=2)
    block = MoEBlock(cfg, device="cpu", dtype=torch.bfloat16, implementation="torch", seed=5)
    x = torch.randn(21, 32, generator=torch.Generator().manual_seed(6)).bfloat16()
    got = token_major_oracle(block, x).float().numpy()
    ids32, _, weights = block.route(x)
    ref = oracle.token_major_forward(x.float().numpy(), block.gate_up_weight.float().numpy(),
                                     block.down_weight.float().numpy(), ids32.numpy(), weights.numpy(),
                                     order="exact")
    # both round the projection, activation and expert output to bf16; the GEMM
    # orders differ, so a rounding can land one bf16 step apart
    assert np.abs(got - ref).max() <= 2.0**-6
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) < 4e-3


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
