"""Randomised hipGraph capture of the block forward, from fixed seeds.

Configurations as in test_gpu_block_sweep.py (hidden and intermediate sizes
from 8 to 2048, 1 to 64 experts, top-1 to top-8, alignment 8 to 128, balanced
or skewed routing), with 1 to 4000 tokens, so that the captured forward meets
every launch path: the decode and persistent GEMMs, the ranked and plain
routes, the packed and row-table dispatches. Each replay equals the eager
forward bit for bit, with eager work on the same workspace between replays,
and again after new tokens are written into the captured input.
"""

import numpy as np
import pytest
import torch

from moe_dispatch.block_benchmark import capture_forward
from moe_dispatch.layer import MoEBlock, MoEConfig
from tests._helpers import gpu

pytestmark = gpu

CASES_PER_SEED = 12


def _configs(seed):
    rng = np.random.default_rng(seed)
    for case in range(CASES_PER_SEED):
        hidden = 8 * int(rng.integers(1, 257)) if rng.random() < 0.5 else 64 * int(rng.integers(1, 33))
        inter = 8 * int(rng.integers(1, 257)) if rng.random() < 0.5 else 64 * int(rng.integers(1, 33))
        experts = int(rng.choice([1, 2, 3, 4, 8, 12, 16, 24, 32, 48, 64]))
        topk = int(rng.integers(1, min(8, experts) + 1))
        alignment = int(rng.choice([8, 16, 32, 64, 128]))
        tokens = int(np.exp(rng.uniform(0, np.log(4000))))
        pattern = str(rng.choice(["balanced", "skewed"]))
        yield case, MoEConfig(hidden, inter, experts, topk, alignment), tokens, pattern


@pytest.mark.parametrize("seed", [51, 52])
def test_random_forward_graphs_replay_like_eager(seed):
    for case, cfg, tokens, pattern in _configs(seed):
        print(f"seed {seed} case {case}: T={tokens} H={cfg.hidden} I={cfg.intermediate} E={cfg.experts} "
              f"K={cfg.topk} a={cfg.alignment} {pattern}", flush=True)
        block = MoEBlock(cfg, device="cuda", implementation="cuda_fused", seed=100 * seed + case)
        block.set_routing_pattern(pattern)
        gen = torch.Generator(device="cuda").manual_seed(100 * seed + case)
        x = torch.randn(tokens, cfg.hidden, device="cuda", generator=gen).bfloat16()
        expected = block(x).clone()
        graph = capture_forward(block, x)
        output = block.workspace(x).transport.output
        other = torch.randn(tokens, cfg.hidden, device="cuda", generator=gen).bfloat16()
        expected_other = block(other).clone()
        for _ in range(2):
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(output, expected), "replay differs from eager"
            assert torch.equal(block(other), expected_other), "eager after a replay differs"
            torch.cuda.synchronize()
        x.copy_(other)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(output, expected_other), "replay on new tokens differs"
        del graph, block
