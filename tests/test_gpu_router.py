"""Routing parity: top-k on given logits (bit-exact ids) and the fused fp32 router.

Mirrors the reference's tests/test_gpu_router.py:11-38 (exact ids vs an
independent top-k, weights within 2e-6, zero-logit tie KAT, empty batch) and
extends K to 1..8 and E to 1..64.
"""

import numpy as np
import pytest
import torch

from oracle import moe_oracle as oracle
from tests._helpers import gpu, route_margin, to_np

pytestmark = gpu


def _route(ext, logits, bias, topk):
    tokens = logits.shape[0]
    ids32 = torch.empty(tokens, topk, device="cuda", dtype=torch.int32)
    ids64 = torch.empty(tokens, topk, device="cuda", dtype=torch.int64)
    weights = torch.empty(tokens, topk, device="cuda")
    ext.topk_route_out(logits, bias, ids32, ids64, weights)
    return ids32, ids64, weights


@pytest.mark.parametrize("experts", [1, 2, 8, 16, 33, 64])
@pytest.mark.parametrize("topk", [1, 2, 6, 8])
def test_topk_route_matches_oracle_and_torch(ext, experts, topk):
    if topk > experts:
        pytest.skip("topk > experts")
    generator = torch.Generator(device="cuda").manual_seed(42)
    logits = torch.randn(257, experts, device="cuda", generator=generator)
    bias = torch.randn(experts, device="cuda", generator=generator)
    ids32, ids64, weights = _route(ext, logits, bias, topk)
    ids_ref, w_ref, _ = oracle.topk_route(to_np(logits), to_np(bias), topk)
    np.testing.assert_array_equal(to_np(ids32), ids_ref)
    np.testing.assert_array_equal(to_np(ids64), ids_ref.astype(np.int64))
    np.testing.assert_allclose(to_np(weights), w_ref, rtol=2e-6, atol=2e-6)
    # Independent library check (continuous scores: no ties).
    selected, expected = torch.topk(logits + bias, topk, dim=-1)
    torch.testing.assert_close(ids64, expected, rtol=0, atol=0)
    torch.testing.assert_close(weights, selected.softmax(-1), rtol=2e-6, atol=2e-6)


@pytest.mark.parametrize("topk", [2, 6])
def test_topk_route_ties_go_to_lower_expert(ext, topk):
    generator = torch.Generator(device="cuda").manual_seed(7)
    logits = torch.randint(0, 3, (513, 64), device="cuda", generator=generator).float()
    bias = torch.zeros(64, device="cuda")
    ids32, _, weights = _route(ext, logits, bias, topk)
    ids_ref, w_ref, _ = oracle.topk_route(to_np(logits), to_np(bias), topk)
    np.testing.assert_array_equal(to_np(ids32), ids_ref)
    np.testing.assert_allclose(to_np(weights), w_ref, rtol=2e-6, atol=2e-6)


def test_zero_logits_known_answer_and_empty_batch(ext):
    for tokens in (0, 5):
        logits = torch.zeros(tokens, 64, device="cuda")
        bias = torch.zeros(64, device="cuda")
        _, ids64, weights = _route(ext, logits, bias, 2)
        expected = torch.tensor([0, 1], device="cuda").expand(tokens, 2)
        torch.testing.assert_close(ids64, expected, rtol=0, atol=0)
        torch.testing.assert_close(weights, torch.full_like(weights, 0.5), rtol=0, atol=0)


@pytest.mark.parametrize(
    "tokens,hidden,experts,topk",
    [(1, 512, 8, 2), (33, 512, 8, 1), (257, 1024, 16, 2), (300, 2048, 64, 6), (64, 4096, 8, 2),
     (100, 136, 5, 3), (1000, 72, 32, 4), (8192, 2048, 64, 6),
     # Split-k routing (tokens <= 64, E <= 16, 16..256 stages of 64 hidden):
     # one token; a ragged last stage inside the last slice; the largest split
     # (16 slices of 16 stages); one stage past it (the single-workgroup path).
     (1, 4096, 8, 2), (16, 4096, 16, 6), (33, 2040, 12, 3), (50, 16384, 4, 2), (3, 16448, 8, 2),
     # E <= 16 past the split sizes: the VGPR-load kernel with 1 to 6 weight fragments
     # (E = 2, 3, 8, 10, 12, 16) and 2, 8 and 16 steps of 64 hidden per wave (ragged
     # last token tile, k tail inside a step); hidden 8200 takes the ring.
     (300, 4096, 8, 2), (1000, 8192, 16, 2), (77, 200, 3, 2), (130, 8200, 8, 2), (90, 256, 2, 1),
     (65, 320, 10, 3), (70, 64, 12, 4),
     # 16 < E <= 64 and hidden <= 4096: the many-expert VGPR-load kernel with 2 to
     # 6 fragments per wave (E = 17, 24, 40, 48; the last wave's range partly past
     # F), 8 to 64 steps of 64 hidden, k tails, ragged token tiles; hidden 4160
     # takes the ring.
     (97, 1000, 17, 3), (33, 520, 24, 2), (129, 3000, 40, 6), (45, 4096, 48, 8), (50, 4160, 32, 4)],
)
def test_fused_router_matches_oracle(ext, tokens, hidden, experts, topk):
    generator = torch.Generator(device="cuda").manual_seed(tokens + hidden)
    x = torch.randn(tokens, hidden, device="cuda", generator=generator).bfloat16()
    w = torch.randn(experts, hidden, device="cuda", generator=generator) / hidden**0.5
    bias = torch.randn(experts, device="cuda", generator=generator) * 0.1
    ids32 = torch.empty(tokens, topk, device="cuda", dtype=torch.int32)
    ids64 = torch.empty(tokens, topk, device="cuda", dtype=torch.int64)
    weights = torch.empty(tokens, topk, device="cuda")
    logits = torch.empty(tokens, experts, device="cuda")
    ext.router_fused_out(x, w, bias, ids32, ids64, weights, logits)
    ref_logits = oracle.router_logits(to_np(x), to_np(w))
    got_logits = to_np(logits)
    # fp32 dot products in a different order: bounded by a few ulp of the row norm.
    scale = np.linalg.norm(to_np(x), axis=1)[:, None] * np.linalg.norm(to_np(w), axis=1)[None, :]
    assert np.all(np.abs(got_logits - ref_logits) <= 1e-6 * scale + 1e-7)
    # Selection on the kernel's own logits is bit-exact against the oracle.
    ids_on_got, w_on_got, _ = oracle.topk_route(got_logits, to_np(bias), topk)
    np.testing.assert_array_equal(to_np(ids32), ids_on_got)
    np.testing.assert_array_equal(to_np(ids64), ids_on_got.astype(np.int64))
    np.testing.assert_allclose(to_np(weights), w_on_got, rtol=2e-6, atol=2e-6)
    # And equal to the oracle's routing on exact logits wherever the margin is not a near-tie.
    ids_ref, _, _ = oracle.topk_route(ref_logits, to_np(bias), topk)
    safe = route_margin(ref_logits, to_np(bias), topk) > 1e-4
    np.testing.assert_array_equal(np.sort(to_np(ids32)[safe], 1), np.sort(ids_ref[safe], 1))


@pytest.mark.parametrize("tokens,hidden", [(70, 128), (40, 2048)])
@pytest.mark.parametrize("experts,topk", [(8, 2), (16, 5), (32, 4), (64, 6), (64, 8)])
def test_fused_router_ties_go_to_lower_expert(ext, experts, topk, tokens, hidden):
    """Zero activations make every logit exactly 0, so the selection is decided by a
    bias full of repeated values: the fused top-k must keep the lower expert id on
    every tie, like the reference (``csrc/dispatch.cu:331-333``). 40 x 2048 with
    E <= 16 takes the split-k path and its separate selection kernel."""
    x = torch.zeros(tokens, hidden, device="cuda", dtype=torch.bfloat16)
    w = torch.randn(experts, hidden, device="cuda") / hidden**0.5
    levels = torch.tensor([0.0, 1.0, 2.0, 0.5], device="cuda")
    bias = levels[torch.arange(experts, device="cuda") * 7 % 4].contiguous()
    ids32 = torch.empty(tokens, topk, device="cuda", dtype=torch.int32)
    ids64 = torch.empty(tokens, topk, device="cuda", dtype=torch.int64)
    weights = torch.empty(tokens, topk, device="cuda")
    ext.router_fused_out(x, w, bias, ids32, ids64, weights)
    ids_ref, w_ref, _ = oracle.topk_route(np.zeros((tokens, experts), np.float32), to_np(bias), topk)
    np.testing.assert_array_equal(to_np(ids32), ids_ref)
    np.testing.assert_allclose(to_np(weights), w_ref, rtol=2e-6, atol=2e-6)


@pytest.mark.parametrize("tokens,hidden", [(300, 512), (8, 4096)])
def test_fused_router_reuses_a_held_split(ext, tokens, hidden):
    """router_weight=None routes with the split the scratch already holds: the same
    logits, ids and weights as passing the weights again, on new tokens (8 x 4096:
    the split-k path, whose partial logits follow the planes in the scratch)."""
    experts, topk = 16, 2
    gen = torch.Generator(device="cuda").manual_seed(5)
    w = torch.randn(experts, hidden, device="cuda", generator=gen) / hidden**0.5
    bias = torch.zeros(experts, device="cuda")
    scratch = torch.empty(ext.router_scratch_bytes(experts, hidden), dtype=torch.uint8, device="cuda")
    first = torch.randn(tokens, hidden, device="cuda", generator=gen).bfloat16()
    x = torch.randn(tokens, hidden, device="cuda", generator=gen).bfloat16()

    def route(tokens_in, weight):
        out = (torch.empty(tokens, topk, device="cuda", dtype=torch.int32),
               torch.empty(tokens, topk, device="cuda", dtype=torch.int64),
               torch.empty(tokens, topk, device="cuda"),
               torch.empty(tokens, experts, device="cuda"))
        ext.router_fused_out(tokens_in, weight, bias, out[0], out[1], out[2], out[3], scratch=scratch)
        return out

    route(first, w)
    reused = route(x, None)
    fresh = route(x, w)
    for a, b in zip(reused, fresh):
        assert torch.equal(a, b)
