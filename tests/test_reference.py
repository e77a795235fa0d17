"""The PyTorch transport variant on CPU against the oracle's canonical layout.

``TorchWorkspace`` sorts stably, so every buffer it fills must equal the
oracle's restatement of the reference dispatch bit for bit: counts, aligned
offsets, inverse map and packed rows (padding zero). Its combine must equal the
oracle's k-order fp32 sum exactly, and the acceptance invariants
(``moe_dispatch.validation``) must hold, including on transport-style ids where
one token may pick the same expert twice.
"""

import numpy as np
import pytest
import torch

from moe_dispatch.reference import TorchWorkspace
from moe_dispatch.routing import make_case, make_transport_case
from moe_dispatch.validation import validate_case
from oracle import moe_oracle as oracle

SHAPES = [(0, 24, 8, 2), (1, 8, 4, 1), (5, 40, 16, 2), (64, 72, 8, 2), (50, 16, 64, 6), (19, 33, 3, 3)]


@pytest.mark.parametrize("alignment", [1, 4, 8, 128])
@pytest.mark.parametrize("shape", SHAPES)
def test_layout_equals_oracle(shape, alignment):
    tokens, hidden, experts, topk = shape
    x, ids32, ids64, _ = make_transport_case(tokens, hidden, experts, topk, torch.bfloat16, seed=tokens + 3,
                                             device="cpu")
    ws = TorchWorkspace(*shape, torch.bfloat16, device="cpu", alignment=alignment)
    ws.dispatch(x, ids32, ids64)
    layout = oracle.dispatch_layout(ids32.numpy(), experts, alignment)
    np.testing.assert_array_equal(ws.counts.numpy(), layout["counts"])
    np.testing.assert_array_equal(ws.offsets.numpy(), layout["offsets"])
    np.testing.assert_array_equal(ws.inverse.numpy(), layout["inverse"])
    used = int(layout["offsets"][-1])
    packed, defined = oracle.pack(x.float().numpy(), layout, topk, ws.capacity_rows)
    assert defined[:used].all() and not defined[used:].any()
    np.testing.assert_array_equal(ws.packed[:used].float().numpy(), packed[:used])


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("shape", SHAPES)
def test_combine_equals_oracle_k_order_sum(dtype, shape):
    tokens, hidden, experts, topk = shape
    x, ids32, ids64, weights = make_transport_case(tokens, hidden, experts, topk, dtype, seed=7, device="cpu")
    ws = TorchWorkspace(*shape, dtype, device="cpu", alignment=8)
    ws.dispatch(x, ids32, ids64)
    y = torch.randn(ws.capacity_rows, hidden, generator=torch.Generator().manual_seed(11)).to(dtype)
    ws.combine(y, weights)
    layout = oracle.dispatch_layout(ids32.numpy(), experts, 8)
    name = {torch.float32: "f32", torch.float16: "f16", torch.bfloat16: "bf16"}[dtype]
    expected = oracle.combine(y.float().numpy(), layout["inverse"], weights.numpy(), name)
    np.testing.assert_array_equal(ws.output.float().numpy(), expected)


@pytest.mark.parametrize("alignment", [1, 8, 16])
@pytest.mark.parametrize("pattern", ["balanced", "skewed"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_acceptance_invariants_hold(dtype, pattern, alignment):
    for shape in SHAPES:
        tokens, hidden, experts, topk = shape
        x, ids32, ids64, weights = make_case(tokens, hidden, experts, topk, dtype, pattern, 5, device="cpu")
        ws = TorchWorkspace(*shape, dtype, device="cpu", alignment=alignment)
        assert validate_case(ws, x, ids32, ids64, weights, experts, 5) < 2e-2


def test_invariants_reject_a_wrong_layout():
    """A workspace that swaps two packed rows of different experts fails the checks."""
    x, ids32, ids64, weights = make_case(16, 8, 4, 2, torch.float32, "balanced", 1, device="cpu")

    class Swapped(TorchWorkspace):
        def dispatch(self, x, ids32, ids64):
            super().dispatch(x, ids32, ids64)
            flat = self.inverse.reshape(-1)
            a = 0
            b = next(i for i in range(flat.numel()) if ids64.reshape(-1)[i] != ids64.reshape(-1)[a])
            flat[a], flat[b] = flat[b].clone(), flat[a].clone()

    with pytest.raises(AssertionError):
        validate_case(Swapped(16, 8, 4, 2, torch.float32, device="cpu"), x, ids32, ids64, weights, 4, 1)
