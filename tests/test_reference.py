"""The PyTorch transport variant on CPU: reference invariants and canonical layout.

Mirrors the reference tests/test_reference.py:8-17 and adds bit-exact layout
parity with the oracle (the variant sorts stably, so its order is canonical).
"""

import numpy as np
import pytest
import torch

from moe_dispatch.reference import TorchWorkspace
from moe_dispatch.routing import make_case
from moe_dispatch.validation import validate_case
from oracle import moe_oracle as oracle


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("alignment", [1, 8, 16])
@pytest.mark.parametrize("shape", [(0, 17, 8, 2), (1, 17, 8, 2), (7, 31, 8, 1), (33, 128, 8, 2), (40, 24, 64, 6)])
def test_packing_and_combine_against_independent_oracle(dtype, alignment, shape):
    tokens, hidden, experts, topk = shape
    x, ids32, ids64, weights = make_case(tokens, hidden, experts, topk, dtype, "skewed", 42, device="cpu")
    workspace = TorchWorkspace(*shape, dtype, device="cpu", alignment=alignment)
    validate_case(workspace, x, ids32, ids64, weights, experts, 42)
    layout = oracle.dispatch_layout(ids32.numpy(), experts, alignment)
    np.testing.assert_array_equal(workspace.counts.numpy(), layout["counts"])
    np.testing.assert_array_equal(workspace.offsets.numpy(), layout["offsets"])
    np.testing.assert_array_equal(workspace.inverse.numpy(), layout["inverse"])
