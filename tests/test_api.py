"""API contracts that hold without a GPU (reference tests/test_api.py:7-22, test_block.py:20-34)."""

import pytest
import torch

from moe_dispatch.experts import resolve_backend
from moe_dispatch.layer import MoEBlock, MoEConfig
from moe_dispatch.ops import validate_inputs
from moe_dispatch.workspace import CudaWorkspace


@pytest.mark.parametrize(
    "bad_ids", [torch.tensor([[0.0, 1.0]]), torch.tensor([[-1, 0]]), torch.tensor([[0, 8]])]
)
def test_invalid_expert_ids_are_rejected(bad_ids):
    with pytest.raises((TypeError, ValueError)):
        validate_inputs(torch.randn(1, 32), bad_ids, 8)


def test_forward_only_contract_is_explicit():
    with pytest.raises(ValueError, match="forward-only"):
        validate_inputs(torch.randn(1, 32, requires_grad=True), torch.tensor([[0, 1]]), 8)


def test_topk_limit_is_eight():
    validate_inputs(torch.randn(2, 32), torch.zeros(2, 8, dtype=torch.int64), 8)
    with pytest.raises(ValueError, match="topk"):
        validate_inputs(torch.randn(2, 32), torch.zeros(2, 9, dtype=torch.int64), 16)


def test_cpu_workspace_does_not_touch_the_gpu():
    with pytest.raises(RuntimeError, match="CUDA GPU"):
        CudaWorkspace(1, 32, 8, 2, torch.float32, device="cpu")


def test_workspace_argument_validation():
    with pytest.raises(ValueError):
        CudaWorkspace(1, 32, 65, 2, torch.float32, device="cpu")
    with pytest.raises(ValueError):
        CudaWorkspace(1, 32, 8, 9, torch.float32, device="cpu")
    with pytest.raises(ValueError):
        CudaWorkspace(1, 32, 8, 2, torch.int32, device="cpu")
    with pytest.raises(ValueError):
        CudaWorkspace(1, 32, 8, 2, torch.float32, device="cpu", alignment=129)


def test_invalid_block_shapes_fail_early():
    with pytest.raises(ValueError, match="multiples of 8"):
        MoEConfig(hidden=17)
    with pytest.raises(ValueError, match="expert/topk"):
        MoEConfig(experts=1, topk=2)
    with pytest.raises(ValueError, match="expert/topk"):
        MoEConfig(experts=64, topk=9)
    with pytest.raises(ValueError, match="alignment"):
        MoEConfig(alignment=4)
    assert MoEConfig(2048, 1408, 64, 6).topk == 6


def test_hip_implementations_need_a_gpu():
    with pytest.raises(RuntimeError):
        MoEBlock(MoEConfig(32, 64, 8, 2), device="cpu", implementation="cuda_fused")
    with pytest.raises(ValueError):
        MoEBlock(MoEConfig(32, 64, 8, 2), device="cpu", implementation="bogus")


def test_backend_resolution():
    assert resolve_backend("cpu", "auto") == "torch"
    with pytest.raises(RuntimeError):
        resolve_backend("cpu", "triton")
    with pytest.raises(RuntimeError):
        resolve_backend("cpu", "hip")
    with pytest.raises(ValueError):
        resolve_backend("cpu", "nope")


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-GPU error path")
def test_extension_refuses_without_gpu():
    from moe_dispatch._extension import get_extension

    with pytest.raises(RuntimeError, match="GPU"):
        get_extension()
