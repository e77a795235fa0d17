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


def test_weight_row_stride_of_each_layout():
    from moe_dispatch._extension import weight_row_stride

    w = torch.zeros(4, 6, 16)
    assert weight_row_stride(w) == 16
    assert weight_row_stride(torch.zeros(4, 6, 24)[:, :, :16]) == 24
    assert weight_row_stride(torch.zeros(3, 1, 24)[:, :, :16]) == 24  # one row per expert
    assert weight_row_stride(torch.zeros(1, 1, 16)) == 16
    assert weight_row_stride(w.transpose(1, 2)) is None  # columns contiguous, not rows
    assert weight_row_stride(w[:, ::2]) == 32  # every other row: evenly spaced
    assert weight_row_stride(torch.zeros(4, 12, 16)[::2, :6]) is None  # experts not rows * stride apart
    assert weight_row_stride(torch.zeros(6, 16)) is None


def test_fused_block_pads_power_of_two_gate_up_rows():
    from moe_dispatch.layer import GATE_UP_ROW_PADDING, padded_gate_up

    for hidden, padded in ((4096, True), (8192, True), (2048, False), (6144, False), (512, False)):
        w = torch.randn(2, 8, hidden).bfloat16()
        p = padded_gate_up(w)
        assert torch.equal(p, w)
        assert p.stride(1) == (hidden + GATE_UP_ROW_PADDING if padded else hidden), hidden
    # fp32 rows of 2048 elements are 8 KiB: padded too.
    assert padded_gate_up(torch.zeros(1, 2, 2048)).stride(1) == 2048 + GATE_UP_ROW_PADDING
