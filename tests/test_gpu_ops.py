"""The standalone transport API on the GPU: ``ops.dispatch`` / ``ops.combine`` / ``PackedTokens``.

Contract of the reference's ``src/moe_dispatch/ops.py:19-77`` (and its use in
README.md:129): int32 or int64 ids (int64 cast to int32), a workspace given or
created on the fly, alignment 1 or 8, views of the workspace returned, and
``ValueError`` for a mismatched workspace or out-of-range ids. Every layout
buffer, every packed row and the combined output are compared bit for bit with
the oracle. Also covered here: operands that start off a 16-byte boundary (an
offset view of a larger tensor): the transport takes narrower accesses and
stays exact, while the GEMMs, which can only read 16-byte vectors, refuse them.
"""

import numpy as np
import pytest
import torch

from moe_dispatch import ops
from moe_dispatch._lib import MoeHipError
from moe_dispatch.routing import make_transport_case
from moe_dispatch.workspace import CudaWorkspace
from oracle import moe_oracle as oracle
from tests._helpers import NP_DTYPE, assert_layout_equal, assert_packed_equal, gpu, to_np

pytestmark = gpu

CASES = [
    # tokens, hidden, experts, topk, dtype, alignment, id dtype, supply the workspace
    (1, 64, 8, 2, torch.bfloat16, 1, torch.int64, False),
    (33, 128, 8, 2, torch.bfloat16, 8, torch.int32, True),
    (257, 96, 16, 1, torch.float16, 8, torch.int64, True),
    (500, 2048, 8, 2, torch.bfloat16, 1, torch.int32, False),
    (129, 40, 64, 6, torch.float32, 8, torch.int64, False),
    (64, 17, 4, 3, torch.bfloat16, 1, torch.int64, True),
]


@pytest.mark.parametrize("tokens,hidden,experts,topk,dtype,alignment,id_dtype,given", CASES)
def test_ops_dispatch_and_combine_bit_exact(tokens, hidden, experts, topk, dtype, alignment, id_dtype, given):
    x, ids32, ids64, weights = make_transport_case(tokens, hidden, experts, topk, dtype, seed=tokens)
    ids = ids32 if id_dtype == torch.int32 else ids64
    workspace = CudaWorkspace(tokens, hidden, experts, topk, dtype, alignment=alignment) if given else None
    batch = ops.dispatch(x, ids, experts, workspace=workspace, alignment=alignment)
    assert isinstance(batch, ops.PackedTokens)
    ws = batch.workspace
    if given:
        assert ws is workspace
    # The batch holds views of the workspace buffers.
    assert batch.packed.data_ptr() == ws.packed.data_ptr() and batch.inverse.data_ptr() == ws.inverse.data_ptr()
    assert batch.counts.data_ptr() == ws.counts.data_ptr() and batch.offsets.data_ptr() == ws.offsets.data_ptr()
    layout = oracle.dispatch_layout(to_np(ids32), experts, alignment)
    assert_layout_equal(ws, layout, tokens, topk, experts)
    assert_packed_equal(batch.packed, x, layout, topk)
    # Combine an arbitrary expert output with weights given in fp16 (converted to fp32).
    gen = torch.Generator(device="cuda").manual_seed(tokens + 1)
    y = torch.randn(batch.packed.shape, device="cuda", generator=gen).to(dtype)
    w16 = weights.half()
    out = ops.combine(y, batch, w16)
    assert out.data_ptr() == ws.output.data_ptr()
    expected = oracle.combine(to_np(y), layout["inverse"], to_np(w16.float()), NP_DTYPE[dtype])
    np.testing.assert_array_equal(to_np(out), expected)


def test_ops_reuse_a_workspace_across_calls():
    x, ids32, ids64, weights = make_transport_case(300, 256, 8, 2, torch.bfloat16, seed=3)
    ws = CudaWorkspace(300, 256, 8, 2, torch.bfloat16, alignment=8)
    first = ops.dispatch(x, ids64, 8, workspace=ws, alignment=8)
    packed_first = first.packed.clone()
    x2, ids2, _, _ = make_transport_case(300, 256, 8, 2, torch.bfloat16, seed=4)
    second = ops.dispatch(x2, ids2, 8, workspace=ws, alignment=8)
    assert second.packed.data_ptr() == first.packed.data_ptr()  # same buffers, new contents
    layout = oracle.dispatch_layout(to_np(ids2), 8, 8)
    assert_packed_equal(second.packed, x2, layout, 2)
    assert not torch.equal(second.packed, packed_first)


def test_ops_errors():
    x, ids32, ids64, weights = make_transport_case(16, 64, 8, 2, torch.bfloat16, seed=1)
    ws = CudaWorkspace(16, 64, 8, 2, torch.bfloat16)
    bad_ids = ids64.clone()
    bad_ids[3, 1] = 8
    with pytest.raises(ValueError, match="out-of-range"):
        ops.dispatch(x, bad_ids, 8)
    bad_ids[3, 1] = -1
    with pytest.raises(ValueError, match="out-of-range"):
        ops.dispatch(x, bad_ids.int(), 8)
    with pytest.raises(ValueError, match="workspace shape/dtype"):
        ops.dispatch(x, ids64, 16, workspace=ws)  # the workspace was built for E=8
    with pytest.raises(ValueError, match="workspace shape/dtype"):
        ops.dispatch(x.half(), ids64, 8, workspace=ws)
    with pytest.raises(ValueError, match="workspace shape/dtype"):
        ops.dispatch(x[:8], ids64[:8], 8, workspace=ws)
    with pytest.raises(TypeError):
        ops.dispatch(x, ids64.float(), 8)
    with pytest.raises(ValueError, match="same device"):
        ops.dispatch(x, ids64.cpu(), 8)
    with pytest.raises(RuntimeError, match="requires a GPU"):
        ops.dispatch(x.cpu(), ids64.cpu(), 8)
    batch = ops.dispatch(x, ids64, 8, workspace=ws)
    y = torch.zeros_like(batch.packed)
    with pytest.raises(ValueError, match=r"shape \[T,K\]"):
        ops.combine(y, batch, weights[:, :1].contiguous())
    with pytest.raises(ValueError, match="shape/dtype must match"):
        ops.combine(y.float(), batch, weights)
    with pytest.raises(TypeError, match="floating point"):
        ops.combine(y, batch, ids32)
    with pytest.raises(ValueError, match="contiguous"):
        ops.combine(y, batch, weights.t().contiguous().t())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_transport_on_views_off_a_16_byte_boundary(dtype):
    """x, packed output and expert rows taken one element into larger buffers."""
    tokens, hidden, experts, topk = 70, 256, 8, 2
    x_full, ids32, ids64, weights = make_transport_case(tokens + 1, hidden, experts, topk, dtype, seed=6)
    flat = x_full.reshape(-1)
    x = flat[1:1 + tokens * hidden].view(tokens, hidden)  # starts one element in
    assert x.data_ptr() % 16 != 0 and x.is_contiguous()
    ids32, ids64, weights = ids32[:tokens].contiguous(), ids64[:tokens].contiguous(), weights[:tokens].contiguous()
    ws = CudaWorkspace(tokens, hidden, experts, topk, dtype, alignment=8)
    ws.dispatch(x, ids32, ids64)
    layout = oracle.dispatch_layout(to_np(ids32), experts, 8)
    assert_layout_equal(ws, layout, tokens, topk, experts)
    assert_packed_equal(ws.packed, x, layout, topk)
    rows = ws.capacity_rows
    y_full = torch.randn(rows * hidden + 1, device="cuda", generator=torch.Generator(device="cuda").manual_seed(7))
    y = y_full.to(dtype)[1:].view(rows, hidden)
    assert y.data_ptr() % 16 != 0
    ws.combine(y, weights)
    expected = oracle.combine(to_np(y), layout["inverse"], to_np(weights), NP_DTYPE[dtype])
    np.testing.assert_array_equal(to_np(ws.output), expected)


def test_gemm_refuses_operands_off_a_16_byte_boundary(ext):
    a_full = torch.randn(64 * 64 + 8, device="cuda").bfloat16()
    a = a_full[8:].view(64, 64)  # 16-byte aligned: accepted
    b = torch.randn(1, 64, 64, device="cuda").bfloat16()
    offsets = torch.tensor([0, 64], device="cuda", dtype=torch.int32)
    out = torch.empty(64, 64, device="cuda", dtype=torch.bfloat16)
    ext.grouped_gemm_out(a, b, offsets, out)
    a_odd = a_full[4:4 + 64 * 64].view(64, 64)  # 8 bytes in
    with pytest.raises(MoeHipError, match="16-byte aligned"):
        ext.grouped_gemm_out(a_odd, b, offsets, out)
    with pytest.raises(MoeHipError, match="16-byte aligned"):
        ext.gateup_swiglu_out(a_odd, torch.randn(1, 128, 64, device="cuda").bfloat16(), offsets,
                              torch.empty(64, 64, device="cuda", dtype=torch.bfloat16))
    torch.cuda.synchronize()
