"""Transport parity: dispatch (counts, offsets, slots, inverse, packed rows) bit-exact
against the oracle's canonical order, and the weighted combine bit-exact against
the oracle's fp32 k-order sum.

Mirrors the reference's tests/test_gpu.py:22-28 (validate_case over dtypes,
alignment and T in {0,1,33,257}) and adds exact layout parity, K up to 8,
E up to 64, odd hidden sizes, the scalar path, masking of out-of-range ids,
run-to-run determinism and the full transport configuration (T=4096, H=2048).
"""

import numpy as np
import pytest
import torch

from moe_dispatch.routing import make_case, make_transport_case
from moe_dispatch.validation import validate_case
from moe_dispatch.workspace import CudaWorkspace
from oracle import moe_oracle as oracle
from tests._helpers import NP_DTYPE, assert_layout_equal, assert_packed_equal, gpu, raw_bits, to_np

pytestmark = gpu


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32, torch.bfloat16])
@pytest.mark.parametrize("alignment", [1, 8])
@pytest.mark.parametrize("tokens", [0, 1, 33, 257])
def test_transport_validate_case(ext, dtype, alignment, tokens):
    x, i32, i64, w = make_case(tokens, 32, 8, 2, dtype, "skewed", 42)
    ws = CudaWorkspace(tokens, 32, 8, 2, dtype, alignment=alignment, extension=ext)
    validate_case(ws, x, i32, i64, w, 8, 42)


CASES = [
    # tokens, hidden, experts, topk, alignment, dtype, vectorized
    (0, 64, 8, 2, 8, torch.bfloat16, True),
    (1, 17, 8, 2, 1, torch.float32, True),
    (7, 31, 8, 1, 16, torch.float16, True),
    (33, 128, 8, 2, 8, torch.bfloat16, True),
    (257, 1024, 16, 2, 1, torch.bfloat16, True),
    (257, 1024, 16, 2, 8, torch.bfloat16, False),
    (513, 256, 64, 6, 8, torch.bfloat16, True),
    (1000, 96, 5, 3, 128, torch.float32, True),
    (2049, 40, 64, 8, 1, torch.float16, True),
    (130, 3, 4, 2, 16, torch.bfloat16, True),
    # Just past the pack kernel's own ranking (1024 assignments), experts 8-15
    # in use, the largest K, the scalar path, and an odd assignment count
    (513, 64, 16, 2, 8, torch.bfloat16, True),
    (2048, 64, 16, 8, 1, torch.float16, True),
    (777, 3, 4, 2, 16, torch.bfloat16, True),
    (3277, 32, 8, 5, 8, torch.bfloat16, True),
]


@pytest.mark.parametrize("tokens,hidden,experts,topk,alignment,dtype,vectorized", CASES)
def test_dispatch_and_combine_bit_exact(ext, tokens, hidden, experts, topk, alignment, dtype, vectorized):
    x, i32, i64, w = make_transport_case(tokens, hidden, experts, topk, dtype, seed=tokens + 3)
    ws = CudaWorkspace(tokens, hidden, experts, topk, dtype, vectorized=vectorized,
                       alignment=alignment, extension=ext)
    ws.dispatch(x, i32, i64)
    layout = oracle.dispatch_layout(to_np(i32), experts, alignment)
    assert_layout_equal(ws, layout, tokens, topk, experts)
    assert_packed_equal(ws.packed, x, layout, topk)
    # Combine of an arbitrary expert output, bit-exact against the oracle.
    y = torch.randn(ws.capacity_rows, hidden, device="cuda", generator=torch.Generator(device="cuda").manual_seed(5)).to(dtype)
    ws.combine(y, w)
    expected = oracle.combine(to_np(y), to_np(ws.inverse), to_np(w), NP_DTYPE[dtype])
    np.testing.assert_array_equal(to_np(ws.output), expected)


def test_combine_k2_matches_torch_weighted_sum_exactly(ext):
    x, i32, i64, w = make_transport_case(300, 256, 8, 2, torch.bfloat16, seed=11)
    ws = CudaWorkspace(300, 256, 8, 2, torch.bfloat16, extension=ext)
    ws.dispatch(x, i32, i64)
    canonical = torch.randn(600, 256, device="cuda").bfloat16()
    y = torch.empty_like(ws.packed)
    y.index_copy_(0, ws.inverse.reshape(-1).long(), canonical)
    ws.combine(y, w)
    expected = (canonical.view(300, 2, 256).float() * w[:, :, None]).sum(1).bfloat16()
    torch.testing.assert_close(ws.output, expected, rtol=0, atol=0)


# 6 tokens: the pack kernel ranks every id itself (up to 1024 assignments);
# 700: the counting kernel first
@pytest.mark.parametrize("tokens", [6, 700])
def test_out_of_range_ids_are_masked(ext, tokens):
    x = torch.randn(tokens, 32, device="cuda").bfloat16()
    if tokens == 6:
        ids = torch.tensor([[0, 9], [1, -1], [2, 2], [7, 0], [8, 3], [1, 1]], device="cuda", dtype=torch.int32)
    else:
        g = torch.Generator(device="cuda").manual_seed(13)
        ids = torch.randint(-2, 11, (tokens, 2), device="cuda", generator=g, dtype=torch.int32)
    ws = CudaWorkspace(tokens, 32, 8, 2, torch.bfloat16, alignment=1, extension=ext)
    ws.inverse.fill_(-7)
    ws.slots.fill_(5)
    # Capacity T*K rows; invalid assignments are not counted and leave inverse untouched.
    ws.dispatch(x, ids)
    layout = oracle.dispatch_layout(to_np(ids), 8, 1)
    np.testing.assert_array_equal(to_np(ws.counts), layout["counts"])
    np.testing.assert_array_equal(to_np(ws.offsets), layout["offsets"])
    got_inv = to_np(ws.inverse).reshape(-1)
    ref_inv = layout["inverse"].reshape(-1)
    valid = ref_inv >= 0
    np.testing.assert_array_equal(got_inv[valid], ref_inv[valid])
    assert np.all(got_inv[~valid] == -7)
    np.testing.assert_array_equal(to_np(ws.slots)[~valid], -1)


@pytest.mark.parametrize("alignment", [1, 8])
def test_dispatch_and_combine_are_deterministic(ext, alignment):
    x, i32, i64, w = make_transport_case(3000, 512, 64, 6, torch.bfloat16, seed=3)
    ws = CudaWorkspace(3000, 512, 64, 6, torch.bfloat16, alignment=alignment, extension=ext)
    y = torch.randn(ws.capacity_rows, 512, device="cuda").bfloat16()
    results = []
    for _ in range(2):
        ws.packed.zero_()
        ws.dispatch(x, i32, i64)
        ws.combine(y, w)
        results.append([raw_bits(t) for t in (ws.packed, ws.inverse, ws.slots, ws.offsets, ws.output)])
    for a, b in zip(*results):
        np.testing.assert_array_equal(a, b)


@pytest.mark.parametrize("experts", [8, 16])
def test_one_expert_takes_every_assignment(ext, experts):
    """16384 assignments to one expert (the last): every chunk's count lands in
    one column of the count table, and one expert's span holds every row."""
    tokens, topk, hidden = 2048, 8, 64
    x = torch.randn(tokens, hidden, device="cuda").bfloat16()
    ids = torch.full((tokens, topk), experts - 1, device="cuda", dtype=torch.int32)
    ws = CudaWorkspace(tokens, hidden, experts, topk, torch.bfloat16, alignment=8, extension=ext)
    ws.dispatch(x, ids)
    layout = oracle.dispatch_layout(to_np(ids), experts, 8)
    assert_layout_equal(ws, layout, tokens, topk, experts)
    assert_packed_equal(ws.packed, x, layout, topk)


def test_full_transport_configuration_bit_exact(ext):
    """T=4096, H=2048, E=8, top-2, compact layout, uniform ids (the transport workload)."""
    tokens, hidden, experts, topk = 4096, 2048, 8, 2
    x, i32, i64, w = make_transport_case(tokens, hidden, experts, topk, torch.bfloat16, seed=0)
    ws = CudaWorkspace(tokens, hidden, experts, topk, torch.bfloat16, extension=ext)
    ws.dispatch(x, i32, i64)
    layout = oracle.dispatch_layout(to_np(i32), experts, 1)
    assert_layout_equal(ws, layout, tokens, topk, experts)
    # Permutation check (size-independent): packed rows gathered through inverse equal x.
    unpacked = ws.packed.index_select(0, ws.inverse.reshape(-1).long()).view(tokens, topk, hidden)
    assert torch.equal(unpacked, x[:, None, :].expand_as(unpacked))
    ws.combine(ws.packed, w)
    expected = oracle.combine(to_np(ws.packed), layout["inverse"], to_np(w), "bf16")
    np.testing.assert_array_equal(to_np(ws.output), expected)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32, torch.bfloat16])
def test_standalone_swiglu_and_unused_rows(ext, dtype):
    projection = torch.randn(37, 34, device="cuda").to(dtype)
    output = torch.empty(37, 17, device="cuda", dtype=dtype)
    rows = torch.tensor([21], device="cuda", dtype=torch.int32)
    ext.swiglu_out(projection, rows, output)
    expected = oracle.swiglu(to_np(projection), 21, NP_DTYPE[dtype])
    np.testing.assert_array_equal(to_np(output), expected)
    # Reference tolerance against torch's own silu (tests/test_gpu.py:31-40).
    gate, up = projection.float().chunk(2, -1)
    torch_ref = (torch.nn.functional.silu(gate) * up).to(dtype)
    tol = {torch.bfloat16: 2e-2, torch.float16: 2e-3, torch.float32: 2e-5}[dtype]
    torch.testing.assert_close(output[:21], torch_ref[:21], rtol=tol, atol=tol)
    assert np.all(to_np(output)[21:] == 0)


def test_reference_runtime_validation_suite(ext):
    """The reference's 36-check runtime suite (validation.py:64-104): FP32/FP16,
    K=1/2, empty batch, empty experts, skew, odd H, scalar and vector paths, plus
    the PyTorch transport variant."""
    from moe_dispatch.validation import run_tests

    summary = run_tests(ext)
    assert summary["passed"] == 36 and summary["failed"] == 0
    assert summary["max_absolute_error"] < 2e-3
