"""moe_dispatch_noalloc against moe_dispatch, through the C ABI.

The allocation-free entry point keeps its count table in the library's static
device array; on two calls in a row (the second smaller, so the array holds the
first call's counters when it starts) every output must equal what moe_dispatch
writes with a workspace scratch buffer, bit for bit: counts, offsets, slots,
inverse and every packed row inside the used spans. The same holds for replays
of a graph that captured the entry point.
"""

import numpy as np
import pytest
import torch

from moe_dispatch import _lib
from moe_dispatch._extension import DTYPE_CODES, current_stream_handle
from moe_dispatch.routing import make_transport_case
from moe_dispatch.workspace import CudaWorkspace
from tests._helpers import gpu, raw_bits

pytestmark = gpu


def _buffers(tokens, hidden, experts, topk, rows, dtype, device):
    return {
        "counts": torch.full((experts,), -7, device=device, dtype=torch.int32),
        "offsets": torch.full((experts + 1,), -7, device=device, dtype=torch.int32),
        "slots": torch.full((tokens * topk,), -7, device=device, dtype=torch.int32),
        "packed": torch.full((rows, hidden), 3.0, device=device, dtype=dtype),
        "inverse": torch.full((tokens, topk), -7, device=device, dtype=torch.int32),
    }


def _launch(lib, x, ids32, out, experts, alignment, rows):
    tokens, hidden = x.shape
    status = lib.moe_dispatch_noalloc(
        x.data_ptr(), DTYPE_CODES[x.dtype], ids32.data_ptr(), out["counts"].data_ptr(), out["offsets"].data_ptr(),
        out["slots"].data_ptr(), out["packed"].data_ptr(), out["inverse"].data_ptr(), tokens, hidden, experts,
        ids32.shape[1], alignment, rows, 1, current_stream_handle(x.device.index))
    lib.check(status, "moe_dispatch_noalloc")


def _noalloc_dispatch(lib, x, ids32, experts, alignment, rows):
    tokens, hidden = x.shape
    out = _buffers(tokens, hidden, experts, ids32.shape[1], rows, x.dtype, x.device)
    _launch(lib, x, ids32, out, experts, alignment, rows)
    return out


@pytest.mark.parametrize("calls", [
    # (tokens, hidden, experts, topk, alignment, dtype) per call; each later call is smaller
    [(3000, 256, 16, 2, 8, torch.bfloat16), (1500, 128, 8, 2, 8, torch.bfloat16)],
    [(4096, 64, 64, 6, 1, torch.float16), (700, 40, 5, 3, 16, torch.float32), (1, 8, 4, 1, 8, torch.bfloat16)],
])
def test_noalloc_dispatch_equals_workspace_dispatch(calls):
    lib = _lib.load_library()
    for seed, (tokens, hidden, experts, topk, alignment, dtype) in enumerate(calls):
        x, ids32, ids64, _ = make_transport_case(tokens, hidden, experts, topk, dtype, seed=seed + 11)
        ws = CudaWorkspace(tokens, hidden, experts, topk, dtype, alignment=alignment)
        ws.dispatch(x, ids32)
        got = _noalloc_dispatch(lib, x, ids32, experts, alignment, ws.capacity_rows)
        torch.cuda.synchronize()
        for name in ("counts", "offsets", "slots", "inverse"):
            assert torch.equal(got[name], getattr(ws, name)), (name, tokens)
        used = int(ws.offsets[-1])
        assert (raw_bits(got["packed"])[:used] == raw_bits(ws.packed)[:used]).all(), tokens


def test_random_noalloc_dispatches_in_a_row():
    """Thirty calls drawn from a fixed seed (fp16/fp32/bf16, any hidden size, 1-64
    experts, top-1 to top-8, alignment 1-128, 1-8000 tokens), one after the other,
    so each starts from the previous call's counters in the static array."""
    lib = _lib.load_library()
    rng = np.random.default_rng(61)
    for case in range(30):
        dtype = (torch.float16, torch.float32, torch.bfloat16)[int(rng.integers(0, 3))]
        experts = int(rng.integers(1, 65))
        topk = int(rng.integers(1, min(8, experts) + 1))
        tokens = int(np.exp(rng.uniform(0, np.log(8000))))
        hidden = int(rng.integers(1, 1500)) if rng.random() < 0.4 else 8 * int(rng.integers(1, 256))
        while tokens * topk * hidden > 4e7:
            tokens = max(1, tokens // 2)
        alignment = int(rng.choice([1, 3, 8, 16, 128]))
        print(f"case {case}: T={tokens} H={hidden} E={experts} K={topk} a={alignment} {dtype}", flush=True)
        x, ids32, _, _ = make_transport_case(tokens, hidden, experts, topk, dtype, seed=200 + case)
        ws = CudaWorkspace(tokens, hidden, experts, topk, dtype, alignment=alignment)
        ws.dispatch(x, ids32)
        got = _noalloc_dispatch(lib, x, ids32, experts, alignment, ws.capacity_rows)
        torch.cuda.synchronize()
        for name in ("counts", "offsets", "slots", "inverse"):
            assert torch.equal(got[name], getattr(ws, name)), (name, case)
        used = int(ws.offsets[-1])
        assert (raw_bits(got["packed"])[:used] == raw_bits(ws.packed)[:used]).all(), case


def test_noalloc_dispatch_validates_like_dispatch():
    lib = _lib.load_library()
    # The same argument checks run before any launch: an undersized packed buffer
    # (real device buffers throughout, so a check that stopped refusing would
    # write a wrong layout, not fault).
    x, ids32, _, _ = make_transport_case(10, 64, 8, 2, torch.bfloat16, seed=1)
    out = _buffers(10, 64, 8, 2, 79, x.dtype, x.device)
    args = [out[k].data_ptr() for k in ("counts", "offsets", "slots", "packed", "inverse")]
    stream = current_stream_handle(x.device.index)
    status = lib.moe_dispatch_noalloc(x.data_ptr(), 2, ids32.data_ptr(), *args, 10, 64, 8, 2, 8, 79, 1, stream)
    assert status == 4 and b"needs 80" in lib.moe_last_error()
    # 65 experts: outside the limits.
    out = _buffers(10, 64, 65, 2, 80, x.dtype, x.device)
    args = [out[k].data_ptr() for k in ("counts", "offsets", "slots", "packed", "inverse")]
    assert lib.moe_dispatch_noalloc(x.data_ptr(), 2, ids32.data_ptr(), *args, 10, 64, 65, 2, 8, 80, 1, stream) == 2
    torch.cuda.synchronize()
    assert int((out["packed"].float() != 3.0).sum()) == 0  # nothing was written


def test_noalloc_dispatch_replays_from_a_captured_graph():
    """One call before capture (the array's address is looked up then), then the
    entry point inside a captured graph: each replay, on new ids and rows written
    into the captured inputs, equals moe_dispatch bit for bit."""
    lib = _lib.load_library()
    tokens, hidden, experts, topk, alignment = 777, 128, 16, 2, 8
    x, ids32, _, _ = make_transport_case(tokens, hidden, experts, topk, torch.bfloat16, seed=3)
    ws = CudaWorkspace(tokens, hidden, experts, topk, torch.bfloat16, alignment=alignment)
    rows = ws.capacity_rows
    _noalloc_dispatch(lib, x, ids32, experts, alignment, rows)  # before capture
    out = _buffers(tokens, hidden, experts, topk, rows, x.dtype, x.device)
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            _launch(lib, x, ids32, out, experts, alignment, rows)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    for seed in (4, 5):
        x_new, ids_new, _, _ = make_transport_case(tokens, hidden, experts, topk, torch.bfloat16, seed=seed)
        x.copy_(x_new)
        ids32.copy_(ids_new)
        ws.dispatch(x, ids32)  # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for name in ("counts", "offsets", "slots", "inverse"):
            assert torch.equal(out[name], getattr(ws, name)), (name, seed)
        used = int(ws.offsets[-1])
        assert (raw_bits(out["packed"])[:used] == raw_bits(ws.packed)[:used]).all(), seed
