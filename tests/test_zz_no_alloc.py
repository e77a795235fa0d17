"""moe_dispatch_noalloc against moe_dispatch, through the C ABI.

The allocation-free entry point keeps its count table in the library's static
device array; on two calls in a row (the second smaller, so the array holds the
first call's counters when it starts) every output must equal what moe_dispatch
writes with a workspace scratch buffer, bit for bit: counts, offsets, slots,
inverse and every packed row inside the used spans.
"""

import pytest
import torch

from moe_dispatch import _lib
from moe_dispatch._extension import DTYPE_CODES, current_stream_handle
from moe_dispatch.routing import make_transport_case
from moe_dispatch.workspace import CudaWorkspace
from tests._helpers import gpu, raw_bits

pytestmark = gpu


def _noalloc_dispatch(lib, x, ids32, experts, alignment, rows):
    tokens, hidden = x.shape
    topk = ids32.shape[1]
    dev = x.device
    out = {
        "counts": torch.full((experts,), -7, device=dev, dtype=torch.int32),
        "offsets": torch.full((experts + 1,), -7, device=dev, dtype=torch.int32),
        "slots": torch.full((tokens * topk,), -7, device=dev, dtype=torch.int32),
        "packed": torch.full((rows, hidden), 3.0, device=dev, dtype=x.dtype),
        "inverse": torch.full((tokens, topk), -7, device=dev, dtype=torch.int32),
    }
    status = lib.moe_dispatch_noalloc(
        x.data_ptr(), DTYPE_CODES[x.dtype], ids32.data_ptr(), out["counts"].data_ptr(), out["offsets"].data_ptr(),
        out["slots"].data_ptr(), out["packed"].data_ptr(), out["inverse"].data_ptr(), tokens, hidden, experts,
        topk, alignment, rows, 1, current_stream_handle(dev.index))
    lib.check(status, "moe_dispatch_noalloc")
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


def test_noalloc_dispatch_validates_like_dispatch():
    lib = _lib.load_library()
    # The same argument checks run before any launch: an undersized packed buffer.
    x, ids32, _, _ = make_transport_case(10, 64, 8, 2, torch.bfloat16, seed=1)
    status = lib.moe_dispatch_noalloc(x.data_ptr(), 2, ids32.data_ptr(), 16, 16, 16, 16, 16, 10, 64, 8, 2, 8, 79,
                                      1, None)
    assert status == 4 and b"needs 80" in lib.moe_last_error()
    assert lib.moe_dispatch_noalloc(None, 2, None, 16, 16, None, None, None, 10, 64, 65, 2, 8, 80, 1, None) == 2
