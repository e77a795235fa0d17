"""Device buffers of the HIP transport, and launches pre-bound to them.

A ``CudaWorkspace`` is the reference's transport workspace
(``src/moe_dispatch/workspace.py:7-87``) on the gfx950 kernels: the constructor
arguments, the buffer attributes (``counts``, ``offsets``, ``slots``,
``packed``, ``inverse``, ``output``), ``capacity_rows``, ``workspace_bytes``
and the two hot-path methods keep their names and meaning. Top-k may be 1..8.

Design. Every buffer the kernels write belongs to the workspace, so their
addresses, the sizes and the dtype code are fixed when it is built. The
workspace binds the two C-ABI calls once (``_Bound``); a ``dispatch`` or
``combine`` call then checks only the caller's tensors (shape, dtype, device,
contiguity: the checks the reference extension makes with ``TORCH_CHECK``,
raising ``RuntimeError``) and makes one ctypes call on the current stream.
Expert ids are not range-checked here (the kernels skip out-of-range ids, as
the reference's do); ``ops.dispatch`` checks them.

A workspace also holds the buffers of a ranked route (``tile_ranks``,
``tile_counts``; ``rank_tile`` tokens per tile, 0 when the shape has none):
the fused router can write the in-tile ranks and per-tile counts itself,
after which ``dispatch_ranked`` runs only the pack pass. ``dispatch_rows`` and
``dispatch_ranked_rows`` write the same layout without copying rows: instead
of ``packed``, ``row_src`` receives each packed row's token (-1 for padding),
which the gathered gate/up GEMM reads x through.

One workspace serves one invocation at a time: its outputs are views that the
next call overwrites.
"""

import torch

from ._extension import DTYPE_CODES, current_stream_handle, get_extension

MAX_EXPERTS = 64
MAX_TOPK = 8
_INT32_LIMIT = 2**31 - 1


def capacity_rows(tokens, experts, topk, alignment):
    """Rows ``packed`` must hold (the reference's formula, ``workspace.py:29-34``).

    With alignment 1 the packed rows are exactly the assignments. Otherwise
    each expert's span is rounded up to a multiple of the alignment, which adds
    at most alignment - 1 rows per expert; the bound adds one spare row and is
    itself rounded up to the alignment.
    """
    assignments = tokens * topk
    if alignment == 1:
        return assignments
    bound = assignments + experts * (alignment - 1) + 1
    return -(-bound // alignment) * alignment


def _check_shape_arguments(tokens, hidden, experts, topk, dtype, alignment):
    if tokens < 0 or hidden < 1 or not 1 <= experts <= MAX_EXPERTS or not 1 <= topk <= MAX_TOPK:
        raise ValueError("supports T>=0, H>=1, 1..64 experts, and topk=1..8")
    if tokens * topk > _INT32_LIMIT or hidden > _INT32_LIMIT:
        raise ValueError("shape exceeds int32 indexing capacity")
    if dtype not in DTYPE_CODES:
        raise ValueError("HIP workspace supports FP16, FP32, and BF16")
    if not 1 <= alignment <= 128:
        raise ValueError("alignment must be 1..128")
    if capacity_rows(tokens, experts, topk, alignment) > _INT32_LIMIT:
        raise ValueError("padded capacity exceeds int32 indexing capacity")


class _Bound:
    """The workspace's two C-ABI calls with every argument but the caller's tensors bound."""

    def __init__(self, ws):
        lib = ws.extension.lib
        tokens, hidden, experts, topk = ws.shape
        nbytes = ws.scratch.numel()
        code = DTYPE_CODES[ws.dtype]
        self.lib = lib
        self.code = code
        self.device_index = ws.device.index if ws.device.index is not None else torch.cuda.current_device()
        self.after_ids = (ws.counts.data_ptr(), ws.offsets.data_ptr(), ws.slots.data_ptr(),
                          ws.packed.data_ptr(), ws.inverse.data_ptr(), ws.scratch.data_ptr(), nbytes,
                          tokens, hidden, experts, topk, ws.alignment, ws.capacity_rows,
                          int(bool(ws.vectorized)))
        self.ranked_after_ids = (ws.counts.data_ptr(), ws.offsets.data_ptr(), ws.slots.data_ptr(),
                                 ws.packed.data_ptr(), ws.inverse.data_ptr(), ws.tile_ranks.data_ptr(),
                                 ws.tile_counts.data_ptr(), ws.tile_counts.numel() * 4, ws.rank_tile, tokens,
                                 hidden, experts, topk, ws.alignment, ws.capacity_rows, int(bool(ws.vectorized)))
        index = (ws.counts.data_ptr(), ws.offsets.data_ptr(), ws.slots.data_ptr(), ws.inverse.data_ptr(),
                 ws.row_src.data_ptr())
        self.rows_after_ids = index + (ws.scratch.data_ptr(), nbytes, tokens, experts, topk, ws.alignment,
                                       ws.capacity_rows)
        self.ranked_rows_after_ids = index + (ws.tile_ranks.data_ptr(), ws.tile_counts.data_ptr(),
                                              ws.tile_counts.numel() * 4, ws.rank_tile, tokens, experts, topk,
                                              ws.alignment, ws.capacity_rows)
        self.output = ws.output.data_ptr()
        self.inverse = ws.inverse.data_ptr()
        self.x_shape = (tokens, hidden)
        self.ids_shape = (tokens, topk)
        self.assignments = tokens * topk
        self.dtype = ws.dtype
        self.device = ws.device
        self.name = "dispatch_out" if ws.alignment == 1 else "dispatch_aligned_out"

    def _require(self, t, shape, dtype, what):
        if not isinstance(t, torch.Tensor):
            raise RuntimeError(f"{what} must be a tensor")
        if t.device != self.device:
            raise RuntimeError(f"{what}: expected a tensor on {self.device}, got {t.device}")
        if tuple(t.shape) != shape or t.dtype != dtype:
            raise RuntimeError(f"{what}: expected {dtype} {list(shape)}, got {t.dtype} {list(t.shape)}")
        if not t.is_contiguous():
            raise RuntimeError(f"{what} must be contiguous")

    def dispatch(self, x, ids32):
        self._require(x, self.x_shape, self.dtype, "x")
        self._require(ids32, self.ids_shape, torch.int32, "ids")
        status = self.lib.moe_dispatch(x.data_ptr(), self.code, ids32.data_ptr(), *self.after_ids,
                                       current_stream_handle(self.device_index))
        self.lib.check(status, self.name)

    def dispatch_ranked(self, x, ids32):
        self._require(x, self.x_shape, self.dtype, "x")
        self._require(ids32, self.ids_shape, torch.int32, "ids")
        status = self.lib.moe_dispatch_ranked(x.data_ptr(), self.code, ids32.data_ptr(), *self.ranked_after_ids,
                                              current_stream_handle(self.device_index))
        self.lib.check(status, self.name)

    def dispatch_rows(self, ids32, ranked):
        self._require(ids32, self.ids_shape, torch.int32, "ids")
        if ranked:
            status = self.lib.moe_dispatch_ranked_rows(ids32.data_ptr(), *self.ranked_rows_after_ids,
                                                       current_stream_handle(self.device_index))
        else:
            status = self.lib.moe_dispatch_rows(ids32.data_ptr(), *self.rows_after_ids,
                                                current_stream_handle(self.device_index))
        self.lib.check(status, "dispatch_rows")

    def combine(self, expert_output, weights):
        # Any row count that holds every assignment (the reference's combine_out
        # takes the same); rows of `inverse` past it are skipped by the kernel.
        rows = expert_output.shape[0] if isinstance(expert_output, torch.Tensor) and expert_output.dim() == 2 else -1
        if rows < self.assignments:
            raise RuntimeError(f"expert output must be [rows >= {self.assignments}, {self.x_shape[1]}]")
        self._require(expert_output, (rows, self.x_shape[1]), self.dtype, "expert output")
        self._require(weights, self.ids_shape, torch.float32, "weights")
        tokens, hidden = self.x_shape
        status = self.lib.moe_combine(expert_output.data_ptr(), self.code, self.inverse, weights.data_ptr(),
                                      self.output, tokens, hidden, self.ids_shape[1], rows,
                                      current_stream_handle(self.device_index))
        self.lib.check(status, "combine_out")


class CudaWorkspace:
    """Reusable transport buffers on one GPU. Use one workspace per concurrent invocation."""

    def __init__(self, tokens, hidden, experts, topk, dtype, vectorized=True, device="cuda",
                 extension=None, alignment=1):
        _check_shape_arguments(tokens, hidden, experts, topk, dtype, alignment)
        device = torch.device(device)
        if device.type != "cuda" or not torch.cuda.is_available():
            raise RuntimeError("CudaWorkspace requires a CUDA GPU device (an AMD GPU under ROCm)")
        if device.index is None:
            device = torch.device("cuda", torch.cuda.current_device())
        self.shape = (tokens, hidden, experts, topk)
        self.dtype = dtype
        self.device = device
        self.vectorized = vectorized
        self.alignment = alignment
        self.capacity_rows = capacity_rows(tokens, experts, topk, alignment)
        self.extension = extension if extension is not None else get_extension()
        rows = self.capacity_rows
        assignments = tokens * topk
        # Tokens per tile of a ranked route for this shape (0: none) and its count table.
        self.rank_tile = self.extension.router_rank_tile(tokens, experts)
        tiles = -(-tokens // self.rank_tile) if self.rank_tile > 0 else 0
        # name -> (shape, dtype); `scratch` holds the dispatch kernels' per-chunk count table.
        layout = {
            "counts": ((experts,), torch.int32),
            "offsets": ((experts + 1,), torch.int32),
            "slots": ((assignments,), torch.int32),
            "packed": ((rows, hidden), dtype),
            "inverse": ((tokens, topk), torch.int32),
            "output": ((tokens, hidden), dtype),
            "scratch": ((max(self.extension.scratch_bytes(tokens, experts, topk), 4),), torch.uint8),
            "tile_ranks": ((assignments if tiles else 1,), torch.int32),
            "tile_counts": ((max(tiles * experts, 1),), torch.int32),
            "row_src": ((rows,), torch.int32),
        }
        self._names = tuple(layout)
        for name, (shape, kind) in layout.items():
            setattr(self, name, torch.empty(shape, device=device, dtype=kind))
        self._bound = _Bound(self)

    def dispatch(self, x, ids32, ids64=None):
        """Hot path: contiguous x[T,H] and int32 ids[T,K] with in-range ids (ids64 is unused)."""
        self._bound.dispatch(x, ids32)

    def dispatch_ranked(self, x, ids32):
        """dispatch() after a ranked route that wrote this workspace's ``tile_ranks``
        and ``tile_counts`` for these ids (``rank_tile`` > 0): the pack pass only."""
        if self.rank_tile <= 0:
            raise RuntimeError("this workspace's shape has no ranked route (rank_tile == 0)")
        self._bound.dispatch_ranked(x, ids32)

    def dispatch_rows(self, ids32):
        """The dispatch layout (counts, offsets, slots, inverse) without copying
        rows: ``row_src`` receives each packed row's token, -1 for padding rows."""
        self._bound.dispatch_rows(ids32, ranked=False)

    def dispatch_ranked_rows(self, ids32):
        """dispatch_rows() after a ranked route (as ``dispatch_ranked``)."""
        if self.rank_tile <= 0:
            raise RuntimeError("this workspace's shape has no ranked route (rank_tile == 0)")
        self._bound.dispatch_rows(ids32, ranked=True)

    def combine(self, expert_output, weights):
        """Hot path: expert_output[R, H] (R >= T*K) of the workspace dtype, fp32 weights[T,K]."""
        self._bound.combine(expert_output, weights)

    @property
    def workspace_bytes(self):
        tensors = (getattr(self, name) for name in self._names)
        return sum(t.numel() * t.element_size() for t in tensors)
