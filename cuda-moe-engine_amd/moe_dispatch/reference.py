"""PyTorch transport variant (``implementation="torch"``), usable on CPU and GPU.

Same contract as the reference ``TorchWorkspace`` (``src/moe_dispatch/reference.py:6-82``):
preallocated buffers, ``dispatch(x, ids32, ids64)`` filling ``counts``,
``offsets``, ``inverse`` and ``packed``, and ``combine(expert_output, weights)``
reducing in fp32 into a reusable ``output`` view.

How it computes them:

* counts by a scatter-add of ones, offsets by a cumulative sum of the spans
  rounded up to the alignment;
* a stable sort of the flat expert ids orders the assignments by (expert,
  flat index p = t*K + k), so the packed order is the canonical one the HIP
  kernels produce (the reference's unstable sort leaves the order within an
  expert unspecified, and the order is not part of its contract);
* destination row = padded start of the expert + rank within the expert;
* combine: the K rows of each token are gathered through ``inverse`` and
  summed in fp32 in k order, one multiply and one add per term, then cast
  once; this is the HIP combine's arithmetic.
"""

import torch

_BUFFERS = ("counts", "offsets", "inverse", "sorted_ids", "order", "token_of", "destination", "position",
            "unit", "packed", "gathered", "output", "accumulated", "term")


class TorchWorkspace:
    """Preallocated PyTorch transport with reusable outputs and FP32 accumulation."""

    def __init__(self, tokens, hidden, experts, topk, dtype, device="cuda", alignment=1):
        if not 1 <= alignment <= 128:
            raise ValueError("alignment must be 1..128")
        from .workspace import capacity_rows

        n = tokens * topk
        self.alignment = alignment
        self.capacity_rows = capacity_rows(tokens, experts, topk, alignment)
        self.tokens, self.hidden, self.topk, self.experts = tokens, hidden, topk, experts
        device = torch.device(device)
        self.device = device
        i32, i64, f32 = torch.int32, torch.int64, torch.float32
        self.counts = torch.empty(experts, device=device, dtype=i32)
        self.offsets = torch.empty(experts + 1, device=device, dtype=i32)
        self.inverse = torch.empty((tokens, topk), device=device, dtype=i64)
        self.sorted_ids = torch.empty(n, device=device, dtype=i64)
        self.order = torch.empty(n, device=device, dtype=i64)
        self.token_of = torch.empty(n, device=device, dtype=i64)
        self.destination = torch.empty(n, device=device, dtype=i64)
        self.position = torch.arange(n, device=device, dtype=i64)
        self.unit = torch.ones(n, device=device, dtype=i32)
        self.packed = torch.empty((self.capacity_rows, hidden), device=device, dtype=dtype)
        self.gathered = torch.empty((n, hidden), device=device, dtype=dtype)
        self.output = torch.empty((tokens, hidden), device=device, dtype=dtype)
        self.accumulated = torch.empty((tokens, hidden), device=device, dtype=f32)
        self.term = torch.empty((tokens, hidden), device=device, dtype=f32)

    def dispatch(self, x, ids32, ids64):
        flat = ids64.reshape(-1)
        self.counts.zero_()
        self.counts.scatter_add_(0, flat, self.unit)
        spans = (self.counts + self.alignment - 1) // self.alignment * self.alignment
        self.offsets[:1].zero_()
        torch.cumsum(spans, dim=0, dtype=torch.int32, out=self.offsets[1:])
        # Stable sort: packed order is (expert, flat assignment index).
        torch.sort(flat, stable=True, out=(self.sorted_ids, self.order))
        torch.div(self.order, self.topk, rounding_mode="floor", out=self.token_of)
        # Rank of each sorted entry inside its expert = position - unpadded start.
        unpadded = torch.cumsum(self.counts, dim=0) - self.counts
        rank = self.position - unpadded.index_select(0, self.sorted_ids)
        torch.add(self.offsets.index_select(0, self.sorted_ids).long(), rank, out=self.destination)
        self.inverse.reshape(-1).scatter_(0, self.order, self.destination)
        if self.alignment > 1:
            self.packed.zero_()
        self.packed.index_copy_(0, self.destination, x.index_select(0, self.token_of))

    def combine(self, expert_output, weights):
        torch.index_select(expert_output, 0, self.inverse.reshape(-1), out=self.gathered)
        rows = self.gathered.view(self.tokens, self.topk, self.hidden)
        w = weights.to(torch.float32)
        acc, term = self.accumulated, self.term
        # k order, separate multiply and add (the HIP combine's sequence).
        torch.mul(rows[:, 0], w[:, 0:1], out=acc)
        for k in range(1, self.topk):
            torch.mul(rows[:, k], w[:, k:k + 1], out=term)
            acc.add_(term)
        self.output.copy_(acc)

    @property
    def workspace_bytes(self):
        return sum(getattr(self, name).numel() * getattr(self, name).element_size() for name in _BUFFERS)
