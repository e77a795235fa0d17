"""PyTorch transport variant (``implementation="torch"``), usable on CPU and GPU.

Restates the reference ``TorchWorkspace`` (``src/moe_dispatch/reference.py:6-82``):
counts by scatter-add, offsets by cumulative sum, a sort of the flat expert ids
to order the assignments, ``index_select``/``index_copy`` for the rows, and an
fp32 multiply + sum for the weighted combine. The sort is stable here, so the
permutation is the canonical one (the reference's unstable sort gives some
order within each expert; the order is not part of its contract).
"""

import torch


class TorchWorkspace:
    """Preallocated PyTorch transport with reusable outputs and FP32 accumulation."""

    def __init__(self, tokens, hidden, experts, topk, dtype, device="cuda", alignment=1):
        if not 1 <= alignment <= 128:
            raise ValueError("alignment must be 1..128")
        n = tokens * topk
        self.alignment = alignment
        self.capacity_rows = (
            n
            if alignment == 1
            else (n + experts * (alignment - 1) + 1 + alignment - 1) // alignment * alignment
        )
        self.tokens, self.hidden, self.topk, self.experts = tokens, hidden, topk, experts
        device = torch.device(device)
        self.device = device
        i32, i64 = torch.int32, torch.int64
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
        self.weighted = torch.empty((tokens, topk, hidden), device=device, dtype=torch.float32)
        self.output = torch.empty((tokens, hidden), device=device, dtype=dtype)
        self.accumulated = (
            self.output
            if dtype == torch.float32
            else torch.empty((tokens, hidden), device=device, dtype=torch.float32)
        )

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
        torch.mul(
            self.gathered.view(self.tokens, self.topk, self.hidden),
            weights.unsqueeze(-1),
            out=self.weighted,
        )
        torch.sum(self.weighted, dim=1, out=self.accumulated)
        if self.output is not self.accumulated:
            self.output.copy_(self.accumulated)

    @property
    def workspace_bytes(self):
        tensors = {t.data_ptr(): t for t in vars(self).values() if isinstance(t, torch.Tensor)}
        return sum(t.numel() * t.element_size() for t in tensors.values())
