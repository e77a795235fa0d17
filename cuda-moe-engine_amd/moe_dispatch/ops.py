"""Standalone transport API with input validation (``PackedTokens``, ``dispatch``, ``combine``).

Public surface of the reference's ``src/moe_dispatch/ops.py:8-77``: the same
names, argument meaning and exception types (``ValueError`` for shapes,
devices, ranges and workspace mismatches, ``TypeError`` for dtypes,
``RuntimeError`` without a GPU). Top-k may be 1..8 here (the reference allows
1 or 2).

The checks are kept as ordered rule tables, so each error names the first
rule a call breaks. The expert-id range check reads the ids' minimum and
maximum back to the host in one transfer (it synchronises the stream): hot
loops should validate once and then call ``CudaWorkspace.dispatch`` directly.
"""

from dataclasses import dataclass

import torch

from .workspace import MAX_EXPERTS, MAX_TOPK, CudaWorkspace

_ROW_DTYPES = (torch.float16, torch.float32, torch.bfloat16)
_ID_DTYPES = (torch.int32, torch.int64)


@dataclass(frozen=True)
class PackedTokens:
    """The packed rows, inverse map, counts and offsets of one dispatch, as views of
    its workspace's buffers: the next call on that workspace overwrites them, so
    clone what must outlive it."""

    packed: torch.Tensor
    inverse: torch.Tensor
    counts: torch.Tensor
    offsets: torch.Tensor
    workspace: CudaWorkspace


# (predicate over (x, ids, experts), exception type, message), checked in order.
_INPUT_RULES = (
    (lambda x, ids, e: x.ndim == 2 and ids.ndim == 2, ValueError, "expected x[T,H] and expert_ids[T,K]"),
    (lambda x, ids, e: x.shape[0] == ids.shape[0] and x.shape[1] >= 1, ValueError,
     "token dimensions must match and H must be positive"),
    (lambda x, ids, e: x.dtype in _ROW_DTYPES, TypeError, "x must be FP16, FP32, or BF16"),
    (lambda x, ids, e: ids.dtype in _ID_DTYPES, TypeError, "expert_ids must be int32 or int64"),
    (lambda x, ids, e: x.device == ids.device, ValueError, "x and expert_ids must be on the same device"),
    (lambda x, ids, e: x.is_contiguous() and ids.is_contiguous(), ValueError, "inputs must be contiguous"),
    (lambda x, ids, e: isinstance(e, int) and 1 <= e <= MAX_EXPERTS, ValueError,
     "experts must be an integer in 1..64"),
    (lambda x, ids, e: 1 <= ids.shape[1] <= MAX_TOPK, ValueError, "topk must be in 1..8"),
    (lambda x, ids, e: not x.requires_grad, ValueError,
     "HIP operators are forward-only; detach inputs or use inference_mode"),
)


def validate_inputs(x, expert_ids, experts):
    """Raise on the first broken rule; the last check reads the id range back to the host."""
    for holds, error, message in _INPUT_RULES:
        if not holds(x, expert_ids, experts):
            raise error(message)
    if expert_ids.numel():
        low, high = (int(v) for v in torch.stack(torch.aminmax(expert_ids)).tolist())
        if low < 0 or high >= experts:
            raise ValueError("expert_ids contains an out-of-range expert")


@torch.inference_mode()
def dispatch(x, expert_ids, experts, *, workspace=None, vectorized=True, alignment=1):
    """Group each token's K routed copies by expert (the reference's ``dispatch``).

    The expert-id range check reads the ids back to the host and so waits for
    the stream; loops that call this repeatedly on checked ids should call the
    workspace's ``dispatch`` instead."""
    validate_inputs(x, expert_ids, experts)
    if not x.is_cuda:
        raise RuntimeError("dispatch requires a GPU; TorchWorkspace provides the CPU reference")
    signature = (x.shape[0], x.shape[1], experts, expert_ids.shape[1])
    if workspace is None:
        workspace = CudaWorkspace(*signature, x.dtype, vectorized=vectorized, device=x.device,
                                  alignment=alignment)
    elif workspace.shape != signature or workspace.dtype != x.dtype:
        raise ValueError("workspace shape/dtype does not match inputs")
    if workspace.packed.device != x.device:
        raise ValueError("workspace device does not match inputs")
    ids32 = expert_ids if expert_ids.dtype == torch.int32 else expert_ids.to(torch.int32)
    workspace.dispatch(x, ids32)
    return PackedTokens(workspace.packed, workspace.inverse, workspace.counts, workspace.offsets, workspace)


# (predicate over (expert_output, batch, weights), exception type, message), checked in order.
_COMBINE_RULES = (
    (lambda y, b, w: w.shape == b.inverse.shape, ValueError, "weights must have shape [T,K]"),
    (lambda y, b, w: y.shape == b.packed.shape and y.dtype == b.packed.dtype, ValueError,
     "expert output shape/dtype must match packed tokens"),
    (lambda y, b, w: w.device == b.packed.device and y.device == b.packed.device, ValueError,
     "all tensors must be on the workspace device"),
    (lambda y, b, w: w.is_contiguous() and y.is_contiguous(), ValueError,
     "expert output and weights must be contiguous"),
    (lambda y, b, w: w.is_floating_point(), TypeError, "weights must be floating point"),
)


@torch.inference_mode()
def combine(expert_output, batch, weights):
    """Sum each token's K expert rows weighted by its routing weights, in fp32 and
    in k order, into the workspace's output buffer (returned as a view that the
    next combine on that workspace overwrites)."""
    for holds, error, message in _COMBINE_RULES:
        if not holds(expert_output, batch, weights):
            raise error(message)
    fp32 = weights if weights.dtype == torch.float32 else weights.to(torch.float32)
    batch.workspace.combine(expert_output, fp32)
    return batch.workspace.output
