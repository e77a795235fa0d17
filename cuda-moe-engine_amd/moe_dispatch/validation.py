"""Acceptance checks of a transport workspace (the invariants of ``src/moe_dispatch/validation.py:9-61``).

``validate_case`` runs one dispatch and one combine through any workspace that
has the transport interface (``CudaWorkspace`` or ``TorchWorkspace``) and then
checks, each by a route independent of the kernels:

1. counts equal a histogram of the ids;
2. each expert's span is its count rounded up to the alignment, spans start
   at 0 and end at the padded total;
3. the inverse map sends the T*K assignments to distinct rows in range (a
   permutation of 0..T*K-1 when the alignment is 1);
4. gathering the packed rows through the inverse map gives x back, bit for bit;
5. every assignment's row lies in its own expert's span;
6. padding rows inside the spans are zero;
7. the weighted combine of an arbitrary expert output equals the fp32 sum
   within the dtype's tolerance.

``run_tests`` is the runtime suite the reference runs on a GPU
(``validation.py:64-104``): six shapes, fp32 and fp16, the PyTorch variant and
the scalar and vectorized HIP paths.
"""

import torch

from .routing import make_case

# Combine tolerance per row dtype (the one rounding of the fp32 sum dominates).
_COMBINE_TOLERANCE = {torch.bfloat16: 2e-2, torch.float16: 2e-3, torch.float32: 2e-5}

# (tokens, hidden, experts, topk) of the runtime suite; even-indexed cases are skewed.
SUITE_SHAPES = ((0, 17, 8, 2), (1, 17, 8, 2), (7, 31, 8, 1), (33, 128, 8, 2), (129, 512, 16, 2),
                (257, 1024, 16, 2))


def _exact(actual, expected, what):
    if not torch.equal(actual, expected.to(actual.dtype)):
        raise AssertionError(f"{what}: expected {expected.tolist()}, got {actual.tolist()}"
                             if actual.numel() <= 64 else f"{what} differs")


def _check_counts(ws, flat_ids, experts):
    histogram = torch.zeros(experts, dtype=torch.int64, device=flat_ids.device)
    histogram.index_add_(0, flat_ids, torch.ones_like(flat_ids))
    _exact(ws.counts, histogram, "counts")
    return histogram


def _check_spans(ws, histogram, alignment):
    spans = torch.div(histogram + alignment - 1, alignment, rounding_mode="floor") * alignment
    offsets = ws.offsets.long()
    _exact(offsets[1:] - offsets[:-1], spans, "span widths")
    if int(offsets[0]) != 0 or int(offsets[-1]) != int(spans.sum()):
        raise AssertionError("offsets must start at 0 and end at the padded total")
    return offsets


def _check_inverse(ws, rows_total, alignment):
    inverse = ws.inverse.reshape(-1).long()
    if alignment == 1:
        _exact(inverse.sort().values, torch.arange(rows_total, device=inverse.device), "inverse permutation")
        return inverse
    if inverse.numel():
        if int(inverse.min()) < 0 or int(inverse.max()) >= ws.packed.shape[0]:
            raise AssertionError("inverse row out of range")
        if inverse.unique().numel() != inverse.numel():
            raise AssertionError("two assignments share a packed row")
    return inverse


def _check_round_trip(ws, x, inverse, topk):
    gathered = ws.packed.index_select(0, inverse)
    expected = x.repeat_interleave(topk, dim=0)
    if not torch.equal(gathered, expected):
        raise AssertionError("packed rows do not reproduce x through the inverse map")


def _check_membership(inverse, offsets, flat_ids):
    owner = torch.searchsorted(offsets[1:], inverse, right=True)
    _exact(owner, flat_ids, "expert of each packed row")


def _check_padding(ws, inverse, offsets):
    used = torch.zeros(ws.packed.shape[0], dtype=torch.bool, device=inverse.device)
    used[inverse] = True
    inside = torch.arange(ws.packed.shape[0], device=inverse.device) < offsets[-1]
    padding = ws.packed[inside & ~used]
    if padding.numel() and bool(padding.ne(0).any()):
        raise AssertionError("padding rows are not zero")


def _check_combine(ws, x, inverse, weights, seed):
    tokens, hidden = x.shape
    topk = weights.shape[1]
    generator = torch.Generator(device=x.device).manual_seed(seed + 501)
    per_assignment = torch.randn((tokens * topk, hidden), device=x.device, dtype=x.dtype, generator=generator)
    expert_output = torch.empty_like(ws.packed)
    expert_output[inverse] = per_assignment
    ws.combine(expert_output, weights)
    expected = torch.bmm(weights.float().unsqueeze(1), per_assignment.float().view(tokens, topk, hidden))
    expected = expected.squeeze(1).to(x.dtype)
    tolerance = _COMBINE_TOLERANCE[x.dtype]
    torch.testing.assert_close(ws.output, expected, rtol=tolerance, atol=tolerance)
    error = (ws.output.float() - expected.float()).abs()
    return float(error.max()) if error.numel() else 0.0


@torch.inference_mode()
def validate_case(workspace, x, ids32, ids64, weights, experts, seed):
    """Dispatch and combine through ``workspace``; raise on a broken invariant, return the combine error."""
    topk = ids32.shape[1]
    alignment = getattr(workspace, "alignment", 1)
    flat_ids = ids64.reshape(-1)
    workspace.dispatch(x, ids32, ids64)
    histogram = _check_counts(workspace, flat_ids, experts)
    offsets = _check_spans(workspace, histogram, alignment)
    inverse = _check_inverse(workspace, flat_ids.numel(), alignment)
    _check_round_trip(workspace, x, inverse, topk)
    _check_membership(inverse, offsets, flat_ids)
    if alignment > 1:
        _check_padding(workspace, inverse, offsets)
    return _check_combine(workspace, x, inverse, weights, seed)


def _suite_cases():
    for dtype in (torch.float32, torch.float16):
        for index, shape in enumerate(SUITE_SHAPES):
            yield dtype, shape, ("skewed" if index % 2 == 0 else "balanced"), 42 + index


@torch.inference_mode()
def run_tests(extension=None):
    """The runtime transport suite on the GPU: 2 dtypes x 6 shapes x 3 workspaces = 36 checks."""
    from .reference import TorchWorkspace
    from .workspace import CudaWorkspace

    errors = []
    for dtype, (tokens, hidden, experts, topk), pattern, seed in _suite_cases():
        x, ids32, ids64, weights = make_case(tokens, hidden, experts, topk, dtype, pattern, seed)
        candidates = [TorchWorkspace(tokens, hidden, experts, topk, dtype)]
        candidates += [CudaWorkspace(tokens, hidden, experts, topk, dtype, vectorized=vectorized,
                                     extension=extension) for vectorized in (False, True)]
        errors += [validate_case(ws, x, ids32, ids64, weights, experts, seed) for ws in candidates]
    torch.cuda.synchronize()
    summary = {
        "passed": len(errors),
        "failed": 0,
        "max_absolute_error": max(errors, default=0.0),
        "coverage": "FP32/FP16; K=1/2; empty batch; empty experts; skew; odd H",
    }
    print(f"Correctness: {summary['passed']} checks passed; "
          f"max absolute error {summary['max_absolute_error']:.3g}", flush=True)
    return summary
