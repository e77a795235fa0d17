"""Grouped expert matmuls with an explicit backend choice.

Mirrors ``src/moe_dispatch/experts.py:7-41``. Backends: ``hip`` (the gfx950
MFMA grouped GEMM of ``libmoe_hip.so``) and ``torch`` (``F.grouped_mm``, or a
per-expert ``mm`` loop where grouped_mm is unavailable). There is no Triton
backend and no automatic fallback from ``hip``.
"""

from collections import Counter

import torch

BACKENDS = ("auto", "torch", "hip")

# Which path each torch-backend call took ("grouped_mm" or "mm_loop"), counted
# per call so that a caller can label a timed run by the path that ran in it.
torch_backend_calls = Counter()


def resolve_backend(device, requested="auto"):
    if requested == "triton":
        raise RuntimeError("the Triton backend does not exist in this build; use 'hip' or 'torch'")
    if requested not in BACKENDS:
        raise ValueError("expert backend must be auto, torch, or hip")
    if torch.device(device).type != "cuda":
        if requested == "hip":
            raise RuntimeError("the HIP grouped GEMM requires an AMD GPU")
        return "torch"
    if requested == "auto":
        return "hip"
    return requested


def _torch_grouped(x, weight, ends):
    logical = weight.transpose(-2, -1)
    function = getattr(torch.nn.functional, "grouped_mm", getattr(torch, "_grouped_mm", None))
    if function is not None:
        try:
            result = function(x, logical, offs=ends)
            torch_backend_calls["grouped_mm"] += 1
            return result, "grouped_mm"
        except (RuntimeError, NotImplementedError):
            pass
    # Per-expert loop (host reads the offsets).
    out = torch.zeros((x.shape[0], weight.shape[1]), device=x.device, dtype=x.dtype)
    bounds = [0] + ends.tolist()
    for e in range(weight.shape[0]):
        s, t = bounds[e], bounds[e + 1]
        if t > s:
            out[s:t] = x[s:t] @ logical[e]
    torch_backend_calls["mm_loop"] += 1
    return out, "mm_loop"


def grouped_linear(x, weight, ends, *, backend, output=None, offsets=None):
    """``out[r] = x[r] @ weight[e]^T`` for rows of expert e; ``weight`` is ``[E,N,K]``.

    ``ends`` are the device-resident group ends (``offsets[1:]``); the HIP
    backend takes the full ``offsets`` (given or rebuilt from ``ends``).
    Rows at or past ``ends[-1]`` are not written by the HIP backend.
    """
    if backend == "hip":
        from ._extension import get_extension

        if offsets is None:
            offsets = torch.cat([ends.new_zeros(1), ends]).contiguous()
        if output is None:
            output = torch.empty((x.shape[0], weight.shape[1]), device=x.device, dtype=x.dtype)
        get_extension().grouped_gemm_out(x, weight, offsets, output)
        return output
    if backend != "torch":
        raise ValueError(f"unknown backend {backend}")
    result, _ = _torch_grouped(x, weight, ends)
    if output is not None:
        output.copy_(result)
        return output
    return result


def backend_label(before, after):
    """The torch GEMM path(s) taken between two snapshots of ``torch_backend_calls``:
    "grouped_mm", "mm_loop", "mixed" (both ran) or "none"."""
    ran = sorted(k for k in ("grouped_mm", "mm_loop") if after[k] > before[k])
    return ran[0] if len(ran) == 1 else ("mixed" if ran else "none")


def swiglu_reference(projection):
    gate, up = projection.chunk(2, dim=-1)
    # FP32 activation and multiply, then one cast (the fused kernels do the same).
    return (torch.nn.functional.silu(gate.float()) * up.float()).to(projection.dtype)
