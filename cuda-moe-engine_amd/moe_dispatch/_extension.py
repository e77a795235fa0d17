"""Tensor-level operators over the C ABI, with the reference extension's names.

``get_extension()`` returns an object exposing the five functions of the
reference's pybind module (``src/moe_dispatch/_extension.py:52-58``,
``csrc/bindings.cpp:3-13``): ``dispatch_out``, ``dispatch_aligned_out``,
``combine_out``, ``swiglu_out`` and ``topk_route_out``, plus the fused router
and grouped GEMM entry points of this build. Each validates its tensors like
the reference's ``TORCH_CHECK`` calls (raising ``RuntimeError``) and launches
on the current torch stream without synchronising.
"""

from __future__ import annotations

from functools import lru_cache
from pathlib import Path

import torch

from . import _lib

DTYPE_CODES = {
    torch.float32: _lib.DTYPE_F32,
    torch.float16: _lib.DTYPE_F16,
    torch.bfloat16: _lib.DTYPE_BF16,
}
_DTYPES = DTYPE_CODES


def _check(condition, message):
    if not condition:
        raise RuntimeError(message)


def _check_gpu_tensor(tensor, anchor, name):
    _check(isinstance(tensor, torch.Tensor), f"{name} must be a tensor")
    _check(tensor.is_cuda, f"{name}: all tensors must be GPU tensors")
    _check(tensor.is_contiguous(), f"{name}: all tensors must be contiguous")
    _check(tensor.device == anchor.device, f"{name}: device mismatch")


def weight_row_stride(weight):
    """Elements from one row of a ``[E, N, K]`` weight tensor to the next when its
    rows are contiguous and evenly spaced (a contiguous tensor: K; a ``[:, :, :K]``
    view of row-padded storage: the padded length), else None."""
    if weight.dim() != 3:
        return None
    experts, rows, k = weight.shape
    if k > 1 and weight.stride(2) != 1:
        return None
    # Row j of expert e sits at element (e * rows + j) * stride.
    stride = weight.stride(1) if rows > 1 else (weight.stride(0) if experts > 1 else k)
    if stride < k or (experts > 1 and weight.stride(0) != rows * stride):
        return None
    return stride


def _check_weight(weight, anchor, name):
    """A GPU weight tensor on x's device whose rows the GEMM kernels can read: contiguous,
    or rows padded to a multiple of 8 elements (16-byte aligned rows)."""
    _check(isinstance(weight, torch.Tensor), f"{name} must be a tensor")
    _check(weight.is_cuda, f"{name}: all tensors must be GPU tensors")
    _check(weight.device == anchor.device, f"{name}: device mismatch")
    stride = weight_row_stride(weight)
    _check(stride is not None and stride % 8 == 0,
           f"{name}: weights must be contiguous, or [E, N, K] rows padded to a multiple of 8 elements")
    return stride


def current_stream_handle(device_index):
    """The current torch stream's HIP handle on a device (torch's raw accessor when it has one)."""
    raw = getattr(torch._C, "_cuda_getCurrentRawStream", None)
    if raw is not None:
        return raw(device_index)
    return torch.cuda.current_stream(device_index).cuda_stream


def _stream(device):
    index = device.index if device.index is not None else torch.cuda.current_device()
    return current_stream_handle(index)


def _ptr(tensor):
    return tensor.data_ptr() if tensor is not None else None


class HipExtension:
    """Operators of ``libmoe_hip.so`` on torch tensors."""

    def __init__(self):
        self.lib = _lib.load_library()

    # -- routing -------------------------------------------------------------
    def topk_route_out(self, logits, bias, ids32, ids64, weights):
        """Reference ``csrc/dispatch.cu:378-402``; K up to 8 here."""
        _check(logits.is_cuda and logits.is_contiguous() and logits.dim() == 2
               and logits.dtype == torch.float32, "expected FP32 GPU logits[T,E]")
        for name, t in (("bias", bias), ("ids32", ids32), ("ids64", ids64), ("weights", weights)):
            _check_gpu_tensor(t, logits, name)
        tokens, experts = logits.shape
        _check(1 <= experts <= 64, "routing supports 1..64 experts and int32 indexing")
        _check(bias.dim() == 1 and bias.numel() == experts and bias.dtype == torch.float32,
               "expected FP32 bias[E]")
        _check(ids32.dim() == 2 and ids32.shape[0] == tokens and ids32.dtype == torch.int32,
               "expected int32 ids[T,K]")
        topk = ids32.shape[1]
        _check(1 <= topk <= min(experts, 8) and ids64.shape == ids32.shape
               and ids64.dtype == torch.int64 and weights.shape == ids32.shape
               and weights.dtype == torch.float32,
               "expected top-k (K <= min(E, 8)) int64 IDs and FP32 weights")
        status = self.lib.moe_topk_route(
            _ptr(logits), _ptr(bias), _ptr(ids32), _ptr(ids64), _ptr(weights),
            tokens, experts, topk, _stream(logits.device))
        self.lib.check(status, "topk_route_out")

    def router_scratch_bytes(self, experts, hidden):
        return int(self.lib.moe_router_scratch_bytes(experts, hidden))

    def router_fused_out(self, x, router_weight, bias, ids32, ids64, weights, logits=None, scratch=None):
        """Fused fp32 router projection + top-k (replaces ``layer.py:123,134``).

        ``scratch`` (uint8, at least ``router_scratch_bytes(E, H)`` bytes, on the
        device) receives the bf16 split of the router weights; when omitted a
        buffer is allocated for this call. ``router_weight=None`` reuses the
        split ``scratch`` already holds from an earlier call with the same E, H.
        """
        self._router_fused(x, router_weight, bias, ids32, ids64, weights, logits, scratch, None)

    def _router_fused(self, x, router_weight, bias, ids32, ids64, weights, logits, scratch, ranked):
        _check(x.is_cuda and x.is_contiguous() and x.dim() == 2 and x.dtype == torch.bfloat16,
               "expected BF16 GPU x[T,H]")
        tokens, hidden = x.shape
        for name, t in (("bias", bias), ("ids32", ids32), ("weights", weights)):
            _check_gpu_tensor(t, x, name)
        if ids64 is not None:
            _check_gpu_tensor(ids64, x, "ids64")
        experts = bias.shape[0] if bias.dim() == 1 else -1
        if router_weight is None:
            _check(scratch is not None, "reusing the router split needs the scratch that holds it")
        else:
            _check_gpu_tensor(router_weight, x, "router_weight")
            _check(router_weight.dtype == torch.float32 and router_weight.shape == (experts, hidden),
                   "expected FP32 router_weight[E,H]")
        _check(bias.dtype == torch.float32 and bias.shape == (experts,), "expected FP32 bias[E]")
        topk = ids32.shape[1] if ids32.dim() == 2 else -1
        _check(ids32.shape == (tokens, topk) and ids32.dtype == torch.int32, "expected int32 ids[T,K]")
        _check(weights.shape == (tokens, topk) and weights.dtype == torch.float32,
               "expected FP32 weights[T,K]")
        if ids64 is not None:
            _check(ids64.shape == (tokens, topk) and ids64.dtype == torch.int64, "expected int64 ids[T,K]")
        if logits is not None:
            _check_gpu_tensor(logits, x, "logits")
            _check(logits.shape == (tokens, experts) and logits.dtype == torch.float32,
                   "expected FP32 logits[T,E]")
        need = self.router_scratch_bytes(experts, hidden)
        if scratch is None:
            scratch = torch.empty(max(need, 1), dtype=torch.uint8, device=x.device)
        _check_gpu_tensor(scratch, x, "scratch")
        args = (_ptr(x), _ptr(router_weight), _ptr(bias), _ptr(ids32), _ptr(ids64), _ptr(weights),
                _ptr(logits), _ptr(scratch), scratch.numel() * scratch.element_size(), tokens, hidden,
                experts, topk)
        if ranked is None:
            status = self.lib.moe_router_fused(*args, _stream(x.device))
        else:
            ranks, tile_counts = ranked
            status = self.lib.moe_router_fused_ranked(*args, _ptr(ranks), _ptr(tile_counts),
                                                      tile_counts.numel() * 4, _stream(x.device))
        self.lib.check(status, "router_fused_out")

    def router_rank_tile(self, tokens, experts):
        """Tokens per tile of a ranked route for (T, E), or 0 when the shape has none."""
        return int(self.lib.moe_router_rank_tile(tokens, experts))

    def router_fused_ranked_out(self, x, router_weight, bias, ids32, ids64, weights, ranks, tile_counts,
                                logits=None, scratch=None):
        """``router_fused_out`` that also writes the dispatch's in-tile ranks into
        ``ranks`` (int32 [T*K]) and per-tile expert counts into ``tile_counts``
        (int32, at least ceil(T / router_rank_tile(T, E)) * E), for
        ``CudaWorkspace.dispatch_ranked``."""
        tokens = x.shape[0] if x.dim() == 2 else -1
        topk = ids32.shape[1] if ids32.dim() == 2 else -1
        for name, t, n in (("ranks", ranks, tokens * topk), ("tile_counts", tile_counts, None)):
            _check_gpu_tensor(t, x, name)
            _check(t.dtype == torch.int32 and t.is_contiguous() and (n is None or t.numel() == n),
                   f"expected contiguous int32 {name}" + (f"[{n}]" if n is not None else ""))
        self._router_fused(x, router_weight, bias, ids32, ids64, weights, logits, scratch, (ranks, tile_counts))

    def router_split_out(self, router_weight, scratch):
        """Write the bf16 split of ``router_weight`` [E,H] fp32 into ``scratch`` alone (no routing)."""
        _check(router_weight.is_cuda and router_weight.is_contiguous() and router_weight.dim() == 2
               and router_weight.dtype == torch.float32, "expected contiguous FP32 GPU router_weight[E,H]")
        _check_gpu_tensor(scratch, router_weight, "scratch")
        experts, hidden = router_weight.shape
        status = self.lib.moe_router_split(_ptr(router_weight), _ptr(scratch), scratch.numel() * scratch.element_size(),
                                           experts, hidden, _stream(router_weight.device))
        self.lib.check(status, "router_split_out")

    # -- transport -----------------------------------------------------------
    def scratch_bytes(self, tokens, experts, topk):
        return int(self.lib.moe_dispatch_scratch_bytes(tokens, experts, topk))

    def _dispatch(self, x, ids, counts, offsets, slots, packed, inverse, vectorized, alignment,
                  scratch, name):
        _check(x.is_cuda and x.is_contiguous(), "x must be contiguous GPU")
        _check(x.dim() == 2 and ids.dim() == 2, "expected x[T,H], ids[T,K]")
        _check(x.dtype in _DTYPES, "only FP32, FP16, and BF16 are supported")
        _check(ids.dtype == torch.int32, "ids must be int32")
        tokens, hidden = x.shape
        topk = ids.shape[1]
        experts = counts.numel()
        _check(ids.shape[0] == tokens and hidden > 0, "incompatible token dimensions")
        _check(1 <= topk <= 8, "topk must be in 1..8")
        _check(1 <= experts <= 64, "supports 1..64 experts")
        for t_name, t in (("ids", ids), ("counts", counts), ("offsets", offsets), ("slots", slots),
                          ("packed", packed), ("inverse", inverse)):
            _check_gpu_tensor(t, x, t_name)
        _check(all(t.dtype == torch.int32 for t in (counts, offsets, slots, inverse)),
               "workspace indices must be int32")
        n = tokens * topk
        _check(offsets.numel() == experts + 1 and slots.numel() == n and inverse.numel() == n,
               "incorrect index workspace size")
        _check(packed.dim() == 2 and packed.shape[1] == hidden and packed.dtype == x.dtype,
               "incorrect packed workspace")
        need = self.scratch_bytes(tokens, experts, topk)
        if scratch is None:
            scratch = torch.empty(max(need, 4), dtype=torch.uint8, device=x.device)
        _check_gpu_tensor(scratch, x, "scratch")
        status = self.lib.moe_dispatch(
            _ptr(x), _DTYPES[x.dtype], _ptr(ids), _ptr(counts), _ptr(offsets), _ptr(slots),
            _ptr(packed), _ptr(inverse), _ptr(scratch), scratch.numel() * scratch.element_size(),
            tokens, hidden, experts, topk, alignment, packed.shape[0], int(bool(vectorized)),
            _stream(x.device))
        self.lib.check(status, name)

    def dispatch_out(self, x, ids, counts, offsets, slots, packed, inverse, vectorized,
                     scratch=None):
        """Compact dispatch (reference ``csrc/dispatch.cu:102-158``)."""
        self._dispatch(x, ids, counts, offsets, slots, packed, inverse, vectorized, 1, scratch,
                       "dispatch_out")

    def dispatch_aligned_out(self, x, ids, counts, offsets, slots, packed, inverse, vectorized,
                             alignment, scratch=None):
        """Aligned dispatch with zeroed padding (reference ``csrc/dispatch.cu:218-275``)."""
        _check(1 <= alignment <= 128, "alignment must be 1..128")
        self._dispatch(x, ids, counts, offsets, slots, packed, inverse, vectorized, alignment,
                       scratch, "dispatch_aligned_out")

    def combine_out(self, packed_output, inverse, weights, output):
        """Weighted gather-reduce (reference ``csrc/dispatch.cu:160-192``)."""
        _check(packed_output.is_cuda and packed_output.is_contiguous(),
               "expert output must be contiguous GPU")
        _check(output.dim() == 2 and inverse.dim() == 2 and weights.dim() == 2,
               "expected output[T,H], inverse[T,K], weights[T,K]")
        _check(packed_output.dim() == 2 and packed_output.dtype in _DTYPES, "unsupported output dtype")
        for name, t in (("inverse", inverse), ("weights", weights), ("output", output)):
            _check_gpu_tensor(t, packed_output, name)
        _check(inverse.dtype == torch.int32 and weights.dtype == torch.float32,
               "inverse must be int32; weights must be FP32")
        tokens, hidden = output.shape
        topk = inverse.shape[1]
        _check(1 <= topk <= 8, "topk must be in 1..8")
        _check(hidden > 0, "invalid output shape")
        _check(inverse.shape[0] == tokens and weights.shape == inverse.shape
               and packed_output.shape[0] >= tokens * topk and packed_output.shape[1] == hidden
               and output.dtype == packed_output.dtype, "shape/dtype mismatch")
        status = self.lib.moe_combine(
            _ptr(packed_output), _DTYPES[packed_output.dtype], _ptr(inverse), _ptr(weights),
            _ptr(output), tokens, hidden, topk, packed_output.shape[0],
            _stream(packed_output.device))
        self.lib.check(status, "combine_out")

    # -- expert compute ------------------------------------------------------
    def swiglu_out(self, projection, valid_rows, output):
        """Standalone SwiGLU (reference ``csrc/dispatch.cu:294-323``)."""
        _check(projection.is_cuda and projection.is_contiguous(), "projection must be contiguous GPU")
        _check(projection.dim() == 2 and output.dim() == 2
               and projection.shape[0] == output.shape[0]
               and projection.shape[1] == output.shape[1] * 2,
               "expected projection[R,2I], output[R,I]")
        _check_gpu_tensor(valid_rows, projection, "valid_rows")
        _check_gpu_tensor(output, projection, "output")
        _check(valid_rows.dtype == torch.int32 and valid_rows.numel() == 1,
               "valid_rows must be a single int32 GPU value")
        _check(output.dtype == projection.dtype and projection.dtype in _DTYPES, "unsupported dtype")
        status = self.lib.moe_swiglu(
            _ptr(projection), _DTYPES[projection.dtype], _ptr(valid_rows), _ptr(output),
            output.shape[0], output.shape[1], _stream(projection.device))
        self.lib.check(status, "swiglu_out")

    def grouped_gemm_out(self, x, weight, offsets, output):
        """``output[r] = x[r] @ weight[e]^T`` for rows of expert e (bf16, fp32 accumulate)."""
        stride = self._check_gemm(x, weight, offsets, output, weight.shape[1])
        status = self.lib.moe_grouped_gemm_strided(
            _ptr(x), _ptr(weight), stride, _ptr(output), _ptr(offsets), x.shape[0], weight.shape[1],
            x.shape[1], weight.shape[0], _stream(x.device))
        self.lib.check(status, "grouped_gemm_out")

    def gateup_swiglu_out(self, x, gate_up, offsets, output):
        """Gate/up grouped GEMM with the SwiGLU epilogue fused; output is ``[R, I]``."""
        _check(gate_up.dim() == 3 and gate_up.shape[1] % 2 == 0, "expected gate_up[E,2I,H]")
        stride = self._check_gemm(x, gate_up, offsets, output, gate_up.shape[1] // 2)
        status = self.lib.moe_grouped_gateup_swiglu_strided(
            _ptr(x), _ptr(gate_up), stride, _ptr(output), _ptr(offsets), x.shape[0], x.shape[1],
            gate_up.shape[1] // 2, gate_up.shape[0], _stream(x.device))
        self.lib.check(status, "gateup_swiglu_out")

    def gateup_swiglu_gathered_out(self, x, row_src, gate_up, offsets, output):
        """gateup_swiglu_out with row r of A read from row ``row_src[r]`` of x
        (zero when negative); output is ``[len(row_src), I]``."""
        _check(gate_up.dim() == 3 and gate_up.shape[1] % 2 == 0, "expected gate_up[E,2I,H]")
        _check(x.is_cuda and x.is_contiguous() and x.dim() == 2 and x.dtype == torch.bfloat16,
               "expected contiguous BF16 GPU x[T,H]")
        _check_gpu_tensor(row_src, x, "row_src")
        _check(row_src.dtype == torch.int32 and row_src.dim() == 1, "expected int32 row_src[R]")
        rows = row_src.numel()
        _check(x.shape[1] % 64 == 0, "gathered gate/up needs hidden a multiple of 64")
        stride = _check_weight(gate_up, x, "gate_up")
        for name, t in (("offsets", offsets), ("output", output)):
            _check_gpu_tensor(t, x, name)
        _check(gate_up.dtype == torch.bfloat16 and gate_up.shape[2] == x.shape[1], "expected BF16 gate_up matching x")
        _check(offsets.dtype == torch.int32 and offsets.numel() == gate_up.shape[0] + 1, "expected int32 offsets[E+1]")
        _check(output.shape == (rows, gate_up.shape[1] // 2) and output.dtype == torch.bfloat16,
               "incorrect grouped-GEMM output buffer")
        status = self.lib.moe_grouped_gateup_swiglu_gathered_strided(
            _ptr(x), _ptr(row_src), x.shape[0], _ptr(gate_up), stride, _ptr(output), _ptr(offsets), rows, x.shape[1],
            gate_up.shape[1] // 2, gate_up.shape[0], _stream(x.device))
        self.lib.check(status, "gateup_swiglu_gathered_out")

    def set_gemm_workgroups(self, workgroups):
        """Bound the persistent grouped GEMM's workgroups (0: one per CU); results do not change."""
        _check(isinstance(workgroups, int) and workgroups >= 0, "workgroups must be a non-negative int")
        self.lib.check(self.lib.moe_set_gemm_workgroups(workgroups), "set_gemm_workgroups")

    @staticmethod
    def _check_gemm(x, weight, offsets, output, out_cols):
        _check(x.is_cuda and x.is_contiguous() and x.dim() == 2 and x.dtype == torch.bfloat16,
               "expected contiguous BF16 GPU x[R,K]")
        _check(isinstance(weight, torch.Tensor) and weight.dim() == 3, "expected BF16 weight[E,N,K] matching x")
        stride = _check_weight(weight, x, "weight")
        for name, t in (("offsets", offsets), ("output", output)):
            _check_gpu_tensor(t, x, name)
        _check(weight.dtype == torch.bfloat16 and weight.shape[2] == x.shape[1],
               "expected BF16 weight[E,N,K] matching x")
        _check(offsets.dtype == torch.int32 and offsets.numel() == weight.shape[0] + 1,
               "expected int32 offsets[E+1]")
        _check(output.shape == (x.shape[0], out_cols) and output.dtype == torch.bfloat16,
               "incorrect grouped-GEMM output buffer")
        _check(x.shape[1] % 8 == 0 and out_cols % 8 == 0, "grouped GEMM dimensions must be multiples of 8")
        return stride


@lru_cache(maxsize=1)
def get_extension():
    """The HIP operator set (reference ``_extension.py:30-63``), loaded once.

    Raises ``RuntimeError`` without a GPU or when ``libmoe_hip.so`` is missing:
    there is no eager or CPU fallback.
    """
    if not torch.cuda.is_available():
        raise RuntimeError("HIP operators require an AMD GPU (MI355X / gfx950). Use the torch "
                           "implementation on CPU.")
    return HipExtension()


def source_hashes():
    """sha256 of every kernel source, the ABI header and the package modules
    (reference ``_extension.py:18-27``); see ``moe_dispatch.evidence.source_files``."""
    from .evidence import source_hashes as hashes

    return hashes()
