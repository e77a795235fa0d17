"""Shared helpers for the parity tests: tensor conversion and oracle comparisons."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import moe_oracle as oracle

gpu = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="AMD GPU required"),
]

NP_DTYPE = {torch.float32: "f32", torch.float16: "f16", torch.bfloat16: "bf16"}


def to_np(t: torch.Tensor) -> np.ndarray:
    """Exact host copy; floating tensors widen to float32 (bf16/f16 values are exact)."""
    t = t.detach().cpu()
    if t.is_floating_point():
        return t.float().numpy()
    return t.numpy()


def raw_bits(t: torch.Tensor) -> np.ndarray:
    """Host copy of the raw bit patterns (for bit-exact comparisons of any dtype)."""
    t = t.detach().cpu().contiguous()
    if t.element_size() == 2:
        return t.view(torch.int16).numpy()
    if t.element_size() == 4:
        return t.view(torch.int32).numpy()
    return t.view(torch.int64).numpy()


def rel_l2(got: np.ndarray, ref: np.ndarray) -> float:
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30))


class LazyExpertWeights:
    """Index by expert to get one expert's weights as float32 numpy (host memory on demand)."""

    def __init__(self, tensor: torch.Tensor):
        self.tensor = tensor
        self.shape = tuple(tensor.shape)
        self._cache = {}

    def __getitem__(self, e):
        if e not in self._cache:
            self._cache[e] = self.tensor[e].float().cpu().numpy()
        return self._cache[e]


def route_margin(logits_ref: np.ndarray, bias: np.ndarray, topk: int) -> np.ndarray:
    """Gap between the K-th and (K+1)-th biased logit of each token (inf when K == E)."""
    v = np.sort(logits_ref.astype(np.float64) + bias.astype(np.float64), axis=1)[:, ::-1]
    if topk >= v.shape[1]:
        return np.full(v.shape[0], np.inf)
    return v[:, topk - 1] - v[:, topk]


def assert_layout_equal(ws, layout, tokens, topk, experts):
    """Bit-exact comparison of counts, offsets, slots and inverse with the oracle layout."""
    np.testing.assert_array_equal(to_np(ws.counts), layout["counts"])
    np.testing.assert_array_equal(to_np(ws.offsets), layout["offsets"])
    np.testing.assert_array_equal(to_np(ws.inverse).reshape(tokens, topk), layout["inverse"])
    np.testing.assert_array_equal(to_np(ws.slots).reshape(-1), layout["slots"])


def assert_packed_equal(packed: torch.Tensor, x: torch.Tensor, layout, topk):
    """Packed rows inside used spans equal the oracle's bit for bit (padding exactly zero)."""
    rows = packed.shape[0]
    expected, defined = oracle.pack(raw_bits(x), layout, topk, rows)
    used = int(layout["offsets"][-1])
    got = raw_bits(packed)[:used]
    np.testing.assert_array_equal(got, expected[:used])


def bf16_step(values: np.ndarray) -> np.ndarray:
    """Spacing of bf16 values at the magnitude of ``values`` (2^(e-7) for |v| in [2^e, 2^(e+1)))."""
    mag = np.abs(np.asarray(values, np.float64))
    _, e = np.frexp(np.where(mag > 0, mag, 2.0**-126))
    return np.ldexp(1.0, e - 8)


def assert_near_bit_exact(got, ref, max_fraction=1e-4, max_steps=1.0):
    """GEMM-derived bf16 outputs against the MFMA-order oracle, given identical inputs.

    The oracle models each bf16 MFMA (v_mfma_f32_16x16x32_bf16 and
    v_mfma_f32_32x32x16_bf16 alike) as: add the exact sum of each ascending
    group of 8 products to the fp32 accumulator with one round-to-nearest-even.
    The hardware adds the 8 products with a limited-width internal alignment,
    so on random data about 0.2-0.3% of single MFMA fp32 results differ from
    the model by one fp32 ulp. After rounding to
    bf16 that leaves about 1e-5 of the outputs one bf16 step away. Requires
    at most ``max_fraction`` of the elements (but always allows one: a single
    flip in a few thousand outputs is within that rate) to differ, each by at most
    ``max_steps`` bf16 steps of its value or 2^-10 of the tensor's RMS (a
    result near zero after cancellation sees the accumulator's ulp at the
    scale of its partial sums).
    """
    got = np.asarray(got, np.float32)
    ref = np.asarray(ref, np.float32)
    assert got.shape == ref.shape
    differ = got != ref
    if not differ.any():
        return
    fraction = differ.mean()
    assert int(differ.sum()) <= max(max_fraction * got.size, 1), (
        f"{int(differ.sum())} of {got.size} elements differ ({fraction:.2e})")
    step = bf16_step(np.maximum(np.abs(got[differ]), np.abs(ref[differ])))
    rms = float(np.sqrt(np.mean(np.square(ref.astype(np.float64)))))
    bound = np.maximum(max_steps * step, 2.0**-10 * rms)
    excess = np.abs(got[differ].astype(np.float64) - ref[differ]) / bound
    assert float(excess.max()) <= 1.0 + 1e-9, f"difference {float(excess.max()):.2f}x the bound"
