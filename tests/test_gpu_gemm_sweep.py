"""Randomised grouped-GEMM sweep: expert counts, shapes and persistent grid
sizes drawn from fixed seeds, so that combinations the hand-picked cases miss
(split plans at N < 256, 33 or 64 experts, one or three k stages, weight-
streaming and persistent launches side by side) are checked against the same
bars as test_gpu_gemm.py:

* the plain GEMM against the oracle's MFMA-order GEMM (near bit-exact), rows
  past offsets[E] untouched;
* the fused gate/up + SwiGLU GEMM against the kernels' own unfused pipeline
  (plain GEMM, bf16 projection, standalone SwiGLU), the projection against the
  oracle;
* the gathered gate/up GEMM (rows read from x through a row table with -1
  entries) bit-exact against the packed one on the gathered rows;
* every one of them again on the same weights stored with padded rows (a
  [:, :, :K] view of storage with 8-1024 NaN elements after each row, read
  through the row-stride entry points): bit-exact against contiguous weights.

This sweep found the column pieces past the last output column
(test_gpu_gemm.py::test_column_pieces_past_the_last_column).
"""

import numpy as np
import pytest
import torch

from oracle import moe_oracle as oracle
from tests._helpers import assert_near_bit_exact, gpu, to_np

pytestmark = gpu

CASES_PER_SEED = 40


def _counts(rng, experts):
    kind = rng.integers(0, 4)
    if kind == 0:
        counts = rng.integers(0, 600, experts)
    elif kind == 1:  # skewed: a few large experts, many small ones
        counts = (rng.pareto(1.2, experts) * 100).astype(int)
    elif kind == 2:  # within a few rows of multiples of 256
        counts = rng.integers(1, 12, experts) * 256 + rng.integers(-3, 4, experts)
    else:  # a few rows each
        counts = rng.integers(0, 40, experts)
    return np.clip(counts, 0, 3000)


def _cases(seed):
    rng = np.random.default_rng(seed)
    for case in range(CASES_PER_SEED):
        experts = int(rng.choice([1, 2, 3, 8, 16, 33, 64]))
        counts = _counts(rng, experts)
        k = int(rng.choice([64, 128, 192, 256, 512, 1024, 2048, 96, 200]))
        n = int(rng.choice([64, 136, 256, 384, 512, 1024]))
        while int(counts.sum()) * n * k > 1.5e9:  # keeps the CPU oracle to about a second
            counts = counts // 2
        alignment = int(rng.choice([1, 8, 16]))
        spans = (counts + alignment - 1) // alignment * alignment
        offsets = np.concatenate([[0], np.cumsum(spans)]).astype(np.int32)
        rows = int(offsets[-1]) + int(rng.integers(0, 9))
        if rows == 0:
            continue
        grid = int(rng.choice([0, 0, 8, 24, 64]))
        swiglu = bool(rng.integers(0, 2)) and k % 64 == 0
        yield case, experts, offsets, rows, k, n, grid, swiglu


def _row_padded(w, case):
    """w as a [:, :, :K] view of storage with NaN padding after each row (8 to 1024
    elements, a multiple of 8, by case)."""
    pad = (8, 64, 136, 1024)[case % 4]
    e, n, k = w.shape
    storage = torch.full((e, n, k + pad), float("nan"), device=w.device, dtype=w.dtype)
    storage[:, :, :k] = w
    return storage[:, :, :k]


def _plain(ext, g, experts, offsets, rows, k, n, case):
    a = torch.randn(rows, k, device="cuda", generator=g).bfloat16()
    w = (torch.randn(experts, n, k, device="cuda", generator=g) / k**0.5).bfloat16()
    c = torch.full((rows, n), 7.0, device="cuda").bfloat16()
    ext.grouped_gemm_out(a, w, torch.tensor(offsets, device="cuda"), c)
    torch.cuda.synchronize()
    used = int(offsets[-1])
    got = to_np(c)
    ref = oracle.bf16_round(oracle.grouped_gemm(to_np(a), to_np(w), offsets, order="mfma"))
    assert_near_bit_exact(got[:used], ref[:used])
    assert np.all(got[used:] == 7.0), "rows past offsets[E] must not be written"
    padded = torch.full((rows, n), 7.0, device="cuda").bfloat16()
    ext.grouped_gemm_out(a, _row_padded(w, case), torch.tensor(offsets, device="cuda"), padded)
    assert torch.equal(padded, c), "row-padded weights differ from contiguous ones"


def _gateup(ext, g, experts, offsets, rows, k, n, case):
    inter = max(n // 2 // 8 * 8, 8)
    off = torch.tensor(offsets, device="cuda")
    used = int(offsets[-1])
    a = torch.randn(rows, k, device="cuda", generator=g).bfloat16()
    w = (torch.randn(experts, 2 * inter, k, device="cuda", generator=g) / k**0.5).bfloat16()
    act = torch.full((rows, inter), 3.0, device="cuda").bfloat16()
    ext.gateup_swiglu_out(a, w, off, act)
    projection = torch.empty(rows, 2 * inter, device="cuda", dtype=torch.bfloat16)
    ext.grouped_gemm_out(a, w, off, projection)
    unfused = torch.empty_like(act)
    ext.swiglu_out(projection, off[-1:], unfused)
    torch.cuda.synchronize()
    got = to_np(act)
    assert_near_bit_exact(got[:used], to_np(unfused)[:used], max_fraction=1e-4, max_steps=1.0)
    assert np.all(got[used:] == 3.0), "rows past offsets[E] must not be written"
    ref = oracle.bf16_round(oracle.grouped_gemm(to_np(a), to_np(w), offsets, order="mfma"))
    assert_near_bit_exact(to_np(projection)[:used], ref[:used])
    # Gathered rows: row r of the product is row src[r] of x (zeros for -1).
    tokens = max(1, rows // 2)
    x = torch.randn(tokens, k, device="cuda", generator=g).bfloat16()
    src = torch.randint(-1, tokens, (rows,), device="cuda", generator=g, dtype=torch.int32)
    packed = torch.where(src[:, None] >= 0, x[src.clamp_min(0).long()], torch.zeros_like(x[:1])).contiguous()
    act_g = torch.full((rows, inter), 3.0, device="cuda").bfloat16()
    ext.gateup_swiglu_gathered_out(x, src, w, off, act_g)
    act_p = torch.full((rows, inter), 3.0, device="cuda").bfloat16()
    ext.gateup_swiglu_out(packed, w, off, act_p)
    torch.cuda.synchronize()
    assert torch.equal(act_g, act_p), "the gathered GEMM differs from the packed one on the same rows"
    w_padded = _row_padded(w, case)
    act_padded = torch.full((rows, inter), 3.0, device="cuda").bfloat16()
    ext.gateup_swiglu_out(a, w_padded, off, act_padded)
    assert torch.equal(act_padded, act), "row-padded weights differ from contiguous ones"
    act_padded.fill_(3.0)
    ext.gateup_swiglu_gathered_out(x, src, w_padded, off, act_padded)
    assert torch.equal(act_padded, act_g), "row-padded weights differ from contiguous ones (gathered)"


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_random_grouped_gemms(ext, seed):
    for case, experts, offsets, rows, k, n, grid, swiglu in _cases(seed):
        print(f"seed {seed} case {case}: E={experts} rows={rows} k={k} n={n} grid={grid} swiglu={swiglu}",
              flush=True)
        g = torch.Generator(device="cuda").manual_seed(1000 * seed + case)
        try:
            ext.set_gemm_workgroups(grid)
            if swiglu:
                _gateup(ext, g, experts, offsets, rows, k, n, case)
            else:
                _plain(ext, g, experts, offsets, rows, k, n, case)
        finally:
            ext.set_gemm_workgroups(0)
