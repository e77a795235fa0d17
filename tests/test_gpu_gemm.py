"""Grouped GEMM parity.

Against the oracle's MFMA-order GEMM (ascending k, groups of 8 products, one
fp32 rounding per group): at least 99.99% of the bf16 outputs identical and the
rest one bf16 step away (see tests/_helpers.assert_near_bit_exact); and,
independently, within one bf16 rounding of the exact float64 product. Covers empty experts,
skewed row counts, partial row tiles, short reductions (K < 64), column counts
that are not multiples of the column tile, decode-sized launches (at most 128
rows, which take 32- and 64-column tiles), and the fused gate/up + SwiGLU
epilogue against the kernels' own unfused pipeline (grouped GEMM -> bf16
projection -> standalone SwiGLU). The two see the same bf16 gate and up values;
the fused epilogue evaluates silu with the hardware exp2 and reciprocal
(v_exp_f32, v_rcp_f32, about 1 ulp each) while the standalone kernel uses the
correctly ordered fp32 sequence the oracle reproduces, so after the bf16
rounding they may differ by one bf16 step in a few elements per 100 000.
"""

import numpy as np
import pytest
import torch

from oracle import moe_oracle as oracle
from tests._helpers import assert_near_bit_exact, gpu, rel_l2, to_np

pytestmark = gpu


def _offsets(counts, alignment):
    spans = [(c + alignment - 1) // alignment * alignment for c in counts]
    return np.concatenate([[0], np.cumsum(spans)]).astype(np.int32)


def _inputs(counts, alignment, k, seed):
    offsets = _offsets(counts, alignment)
    rows = int(offsets[-1]) + 5  # spare rows past offsets[E] must stay untouched
    g = torch.Generator(device="cuda").manual_seed(seed)
    a = torch.randn(rows, k, device="cuda", generator=g).bfloat16()
    return a, torch.tensor(offsets, device="cuda"), rows


GEMM_CASES = [
    # counts per expert, alignment, n, k
    ([5, 0, 37, 300, 8, 0, 1, 64], 8, 256, 64),
    ([0, 0, 0, 1], 8, 512, 128),
    ([700, 3, 0, 260], 8, 384, 32),
    ([1024, 1030, 998, 1051], 8, 264, 200),
    ([33] * 16, 1, 128, 1024),
    ([2000, 0], 8, 1024, 512),
    # at most 128 rows in all: the 32-column decode tiles (K % 64 == 0; K=96 takes the generic path)
    ([90, 20, 0], 8, 200, 96),
    ([1, 0, 1], 1, 1000, 64),
    ([90, 20, 0], 8, 200, 128),
    ([7, 0, 40], 1, 96, 192),
    ([2, 2], 1, 4096, 1024),
    # generic path (K % 64 != 0) with one or two column tiles: 9 row tiles of one
    # expert need every one of the 8 * ceil(9 / 8) workgroup slots
    ([2304], 8, 256, 200),
    ([1500, 100, 3, 0], 8, 256, 1000),
]


@pytest.mark.parametrize("counts,alignment,n,k", GEMM_CASES)
def test_grouped_gemm_matches_float64(ext, counts, alignment, n, k):
    experts = len(counts)
    a, offsets, rows = _inputs(counts, alignment, k, seed=n + k)
    g = torch.Generator(device="cuda").manual_seed(3 * n + k)
    b = (torch.randn(experts, n, k, device="cuda", generator=g) / k**0.5).bfloat16()
    c = torch.full((rows, n), 7.0, device="cuda").bfloat16()
    ext.grouped_gemm_out(a, b, offsets, c)
    exact = oracle.grouped_gemm(to_np(a), to_np(b), to_np(offsets), order="exact")
    mfma = oracle.grouped_gemm(to_np(a), to_np(b), to_np(offsets), order="mfma")
    used = int(to_np(offsets)[-1])
    got = to_np(c)
    assert_near_bit_exact(got[:used], oracle.bf16_round(mfma)[:used])
    ref = exact[:used]
    # bf16 output: at most one rounding of the fp32 accumulator away from the exact value.
    assert np.all(np.abs(got[:used] - ref) <= 2.0**-8 * np.abs(ref) + 1e-4), "beyond one bf16 rounding"
    assert rel_l2(got[:used], oracle.bf16_round(ref)) < 2e-3
    assert np.all(got[used:] == 7.0), "rows past offsets[E] must not be written"


SCHEDULE_CASES = [
    # counts, alignment, output columns (N, or I for gate/up), k, gate/up?, workgroup bounds.
    # With 8-40 workgroups these small launches take every path of the persistent plan:
    # slots carrying two short tiles, an extra round, leftovers after the rounds, split
    # halves and quarters, a partial last round, phase 1 as halves in the rounds
    # (tests/test_ring_plan.py checks which case reaches which).
    ([300, 700, 3, 260, 40, 1, 129, 520], 8, 512, 128, False, (8, 24)),
    ([300, 700, 3, 260, 40, 1, 129, 520], 8, 512, 128, True, (8, 16, 40)),
    ([1030, 20, 5, 257, 64, 600, 0, 90], 8, 1024, 192, False, (8, 16, 40)),
    ([1030, 20, 5, 257, 64, 600, 0, 90], 8, 640, 64, True, (8, 16, 24)),
    ([512, 256], 8, 1024, 128, False, (8,)),
    # 32 full tiles in whole rounds, 4 short ones left over: 64-column quarters at
    # 16 workgroups, 128-column halves at 8
    ([1030, 1030, 2048], 8, 512, 128, False, (8, 16)),
    # 6 full tiles beside 4 short ones: halves in the rounds from 16 workgroups on
    ([300, 40, 512], 8, 512, 128, False, (8, 16, 40)),
    # gate/up at K = 2048: balanced row tiles of 160, 224, 192 and 256 rows
    # (experts of 304, 424, 520 and 704 rows), 1040 rows as five of 224, and a
    # phase-2 tile of 104 rows
    ([300, 420, 520, 700, 1034, 100], 8, 136, 2048, True, (8, 24, 64)),
    # experts of more than 8 row tiles (2600 and 4100 rows): their phase-1 tiles
    # run in groups of at most 8 row tiles
    ([2600, 300, 4100, 40], 8, 512, 128, False, (8, 24)),
    ([2600, 300, 4100, 40], 8, 384, 128, True, (8, 24)),
]


@pytest.mark.parametrize("counts,alignment,n,k,swiglu,grids", SCHEDULE_CASES)
def test_schedule_does_not_change_results(ext, counts, alignment, n, k, swiglu, grids):
    """Every tile is written, and by the same MFMA chain, whatever the persistent grid."""
    experts = len(counts)
    a, offsets, rows = _inputs(counts, alignment, k, seed=n + 3 * k)
    g = torch.Generator(device="cuda").manual_seed(5 * n + k)
    w = (torch.randn(experts, 2 * n if swiglu else n, k, device="cuda", generator=g) / k**0.5).bfloat16()
    run = ext.gateup_swiglu_out if swiglu else ext.grouped_gemm_out

    def once():
        out = torch.full((rows, n), 5.0, device="cuda").bfloat16()
        run(a, w, offsets, out)
        torch.cuda.synchronize()
        return out

    try:
        ext.set_gemm_workgroups(0)
        default = once()
        for grid in grids:
            ext.set_gemm_workgroups(grid)
            assert torch.equal(once(), default), f"{grid} workgroups changed the output"
    finally:
        ext.set_gemm_workgroups(0)
    off = to_np(offsets)
    used = int(off[-1])
    got = to_np(default)
    assert np.all(got[used:] == 5.0), "rows past offsets[E] must not be written"
    ref = np.zeros((used, n), dtype=np.float32)
    for e in range(experts):
        lo, hi = int(off[e]), int(off[e + 1])
        if hi > lo:
            proj = (a[lo:hi].float() @ w[e].float().t())
            if swiglu:
                g, u = proj[:, :n].bfloat16().float(), proj[:, n:].bfloat16().float()
                proj = torch.nn.functional.silu(g) * u
            ref[lo:hi] = to_np(proj)
    assert rel_l2(got[:used], ref) < 3e-3


# counts, alignment, n, grid: plans whose split tiles have 128- or 64-column pieces
# starting at or past the last output column (N < 256, or a last column tile of
# 64-192 columns); such a piece has no work and its weight rows would start past
# the expert's (a wrapped buffer range once read past the weights).
EDGE_PIECE_CASES = [
    ([169], 1, 64, 8),
    ([520, 20], 8, 192, 8),
    ([1000, 20, 300], 8, 320, 24),
    ([300, 420, 520, 700, 1034, 100], 8, 128, 24),
    ([300, 420, 520, 700, 1034, 100], 8, 64, 0),
]


@pytest.mark.parametrize("counts,alignment,n,grid", EDGE_PIECE_CASES)
def test_column_pieces_past_the_last_column(ext, counts, alignment, n, grid):
    experts, k = len(counts), 256
    a, offsets, rows = _inputs(counts, alignment, k, seed=n + grid)
    g = torch.Generator(device="cuda").manual_seed(7 * n + grid)
    b = (torch.randn(experts, n, k, device="cuda", generator=g) / k**0.5).bfloat16()
    c = torch.full((rows, n), 7.0, device="cuda").bfloat16()
    try:
        ext.set_gemm_workgroups(grid)
        ext.grouped_gemm_out(a, b, offsets, c)
        torch.cuda.synchronize()
    finally:
        ext.set_gemm_workgroups(0)
    used = int(to_np(offsets)[-1])
    got = to_np(c)
    mfma = oracle.grouped_gemm(to_np(a), to_np(b), to_np(offsets), order="mfma")
    assert_near_bit_exact(got[:used], oracle.bf16_round(mfma)[:used])
    assert np.all(got[used:] == 7.0), "rows past offsets[E] must not be written"


# rows of A, ascending offsets as given (past the rows, negative), the same clamped to [0, rows]
CLAMP_CASES = [
    (600, [0, 100, 2_000_000_000, 2_147_483_000], [0, 100, 600, 600]),
    (600, [-50, 300, 350, 900], [0, 300, 350, 600]),
    (100, [0, 40, 1_000_000, 1_000_000], [0, 40, 100, 100]),  # at most 128 rows: the weight-streaming kernel
]


@pytest.mark.parametrize("swiglu", [False, True])
@pytest.mark.parametrize("rows,given,clamped", CLAMP_CASES)
def test_offsets_outside_the_rows_act_as_clamped(ext, rows, given, clamped, swiglu):
    """Offsets read from device memory are clamped to [0, rows] before they size
    the tile walk: offsets past the rows (counts that disagree with the buffer)
    give the output of the clamped offsets, promptly, and no row past them is
    written."""
    n, k = 256, 256
    g = torch.Generator(device="cuda").manual_seed(rows + 7)
    a = torch.randn(rows, k, device="cuda", generator=g).bfloat16()
    w = (torch.randn(3, 2 * n if swiglu else n, k, device="cuda", generator=g) / k**0.5).bfloat16()
    run = ext.gateup_swiglu_out if swiglu else ext.grouped_gemm_out
    outs = []
    for off in (given, clamped):
        out = torch.full((rows, n), 5.0, device="cuda").bfloat16()
        run(a, w, torch.tensor(off, device="cuda", dtype=torch.int32), out)
        torch.cuda.synchronize()
        outs.append(out)
    assert torch.equal(outs[0], outs[1])


GATEUP_CASES = [
    # counts, alignment, hidden, intermediate
    ([5, 0, 37, 300, 8, 0, 1, 64], 8, 64, 128),
    ([0, 1], 8, 256, 256),
    ([700, 3, 0, 260], 8, 32, 384),
    ([129, 255, 256, 257], 8, 512, 136),
    ([2000, 17], 8, 1024, 1408),
    # K = 2048: balanced row tiles (160 to 256 rows; five of 224 rows for 1040)
    ([300, 420, 100, 1034, 520, 700, 0], 8, 2048, 136),
    # at most 128 rows in all: the 64-column decode tiles
    ([70, 9], 8, 96, 200),
    ([2, 0, 0, 1], 1, 512, 64),
]


@pytest.mark.parametrize("counts,alignment,hidden,inter", GATEUP_CASES)
def test_gateup_swiglu_matches_unfused_pipeline(ext, counts, alignment, hidden, inter):
    experts = len(counts)
    a, offsets, rows = _inputs(counts, alignment, hidden, seed=hidden + inter)
    g = torch.Generator(device="cuda").manual_seed(3 * hidden + inter)
    w = (torch.randn(experts, 2 * inter, hidden, device="cuda", generator=g) / hidden**0.5).bfloat16()
    act = torch.full((rows, inter), 3.0, device="cuda").bfloat16()
    ext.gateup_swiglu_out(a, w, offsets, act)
    used = int(to_np(offsets)[-1])
    proj = oracle.bf16_round(oracle.grouped_gemm(to_np(a), to_np(w), to_np(offsets), order="mfma"))
    ref = oracle.swiglu(proj, used)[:used]
    got = to_np(act)
    # A one-step flip of g or u moves silu(g)*u by up to ~2 bf16 steps.
    assert_near_bit_exact(got[:used], ref, max_fraction=2e-4, max_steps=2.0)
    exact = oracle.swiglu(oracle.bf16_round(oracle.grouped_gemm(to_np(a), to_np(w), to_np(offsets), order="exact")), used)
    assert rel_l2(got[:used], exact[:used]) < 3e-3
    assert np.all(got[used:] == 3.0), "rows past offsets[E] must not be written"
    # The same kernels unfused (plain GEMM -> standalone SwiGLU): identical up to the
    # rounding of silu's exp/reciprocal (one bf16 step, rarely).
    projection = torch.empty(rows, 2 * inter, device="cuda", dtype=torch.bfloat16)
    ext.grouped_gemm_out(a, w, offsets, projection)
    unfused = torch.empty_like(act)
    ext.swiglu_out(projection, offsets[-1:], unfused)
    assert_near_bit_exact(got[:used], to_np(unfused)[:used], max_fraction=1e-4, max_steps=1.0)


STRIDED_CASES = [
    # counts per expert, alignment, n (intermediate for gate/up), k (hidden), padding per row
    ([2, 2], 1, 1024, 4096, 64),                 # weight-streaming kernel, 64-row instance
    ([60, 40, 20], 8, 512, 2048, 64),            # weight-streaming kernel, 128-row instance
    ([700, 3, 0, 260, 1100], 8, 384, 1024, 64),  # persistent kernel: full, short and split tiles
    ([300, 420, 520, 700, 1034, 100], 8, 128, 512, 8),
    ([1500, 100, 3, 0], 8, 256, 200, 8),         # generic kernel (K % 64 != 0)
]


def _row_padded(w, pad):
    """w as a [:, :, :K] view of storage with `pad` NaN elements after each row."""
    e, n, k = w.shape
    storage = torch.full((e, n, k + pad), float("nan"), device=w.device, dtype=w.dtype)
    storage[:, :, :k] = w
    view = storage[:, :, :k]
    assert not view.is_contiguous() and view.stride(1) == k + pad
    return view


@pytest.mark.parametrize("counts,alignment,n,k,pad", STRIDED_CASES)
def test_row_padded_weights_equal_contiguous(ext, counts, alignment, n, k, pad):
    """Weights read through a row stride (the _strided entry points, through the
    extension's view handling) give the contiguous weights' outputs bit for bit:
    the plain GEMM, the gate/up GEMM with the SwiGLU epilogue, and the gathered
    gate/up GEMM. The padding holds NaN, so a read of it would show."""
    experts = len(counts)
    a, offsets, rows = _inputs(counts, alignment, k, seed=k + n + pad)
    g = torch.Generator(device="cuda").manual_seed(7 * k + n)
    w = (torch.randn(experts, n, k, device="cuda", generator=g) / k**0.5).bfloat16()
    gu = (torch.randn(experts, 2 * n, k, device="cuda", generator=g) / k**0.5).bfloat16()
    used = int(to_np(offsets)[-1])
    plain = [torch.full((rows, n), 3.0, device="cuda").bfloat16() for _ in range(2)]
    ext.grouped_gemm_out(a, w, offsets, plain[0])
    ext.grouped_gemm_out(a, _row_padded(w, pad), offsets, plain[1])
    act = [torch.full((rows, n), 3.0, device="cuda").bfloat16() for _ in range(2)]
    ext.gateup_swiglu_out(a, gu, offsets, act[0])
    ext.gateup_swiglu_out(a, _row_padded(gu, pad), offsets, act[1])
    for got, ref in (plain[::-1], act[::-1]):
        assert torch.equal(got, ref)
        assert not torch.isnan(got[:used].float()).any()
    if k % 64 == 0:
        row_src = torch.arange(rows, device="cuda", dtype=torch.int32)
        gathered = [torch.full((rows, n), 3.0, device="cuda").bfloat16() for _ in range(2)]
        ext.gateup_swiglu_gathered_out(a, row_src, gu, offsets, gathered[0])
        ext.gateup_swiglu_gathered_out(a, row_src, _row_padded(gu, pad), offsets, gathered[1])
        assert torch.equal(gathered[0], gathered[1])
        assert torch.equal(gathered[0], act[0])


def test_weights_of_other_layouts_are_refused(ext):
    a, offsets, rows = _inputs([10, 20], 8, 64, seed=1)
    out = torch.empty(rows, 64, device="cuda", dtype=torch.bfloat16)
    w = torch.randn(2, 64, 64, device="cuda").bfloat16()
    with pytest.raises(RuntimeError, match="contiguous, or"):
        ext.grouped_gemm_out(a, w.transpose(1, 2), offsets, out)  # columns, not rows, contiguous
    with pytest.raises(RuntimeError, match="multiple of 8"):
        storage = torch.zeros(2, 64, 68, device="cuda").bfloat16()
        ext.grouped_gemm_out(a, storage[:, :, :64], offsets, out)  # rows not 16-byte aligned
