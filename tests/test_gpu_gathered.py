"""The dispatch without the row copy, and the gate/up GEMM that gathers from x.

``moe_dispatch_rows`` / ``moe_dispatch_ranked_rows`` write the dispatch layout
(counts, offsets, slots, inverse) and, instead of packed rows, the row table
``row_src``: each used packed row's token, -1 for padding rows, rows past
offsets[E] untouched. ``moe_grouped_gateup_swiglu_gathered`` reads A row r
from x[row_src[r]] (zeros for -1). Checked here, bit for bit:

* the layout equals moe_dispatch's (and the oracle's), with and without a
  ranked route, counted in the pack kernel (small batches) or by the counting
  kernel first;
* the table equals its definition from the oracle's inverse permutation;
* the gathered GEMM equals the packed GEMM on moe_dispatch's rows, on the
  persistent kernel (balanced row tiles at K >= 2048, plain below, chained
  tiles) and on the weight-streaming kernel (at most 128 rows), and at other
  persistent grid sizes (which change which tiles chain);
* a table entry out of x's range reads zeros instead of faulting;
* edge cases: no tokens, and most experts empty (skewed routing).
"""

import numpy as np
import pytest
import torch

from moe_dispatch.routing import make_case, make_transport_case
from moe_dispatch.workspace import CudaWorkspace
from oracle import moe_oracle as oracle
from tests._helpers import assert_layout_equal, gpu, to_np

pytestmark = gpu


def _expected_table(layout, topk):
    used = int(layout["offsets"][-1])
    table = np.full(used, -1, np.int64)
    inverse = layout["inverse"].reshape(-1)
    table[inverse] = np.arange(inverse.size) // topk
    return table


def _ranked(ext, ws, x, experts, topk, seed):
    """A ranked route of random weights for ws (its ranks and tile counts), and its ids."""
    tokens, hidden = x.shape
    g = torch.Generator(device="cuda").manual_seed(seed)
    w = torch.randn(experts, hidden, device="cuda", generator=g) / hidden**0.5
    bias = torch.zeros(experts, device="cuda")
    ids32 = torch.empty(tokens, topk, device="cuda", dtype=torch.int32)
    ids64 = torch.empty(tokens, topk, device="cuda", dtype=torch.int64)
    weights = torch.empty(tokens, topk, device="cuda")
    ext.router_fused_ranked_out(x, w, bias, ids32, ids64, weights, ws.tile_ranks, ws.tile_counts)
    return ids32


DISPATCH_CASES = [
    # tokens, hidden, experts, topk, alignment, ranked
    (0, 64, 8, 3, 8, False),       # no tokens: every row left as it was
    (1, 64, 8, 2, 8, False),       # one token, counted in the pack kernel
    (300, 128, 8, 2, 8, False),    # 600 assignments: counted in the pack kernel
    (4096, 64, 8, 2, 8, False),    # the counting kernel, then the pack kernel
    (1000, 128, 64, 6, 1, False),  # many experts, alignment 1
    (300, 256, 8, 2, 8, True),     # ranked route, 16-token tiles
    (777, 512, 32, 4, 16, True),   # ranked route, 32-token tiles, ragged last tile
]


@pytest.mark.parametrize("tokens,hidden,experts,topk,alignment,ranked", DISPATCH_CASES)
def test_row_table_dispatch_matches_the_packed_dispatch(ext, tokens, hidden, experts, topk, alignment, ranked):
    x, ids32, ids64, _ = make_transport_case(tokens, hidden, experts, topk, torch.bfloat16, seed=tokens)
    packed_ws = CudaWorkspace(tokens, hidden, experts, topk, torch.bfloat16, alignment=alignment, extension=ext)
    rows_ws = CudaWorkspace(tokens, hidden, experts, topk, torch.bfloat16, alignment=alignment, extension=ext)
    if ranked:
        ids32 = _ranked(ext, rows_ws, x, experts, topk, seed=tokens)
    packed_ws.dispatch(x, ids32)
    rows_ws.row_src.fill_(-7)
    rows_ws.packed.fill_(3.0)
    for _ in range(2):  # repeatable: the ranked form only reads the ranks
        if ranked:
            rows_ws.dispatch_ranked_rows(ids32)
        else:
            rows_ws.dispatch_rows(ids32)
        layout = oracle.dispatch_layout(to_np(ids32), experts, alignment)
        assert_layout_equal(rows_ws, layout, tokens, topk, experts)
        for name in ("counts", "offsets", "slots", "inverse"):
            assert torch.equal(getattr(rows_ws, name), getattr(packed_ws, name)), name
        used = int(layout["offsets"][-1])
        np.testing.assert_array_equal(to_np(rows_ws.row_src[:used]), _expected_table(layout, topk))
        assert bool((rows_ws.row_src[used:] == -7).all()), "rows past offsets[E] must not be written"
        assert bool((rows_ws.packed == 3.0).all()), "no rows are copied"


GEMM_CASES = [
    # tokens, hidden, intermediate, experts, topk, alignment[, skewed]
    (1500, 2048, 256, 8, 2, 8),    # persistent kernel, balanced row tiles (K = 2048)
    (900, 1024, 256, 16, 3, 8, True),  # skewed: experts 0-2 hold nearly every row, most others none
    (30, 2048, 128, 16, 4, 1, True),   # skewed (experts 0-3), weight-streaming kernel
    (1100, 1024, 384, 16, 2, 8),   # persistent kernel, plain row tiles (K = 1024), short tiles
    (2100, 4096, 136, 4, 2, 1),    # K = 4096, two column tiles (136 = 128 + 8), alignment 1
    (40, 512, 256, 8, 2, 8),       # at most 128 rows: the weight-streaming kernel
    (3, 2048, 192, 8, 2, 1),       # one-token-ish decode: 64-row weight-streaming tiles
    (600, 64, 128, 16, 3, 8),      # K = 64: one stage per tile
]


@pytest.mark.parametrize("case", GEMM_CASES)
def test_gathered_gateup_equals_the_packed_gateup(ext, case):
    tokens, hidden, inter, experts, topk, alignment = case[:6]
    if len(case) > 6:
        x, ids32, _, _ = make_case(tokens, hidden, experts, topk, torch.bfloat16, "skewed", seed=tokens)
    else:
        x, ids32, _, _ = make_transport_case(tokens, hidden, experts, topk, torch.bfloat16, seed=hidden + tokens)
    ws = CudaWorkspace(tokens, hidden, experts, topk, torch.bfloat16, alignment=alignment, extension=ext)
    ws.dispatch(x, ids32)
    ws.dispatch_rows(ids32)  # the same offsets; row_src for the gathered GEMM
    rows = ws.capacity_rows
    used = int(ws.offsets[-1])
    g = torch.Generator(device="cuda").manual_seed(inter)
    gate_up = (torch.randn(experts, 2 * inter, hidden, device="cuda", generator=g) / hidden**0.5).bfloat16()

    def run(gathered):
        out = torch.full((rows, inter), 5.0, device="cuda").bfloat16()
        if gathered:
            ext.gateup_swiglu_gathered_out(x, ws.row_src, gate_up, ws.offsets, out)
        else:
            ext.gateup_swiglu_out(ws.packed, gate_up, ws.offsets, out)
        torch.cuda.synchronize()
        return out

    try:
        for grid in (0, 8, 24):
            ext.set_gemm_workgroups(grid)
            packed, gathered = run(False), run(True)
            assert torch.equal(gathered[:used], packed[:used]), f"{grid} workgroups"
            assert bool((gathered[used:] == 5.0).all()), "rows past offsets[E] must not be written"
    finally:
        ext.set_gemm_workgroups(0)


def test_table_entries_out_of_range_read_zeros(ext):
    """A row index past x's rows (or negative) gathers zeros: that row's outputs
    are silu(0) * 0 = 0, and no access leaves x's buffer."""
    tokens, hidden, inter, experts = 64, 512, 128, 2
    g = torch.Generator(device="cuda").manual_seed(9)
    x = torch.randn(tokens, hidden, device="cuda", generator=g).bfloat16()
    gate_up = (torch.randn(experts, 2 * inter, hidden, device="cuda", generator=g) / hidden**0.5).bfloat16()
    offsets = torch.tensor([0, 96, 160], device="cuda", dtype=torch.int32)
    table = torch.arange(160, device="cuda", dtype=torch.int32) % tokens
    table[5] = tokens        # one past x
    table[70] = 1 << 30      # far past x
    table[100] = -1          # padding
    out = torch.full((160, inter), 5.0, device="cuda").bfloat16()
    ext.gateup_swiglu_gathered_out(x, table, gate_up, offsets, out)
    rows = x.index_select(0, table.clamp(0, tokens - 1).long())
    rows[5] = 0
    rows[70] = 0
    rows[100] = 0
    ref = torch.full_like(out, 5.0)
    ext.gateup_swiglu_out(rows.contiguous(), gate_up, offsets, ref)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    assert bool((out[[5, 70, 100]] == 0).all())


def test_gathered_gateup_rejects_hidden_not_a_multiple_of_64(ext):
    x = torch.zeros(8, 96, device="cuda", dtype=torch.bfloat16)
    table = torch.zeros(8, device="cuda", dtype=torch.int32)
    gate_up = torch.zeros(1, 16, 96, device="cuda", dtype=torch.bfloat16)
    offsets = torch.tensor([0, 8], device="cuda", dtype=torch.int32)
    out = torch.empty(8, 8, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(Exception, match="multiple of 64"):
        ext.gateup_swiglu_gathered_out(x, table, gate_up, offsets, out)


@pytest.mark.parametrize("cfg,tokens,gathers", [
    ((2048, 1408, 64, 6), 700, True),   # top-6: the row table
    ((256, 128, 16, 3), 300, True),     # top-3, hidden a multiple of 64
    ((512, 1024, 8, 2), 128, False),    # top-2 packs (the gathered GEMM's loads cost more than the copy)
    ((96, 256, 8, 4), 100, False),      # hidden not a multiple of 64: the generic GEMM cannot gather
])
def test_block_forward_gathers_from_top3_on_and_matches_the_packed_forward(monkeypatch, cfg, tokens, gathers):
    """The block's forward, gathered or packed, is the same bit for bit."""
    from moe_dispatch import layer
    from moe_dispatch.layer import MoEBlock, MoEConfig

    config = MoEConfig(*cfg)
    block = MoEBlock(config, device="cuda", implementation="cuda_fused", seed=3)
    gen = torch.Generator(device="cuda").manual_seed(4)
    x = torch.randn(tokens, config.hidden, device="cuda", generator=gen).bfloat16()
    first = block(x).clone()
    assert block._launches[(tokens, x.device)].gathered == gathers
    again = block(x).clone()  # the pre-bound launches
    monkeypatch.setattr(layer, "_gathers", lambda x, topk: False)
    packed_block = MoEBlock(config, device="cuda", implementation="cuda_fused", seed=3)
    packed = packed_block(x).clone()
    assert not packed_block._launches[(tokens, x.device)].gathered
    torch.cuda.synchronize()
    assert torch.equal(first, packed) and torch.equal(again, packed)
