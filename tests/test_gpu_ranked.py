"""The ranked route: the fused router does the dispatch's counting pass.

``router_fused_ranked_out`` writes, for each tile of ``router_rank_tile(T, E)``
tokens, the tile's expert counts and every assignment's rank among the
tile's earlier assignments to the same expert (flat order p = t*K + k);
``CudaWorkspace.dispatch_ranked`` then runs only the pack pass. Checked here
on every router kernel (the VGPR-load kernels: 16-token tiles for E <= 16,
32-token tiles above; split-k small batches; the LDS ring for hidden > 8192 at
E <= 16 and hidden > 4096 above; ragged last tiles, alignment 1 and 8):

* ranks and tile counts equal a numpy restatement of their definition;
* ids, weights and the whole dispatch layout (counts, offsets, slots,
  inverse, packed rows) equal the unranked route + dispatch bit for bit, and
  the layout equals the oracle's;
* dispatch_ranked can be repeated (it only reads the ranks).
"""

import numpy as np
import pytest
import torch

from moe_dispatch.workspace import CudaWorkspace
from oracle import moe_oracle as oracle
from tests._helpers import assert_layout_equal, assert_packed_equal, gpu, raw_bits, to_np

pytestmark = gpu

CASES = [
    # tokens, hidden, experts, topk, alignment
    (300, 512, 8, 2, 8),      # VGPR-load router, ragged last tile
    (1000, 1024, 16, 2, 1),   # VGPR-load router, E = 16
    (40, 2048, 8, 2, 8),      # split-k router (T <= 64) and its selection kernel
    (130, 8200, 8, 2, 1),     # LDS ring router, E <= 16
    (200, 256, 32, 4, 8),     # many-expert VGPR-load router, E = 32: 32-token tiles
    (100, 128, 64, 6, 1),     # many-expert VGPR-load router, E = 64
    (70, 4160, 32, 4, 8),     # LDS ring router, E = 32
    (17, 64, 5, 3, 16),       # one partial tile
]


def _tile_reference(ids, tile, experts):
    """In-tile ranks (flat order) and per-tile expert counts, from their definition."""
    tokens, topk = ids.shape
    flat = ids.reshape(-1)
    ranks = np.empty_like(flat)
    tiles = -(-tokens // tile)
    counts = np.zeros((tiles, experts), np.int32)
    for p, e in enumerate(flat):
        t = p // topk // tile
        ranks[p] = counts[t, e]
        counts[t, e] += 1
    return ranks, counts.reshape(-1)


@pytest.mark.parametrize("tokens,hidden,experts,topk,alignment", CASES)
def test_ranked_route_and_dispatch_match_the_unranked_pair(ext, tokens, hidden, experts, topk, alignment):
    gen = torch.Generator(device="cuda").manual_seed(tokens + hidden)
    x = torch.randn(tokens, hidden, device="cuda", generator=gen).bfloat16()
    w = torch.randn(experts, hidden, device="cuda", generator=gen) / hidden**0.5
    bias = torch.randn(experts, device="cuda", generator=gen) * 0.1
    tile = ext.router_rank_tile(tokens, experts)
    assert tile == (16 if experts <= 16 else 32)

    def buffers():
        shape = (tokens, topk)
        return (torch.empty(shape, device="cuda", dtype=torch.int32),
                torch.empty(shape, device="cuda", dtype=torch.int64),
                torch.empty(shape, device="cuda"))

    plain, ranked = buffers(), buffers()
    ws_plain = CudaWorkspace(tokens, hidden, experts, topk, torch.bfloat16, alignment=alignment, extension=ext)
    ws_ranked = CudaWorkspace(tokens, hidden, experts, topk, torch.bfloat16, alignment=alignment, extension=ext)
    assert ws_ranked.rank_tile == tile
    ext.router_fused_out(x, w, bias, *plain)
    ws_plain.dispatch(x, plain[0], plain[1])
    ws_ranked.tile_ranks.fill_(-7)
    ext.router_fused_ranked_out(x, w, bias, *ranked, ws_ranked.tile_ranks, ws_ranked.tile_counts)
    for a, b in zip(plain, ranked):
        assert torch.equal(a, b)
    ids = to_np(ranked[0])
    ranks, counts = _tile_reference(ids, tile, experts)
    np.testing.assert_array_equal(to_np(ws_ranked.tile_ranks), ranks)
    np.testing.assert_array_equal(to_np(ws_ranked.tile_counts)[: counts.size], counts)
    layout = oracle.dispatch_layout(ids, experts, alignment)
    for _ in range(2):  # the pack pass reads the ranks only: a second call is the same
        ws_ranked.dispatch_ranked(x, ranked[0])
        assert_layout_equal(ws_ranked, layout, tokens, topk, experts)
        assert_packed_equal(ws_ranked.packed, x, layout, topk)
    used = int(layout["offsets"][-1])
    np.testing.assert_array_equal(raw_bits(ws_ranked.packed)[:used], raw_bits(ws_plain.packed)[:used])
    for name in ("counts", "offsets", "slots", "inverse"):
        assert torch.equal(getattr(ws_ranked, name), getattr(ws_plain, name)), name


def test_shapes_without_a_ranked_route_keep_the_counting_pass(ext):
    # 8192 tokens x 64 experts: 256 tiles x 64 counts exceed the table bound.
    assert ext.router_rank_tile(8192, 64) == 0
    ws = CudaWorkspace(8192, 64, 64, 6, torch.bfloat16, extension=ext)
    assert ws.rank_tile == 0
    x = torch.zeros(8192, 64, device="cuda", dtype=torch.bfloat16)
    ids = torch.zeros(8192, 6, device="cuda", dtype=torch.int32)
    with pytest.raises(RuntimeError, match="no ranked route"):
        ws.dispatch_ranked(x, ids)


@pytest.mark.parametrize("tokens,hidden,experts,topk", [(4096, 4096, 8, 2), (4096, 1024, 16, 2)])
def test_benchmark_routing_on_every_token(ext, tokens, hidden, experts, topk):
    """The ranked route the block's forward takes at C4 T=4096 (H=4096, E=8, top-2;
    the timed benchmark) and C3 T=4096 (H=1024, E=16), over every token: the
    logits are within the fp32 bound of the float64 logits, the ids equal the
    oracle's selection on the kernel's own logits bit for bit (weights within
    2e-6), the call without logits (as the forward makes it) selects the same ids
    and weights, and ranks and tile counts equal their definition."""
    gen = torch.Generator(device="cuda").manual_seed(0)
    x = torch.randn(tokens, hidden, device="cuda", generator=gen).bfloat16()
    w = torch.randn(experts, hidden, device="cuda", generator=gen) / hidden**0.5
    bias = torch.zeros(experts, device="cuda")
    tile = ext.router_rank_tile(tokens, experts)
    assert tile == 16
    tables = -(-tokens // tile) * experts

    def run(with_logits):
        shape = (tokens, topk)
        out = [torch.empty(shape, device="cuda", dtype=torch.int32),
               torch.empty(shape, device="cuda", dtype=torch.int64),
               torch.empty(shape, device="cuda"),
               torch.full((tokens * topk,), -7, device="cuda", dtype=torch.int32),
               torch.full((tables,), -7, device="cuda", dtype=torch.int32)]
        logits = torch.empty(tokens, experts, device="cuda") if with_logits else None
        ext.router_fused_ranked_out(x, w, bias, *out, logits=logits)
        return out, logits

    (ids32, ids64, weights, ranks, tile_counts), logits = run(True)
    got_logits = to_np(logits)
    ref_logits = oracle.router_logits(to_np(x), to_np(w))
    scale = np.linalg.norm(to_np(x).astype(np.float64), axis=1)[:, None] * np.linalg.norm(to_np(w), axis=1)[None, :]
    assert np.all(np.abs(got_logits - ref_logits) <= 1e-6 * scale + 1e-7)
    ids_ref, w_ref, _ = oracle.topk_route(got_logits, to_np(bias), topk)
    np.testing.assert_array_equal(to_np(ids32), ids_ref)
    np.testing.assert_array_equal(to_np(ids64), ids_ref.astype(np.int64))
    np.testing.assert_allclose(to_np(weights), w_ref, rtol=2e-6, atol=2e-6)
    plain, none = run(False)
    assert none is None
    for a, b in zip(plain, (ids32, ids64, weights, ranks, tile_counts)):
        assert torch.equal(a, b)
    r_ref, c_ref = _tile_reference(ids_ref, tile, experts)
    np.testing.assert_array_equal(to_np(ranks), r_ref)
    np.testing.assert_array_equal(to_np(tile_counts), c_ref)
