"""Randomised routing and transport sweeps, from fixed seeds.

* Router: tokens (1-6000), hidden (multiples of 8 up to 8800, and the split-k
  and LDS-ring sizes above 8192), 1-64 experts and top-1 to top-8 drawn at
  random, so that every router kernel meets shapes the hand-picked cases do
  not. Checked as test_gpu_router.py checks it (logits against float64 within
  the fp32 bound, selection bit-exact on the kernel's own logits, equal to the
  exact-logit selection off near-ties), then the ranked route (ids, weights,
  in-tile ranks and tile counts from their definition), and the dispatch of
  those ids in both layouts (packed and row table, plain and ranked) and the
  combine, bit-exact against the oracle.
* Transport: fp16, fp32 and bf16 rows, any hidden size (the scalar path for
  sizes that are not multiples of 8), alignment 1-128, 1-64 experts, top-1
  to top-8, and ids partly out of range (masked: not counted, inverse left as
  it was, slot -1), as test_gpu_transport.py checks them.
"""

import numpy as np
import pytest
import torch

from moe_dispatch.workspace import CudaWorkspace
from oracle import moe_oracle as oracle
from tests._helpers import NP_DTYPE, assert_layout_equal, assert_packed_equal, gpu, route_margin, to_np

pytestmark = gpu


def _tile_reference(ids, tile, experts):
    """In-tile ranks (flat order) and per-tile expert counts, from their definition."""
    tokens, topk = ids.shape
    flat = ids.reshape(-1)
    ranks = np.empty_like(flat)
    counts = np.zeros((-(-tokens // tile), experts), np.int32)
    for p, e in enumerate(flat):
        t = p // topk // tile
        ranks[p] = counts[t, e]
        counts[t, e] += 1
    return ranks, counts.reshape(-1)


def _row_table(layout, topk):
    used = int(layout["offsets"][-1])
    table = np.full(used, -1, np.int64)
    inverse = layout["inverse"].reshape(-1)
    table[inverse] = np.arange(inverse.size) // topk
    return table


def _route_cases(seed, n):
    rng = np.random.default_rng(seed)
    for case in range(n):
        experts = int(rng.choice([1, 2, 3, 5, 8, 12, 16, 17, 24, 32, 33, 40, 48, 64]))
        topk = int(rng.integers(1, min(8, experts) + 1))
        tokens = int(np.exp(rng.uniform(0, np.log(6000))))
        if rng.random() < 0.2:
            tokens = int(rng.integers(1, 65))
        hidden = 8 * int(rng.integers(1, 1100))
        if rng.random() < 0.1 and experts <= 16:
            hidden = 64 * int(rng.integers(128, 258))
        while tokens * hidden > 3e7:  # keeps the float64 oracle to about a second
            tokens = max(1, tokens // 2)
        alignment = int(rng.choice([1, 8, 16, 128]))
        yield case, tokens, hidden, experts, topk, alignment


@pytest.mark.parametrize("seed", [31, 32])
def test_random_routes_and_dispatches(ext, seed):
    for case, tokens, hidden, experts, topk, alignment in _route_cases(seed, 30):
        print(f"seed {seed} case {case}: T={tokens} H={hidden} E={experts} K={topk} a={alignment}", flush=True)
        g = torch.Generator(device="cuda").manual_seed(100 * seed + case)
        x = torch.randn(tokens, hidden, device="cuda", generator=g).bfloat16()
        w = torch.randn(experts, hidden, device="cuda", generator=g) / hidden**0.5
        bias = torch.randn(experts, device="cuda", generator=g) * 0.1
        shape = (tokens, topk)
        ids32 = torch.empty(shape, device="cuda", dtype=torch.int32)
        ids64 = torch.empty(shape, device="cuda", dtype=torch.int64)
        weights = torch.empty(shape, device="cuda")
        logits = torch.empty(tokens, experts, device="cuda")
        ext.router_fused_out(x, w, bias, ids32, ids64, weights, logits)
        ref_logits = oracle.router_logits(to_np(x), to_np(w))
        got_logits = to_np(logits)
        scale = np.linalg.norm(to_np(x), axis=1)[:, None] * np.linalg.norm(to_np(w), axis=1)[None, :]
        assert np.all(np.abs(got_logits - ref_logits) <= 1e-6 * scale + 1e-7)
        ids_on_got, w_on_got, _ = oracle.topk_route(got_logits, to_np(bias), topk)
        np.testing.assert_array_equal(to_np(ids32), ids_on_got)
        np.testing.assert_array_equal(to_np(ids64), ids_on_got.astype(np.int64))
        np.testing.assert_allclose(to_np(weights), w_on_got, rtol=2e-6, atol=2e-6)
        ids_ref, _, _ = oracle.topk_route(ref_logits, to_np(bias), topk)
        safe = route_margin(ref_logits, to_np(bias), topk) > 1e-4
        np.testing.assert_array_equal(np.sort(to_np(ids32)[safe], 1), np.sort(ids_ref[safe], 1))
        ids = to_np(ids32)
        layout = oracle.dispatch_layout(ids, experts, alignment)
        used = int(layout["offsets"][-1])

        def workspace():
            return CudaWorkspace(tokens, hidden, experts, topk, torch.bfloat16, alignment=alignment, extension=ext)

        ws = workspace()
        ws.dispatch(x, ids32, ids64)
        assert_layout_equal(ws, layout, tokens, topk, experts)
        assert_packed_equal(ws.packed, x, layout, topk)
        y = torch.randn(ws.capacity_rows, hidden, device="cuda", generator=g).bfloat16()
        ws.combine(y, weights)
        np.testing.assert_array_equal(to_np(ws.output),
                                      oracle.combine(to_np(y), to_np(ws.inverse), to_np(weights), "bf16"))
        rows = workspace()
        rows.row_src.fill_(-7)
        rows.dispatch_rows(ids32)
        assert_layout_equal(rows, layout, tokens, topk, experts)
        np.testing.assert_array_equal(to_np(rows.row_src[:used]), _row_table(layout, topk))
        assert bool((rows.row_src[used:] == -7).all()), "rows past offsets[E] must not be written"
        tile = ext.router_rank_tile(tokens, experts)
        if tile <= 0:
            continue
        for rows_mode in (False, True):
            ranked = workspace()
            r = (torch.empty_like(ids32), torch.empty_like(ids64), torch.empty_like(weights))
            ext.router_fused_ranked_out(x, w, bias, *r, ranked.tile_ranks, ranked.tile_counts)
            assert torch.equal(r[0], ids32) and torch.equal(r[2], weights)
            ranks, counts = _tile_reference(ids, tile, experts)
            np.testing.assert_array_equal(to_np(ranked.tile_ranks).reshape(-1)[: ranks.size], ranks)
            np.testing.assert_array_equal(to_np(ranked.tile_counts).reshape(-1)[: counts.size], counts)
            if rows_mode:
                ranked.dispatch_ranked_rows(r[0])
                np.testing.assert_array_equal(to_np(ranked.row_src[:used]), _row_table(layout, topk))
            else:
                ranked.dispatch_ranked(x, r[0])
                assert_packed_equal(ranked.packed, x, layout, topk)
            assert_layout_equal(ranked, layout, tokens, topk, experts)


def _transport_cases(seed, n):
    rng = np.random.default_rng(seed)
    for case in range(n):
        dtype = (torch.float16, torch.float32, torch.bfloat16)[int(rng.integers(0, 3))]
        experts = int(rng.integers(1, 65))
        topk = int(rng.integers(1, min(8, experts) + 1))
        tokens = int(np.exp(rng.uniform(0, np.log(6000)))) if rng.random() > 0.05 else 0
        hidden = int(rng.integers(1, 2100)) if rng.random() < 0.5 else 8 * int(rng.integers(1, 300))
        while tokens * topk * hidden > 4e7:
            tokens = max(1, tokens // 2)
        alignment = int(rng.choice([1, 2, 3, 8, 16, 64, 128]))
        vectorized = bool(rng.integers(0, 4))
        out_of_range = rng.random() < 0.2
        yield case, dtype, tokens, hidden, experts, topk, alignment, vectorized, out_of_range


@pytest.mark.parametrize("seed", [41, 42, 43])
def test_random_transports(ext, seed):
    for case, dtype, tokens, hidden, experts, topk, alignment, vectorized, out_of_range in _transport_cases(seed, 40):
        print(f"seed {seed} case {case}: T={tokens} H={hidden} E={experts} K={topk} a={alignment} {dtype} "
              f"vectorized={vectorized} out_of_range={out_of_range}", flush=True)
        g = torch.Generator(device="cuda").manual_seed(100 * seed + case)
        x = torch.randn(tokens, hidden, device="cuda", generator=g).to(dtype)
        low, high = (-2, experts + 2) if out_of_range else (0, experts)
        ids = torch.randint(low, high, (tokens, topk), device="cuda", generator=g, dtype=torch.int32)
        w = torch.rand(tokens, topk, device="cuda", generator=g)
        ws = CudaWorkspace(tokens, hidden, experts, topk, dtype, vectorized=vectorized, alignment=alignment,
                           extension=ext)
        ws.inverse.fill_(-7)
        ws.dispatch(x, ids)
        layout = oracle.dispatch_layout(to_np(ids), experts, alignment)
        if out_of_range:
            np.testing.assert_array_equal(to_np(ws.counts), layout["counts"])
            np.testing.assert_array_equal(to_np(ws.offsets), layout["offsets"])
            got = to_np(ws.inverse).reshape(-1)
            ref = layout["inverse"].reshape(-1)
            valid = ref >= 0
            np.testing.assert_array_equal(got[valid], ref[valid])
            assert np.all(got[~valid] == -7)
            np.testing.assert_array_equal(to_np(ws.slots)[~valid], -1)
            continue
        assert_layout_equal(ws, layout, tokens, topk, experts)
        assert_packed_equal(ws.packed, x, layout, topk)
        y = torch.randn(ws.capacity_rows, hidden, device="cuda", generator=g).to(dtype)
        ws.combine(y, w)
        np.testing.assert_array_equal(to_np(ws.output),
                                      oracle.combine(to_np(y), to_np(ws.inverse), to_np(w), NP_DTYPE[dtype]))
