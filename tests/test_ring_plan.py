"""The persistent grouped GEMM's tile plan, restated and checked on the CPU.

grouped_gemm_persistent_kernel (cuda-moe-engine_amd/csrc/gemm.hip: ring_plan,
ring_slot) walks virtual workgroups q = blockIdx.x + i*G in rounds of G. Full
row tiles (phase 1) run in 8 XCD-contiguous ranges, cpr per XCD and round;
the other slots of the rounds carry one or two of the experts' short last row
tiles (phase 2); phase-2 tiles the rounds do not take, or phase 1 when there is
no phase 2, run after the rounds with an optional split of a short last round
into 128-column pieces (plain GEMM only); a phase 1 that fills at most half of
one round beside a phase 2 runs in the rounds as 128-column halves (plain GEMM
only). The gate/up GEMM at K >= 2048 cuts each expert of more than 128 rows
into ceil(rows/256) balanced row tiles, all in phase 1. This restates those
formulas and checks that every tile (or both halves of a split tile) is
assigned exactly once for random expert layouts and grid sizes, that the
rounds keep each XCD's phase-1 tiles in order, that balanced tiles cover each
expert's rows once, and that the measured shapes get the intended plans.
The GPU test tests/test_gpu_gemm.py::test_schedule_does_not_change_results runs
the kernel itself at the grid sizes used here.
"""

import random

import pytest

XCD = 8


def phase_tiles(span, balanced):
    """(phase-1 row tiles, their height) of one expert (ring_table, ring_locate)."""
    tiles = -(-span // 256)
    if not balanced:
        return span // 256 + (1 if span % 256 > 128 else 0), 256
    mf = tiles if span > 128 else 0
    return mf, (-(-span // mf) + 31) // 32 * 32 if mf else 256


def phase_counts(counts, alignment, n_tiles, balanced=False):
    spans = [(c + alignment - 1) // alignment * alignment for c in counts]
    mf = [phase_tiles(s, balanced)[0] for s in spans]
    n1 = sum(m * n_tiles for m in mf)
    n2 = sum((-(-s // 256) - m) * n_tiles for s, m in zip(spans, mf))
    return n1, n2


def balanced_for(swiglu, k):
    return swiglu and k >= 2048


def ring_phase(count, grid, allow_split, short_tiles=False):
    rem = count % grid
    split = allow_split and rem > 0 and 2 * rem <= grid
    ways = 4 if short_tiles and 4 * rem <= grid else 2
    main = count - rem if split else count
    return {"main": main, "blocks": (main + XCD - 1) // XCD * XCD, "pieces": ways * rem if split else 0,
            "ways": ways}


def ring_plan(n1, n2, grid, allow_split):
    half1 = allow_split and n2 > 0 and n1 > 0 and 2 * n1 <= grid
    pl = {"n1": n1, "n2": n2, "half1": half1, "u1": 2 * n1 if half1 else n1, "per1": 0, "cpr": 0, "rounds": 0,
          "full_rounds": 0, "last_cols": 0, "slots": 0, "carried": 0}
    if n2 > 0 and n1 > 0:
        per1 = (pl["u1"] + XCD - 1) // XCD
        rounds = (per1 + grid // XCD - 1) // (grid // XCD)
        if n2 - 2 * (rounds * grid - XCD * per1) > grid:
            rounds += 1
        cpr = (per1 + rounds - 1) // rounds
        slots = rounds * grid - XCD * per1
        pl.update(per1=per1, rounds=rounds, cpr=cpr, full_rounds=per1 // cpr,
                  last_cols=per1 - (per1 // cpr) * cpr, slots=slots, carried=min(n2, 2 * slots))
    pl["rest"] = ring_phase(n2 - pl["carried"] if n2 > 0 else n1, grid, allow_split, n2 > 0)
    pl["virtual_blocks"] = pl["rounds"] * grid + pl["rest"]["blocks"] + pl["rest"]["pieces"]
    return pl


def ring_slot(pl, grid, q, sub):
    """(phase, tile, piece) of tile `sub` of virtual workgroup q, or None."""
    base = pl["rounds"] * grid
    if q < base:
        r, pos = divmod(q, grid)
        per_xcd = grid // XCD
        j = (pos // XCD + r * (per_xcd - pl["cpr"])) % per_xcd  # rotated per round
        cols = pl["cpr"] if r < pl["full_rounds"] else (pl["last_cols"] if r == pl["full_rounds"] else 0)
        if j < cols:
            unit = (pos % XCD) * pl["per1"] + r * pl["cpr"] + j
            if sub or unit >= pl["u1"]:
                return None
            return (0, unit // 2, unit % 2) if pl["half1"] else (0, unit, -1)
        per_round = grid - XCD * pl["cpr"]
        if r <= pl["full_rounds"]:
            idx = r * per_round
        else:
            idx = pl["full_rounds"] * per_round + grid - XCD * pl["last_cols"] + (r - pl["full_rounds"] - 1) * grid
        idx += (j - cols) * XCD + pos % XCD
        lo = idx * pl["carried"] // pl["slots"]
        hi = (idx + 1) * pl["carried"] // pl["slots"]
        return (1, lo + sub, -1) if lo + sub < hi else None
    if sub:
        return None
    phase = 1 if pl["n2"] > 0 else 0
    first = pl["carried"] if pl["n2"] > 0 else 0
    rest, v = pl["rest"], q - base
    if v < rest["blocks"]:
        per = rest["blocks"] // XCD
        tile = (v % XCD) * per + v // XCD
        return (phase, first + tile, -1) if tile < rest["main"] else None
    if v - rest["blocks"] < rest["pieces"]:
        r = v - rest["blocks"]
        ways = rest["ways"]
        return (phase, first + rest["main"] + r // ways, 4 + r % 4 if ways == 4 else r % 2)
    return None


def walk(n1, n2, grid, allow_split):
    """Per workgroup, the (phase, tile, piece) sequence it runs."""
    pl = ring_plan(n1, n2, grid, allow_split)
    runs = []
    for wg in range(grid):
        seq = []
        for q in range(wg, pl["virtual_blocks"], grid):
            for sub in (0, 1):
                s = ring_slot(pl, grid, q, sub)
                if s is not None:
                    seq.append((q, s))
        runs.append(seq)
    return pl, runs


def check_cover(n1, n2, grid, allow_split):
    pl, runs = walk(n1, n2, grid, allow_split)
    seen = {}
    for seq in runs:
        for _, (phase, tile, piece) in seq:
            key = (phase, tile, piece)
            assert key not in seen, f"tile {key} assigned twice"
            seen[key] = True
    parts = {}
    for phase, tile, piece in seen:
        parts.setdefault((phase, tile), set()).add(piece)
    assert set(parts) == {(0, t) for t in range(n1)} | {(1, t) for t in range(n2)}
    assert all(p in ({-1}, {0, 1}, {4, 5, 6, 7}) for p in parts.values())
    # Quarters only for short tiles (phase 2), halves for either phase.
    assert all(phase == 1 for (phase, _), p in parts.items() if p == {4, 5, 6, 7})
    assert not (pl["carried"] and not allow_split and pl["rest"]["pieces"])
    # In the rounds, the workgroups of XCD x (those with blockIdx % 8 == x) run
    # exactly phase-1 range x (of tiles, or of halves), each round's before the next round's.
    for x in range(XCD):
        ranged = sorted((q // grid, 2 * s[1] + s[2] if pl["half1"] else s[1]) for seq in runs[x::XCD]
                        for q, s in seq if s[0] == 0 and q < pl["rounds"] * grid)
        first = x * pl["per1"]
        assert [t for _, t in ranged] == list(range(first, min(first + pl["per1"], pl["u1"])))
    assert not pl["half1"] or allow_split
    return pl, runs


@pytest.mark.parametrize("seed", range(6))
def test_every_tile_runs_once(seed):
    rng = random.Random(seed)
    for _ in range(120):
        experts = rng.randint(1, 64)
        counts = [rng.choice([0, rng.randint(1, 40), rng.randint(0, 600), rng.randint(0, 3000)])
                  for _ in range(experts)]
        n1, n2 = phase_counts(counts, rng.choice([1, 8]), rng.randint(1, 40), rng.random() < 0.5)
        check_cover(n1, n2, rng.choice([8, 16, 24, 64, 256]), rng.random() < 0.5)


def test_balanced_row_tiles_cover_each_expert_once():
    """Balanced phase-1 tiles: ceil(rows/256) tiles of one height, a multiple of
    32 between 160 and 256 (the row variants that exist) when there are two or
    more, none empty, together covering the expert's rows exactly once; the
    tile count per expert is the plain rule's."""
    for span in range(1, 12000):
        plain_tiles = -(-span // 256)
        mf, h = phase_tiles(span, True)
        if span <= 128:
            assert mf == 0
            continue
        assert mf == plain_tiles
        assert h % 32 == 0 and h <= 256 and (mf == 1 or h >= 160)
        rows = [r for m in range(mf) for r in range(m * h, min((m + 1) * h, span))]
        assert rows == list(range(span)), span
        assert (mf - 1) * h < span, f"empty last tile at {span} rows"


def test_grid_sizes_used_on_the_gpu_cover_each_path():
    """The GPU schedule test's cases reach the two-tile slots, leftovers and split pieces."""
    from tests.test_gpu_gemm import SCHEDULE_CASES

    reached = set()
    for counts, alignment, n, k, swiglu, grids in SCHEDULE_CASES:
        n_tiles = -(-n // (128 if swiglu else 256))
        n1, n2 = phase_counts(counts, alignment, n_tiles, balanced_for(swiglu, k))
        for grid in grids:
            pl, runs = check_cover(n1, n2, grid, not swiglu)
            per_q = {}
            for seq in runs:
                for q, _ in seq:
                    per_q[q] = per_q.get(q, 0) + 1
            if max(per_q.values(), default=0) == 2:
                reached.add("two tiles in a slot")
            if pl["carried"] and pl["carried"] < n2:
                reached.add("leftover after the rounds")
            if pl["rest"]["pieces"]:
                reached.add("quarters" if pl["rest"]["ways"] == 4 else "pieces")
            if pl["rounds"] and pl["last_cols"]:
                reached.add("partial last round")
            if pl["rounds"] > (pl["per1"] + grid // XCD - 1) // (grid // XCD):
                reached.add("extra round")
            if pl["half1"]:
                reached.add("halves in the rounds")
    assert reached == {"two tiles in a slot", "leftover after the rounds", "pieces", "quarters",
                       "partial last round", "extra round", "halves in the rounds"}


def test_phase2_slots_rotate_over_the_cus():
    # Plain row tiles, 14 rounds of 30 phase-1 columns per XCD: each workgroup
    # carries short tiles in at most one round.
    c4 = [1040, 1095, 1010, 1026, 1019, 1025, 1003, 974]
    pl, runs = check_cover(*phase_counts(c4, 8, 112), 256, False)
    rounds_carrying = [len({q for q, s in seq if s[0] == 1}) for seq in runs]
    assert max(rounds_carrying) == 1 and sum(rounds_carrying) == pl["slots"] == 256


def test_measured_shapes_get_the_intended_plans():
    # H=4096, I=14336, E=8, 4096 tokens (counts from the bench). Gate/up GEMM
    # (K=4096: balanced row tiles): the four experts of 1032-1096 rows get five
    # 224-row tiles each, the others four of 256; no short tiles, so phase 1
    # runs alone: 4032 tiles, 15.75 rounds.
    c4 = [1040, 1095, 1010, 1026, 1019, 1025, 1003, 974]
    assert [phase_tiles(-(-c // 8) * 8, True) for c in c4] == [(5, 224), (5, 224), (4, 256), (5, 224), (4, 256),
                                                               (5, 224), (4, 256), (4, 256)]
    pl = ring_plan(*phase_counts(c4, 8, 112, balanced_for(True, 4096)), 256, False)
    assert (pl["rounds"], pl["n2"], pl["rest"]["blocks"]) == (0, 0, 4032)
    # With plain row tiles, 14 rounds of phase 1 alone would leave 448 short
    # tiles for the end; one more round carries them all.
    pl = ring_plan(*phase_counts(c4, 8, 112), 256, False)
    assert (pl["rounds"], pl["cpr"], pl["carried"], pl["n2"]) == (15, 30, 448, 448)
    # Its down GEMM (512 full tiles = 2 rounds, 64 short tiles): no extra round;
    # the short tiles run last as 256 quarters, one per workgroup.
    pl = ring_plan(*phase_counts(c4, 8, 16), 256, True)
    assert (pl["rounds"], pl["carried"], pl["rest"]["pieces"], pl["rest"]["ways"]) == (2, 0, 256, 4)
    # H=1024, I=2048, E=16, 4096 tokens, down GEMM (4 column tiles): 128 full
    # tiles run as 256 halves in one round; the short tiles follow as quarters.
    c3 = [510, 525, 498, 530, 515, 505, 520, 490, 512, 507, 533, 495, 516, 511, 522, 503]
    pl = ring_plan(*phase_counts(c3, 8, 4), 256, True)
    assert (pl["half1"], pl["u1"], pl["rounds"], pl["carried"], pl["rest"]["ways"]) == (True, 256, 1, 0, 4)
    assert not ring_plan(*phase_counts(c3, 8, 8), 256, False)["half1"]  # its gate/up GEMM: never split
    # No short tiles: phase 1 alone, as before.
    pl = ring_plan(*phase_counts([1024] * 8, 8, 112), 256, False)
    assert (pl["rounds"], pl["rest"]["blocks"]) == (0, 3584)


def phase1_tile(rel, mf, n_tiles):
    """ring_locate's phase-1 mapping: an expert's row tiles in groups of at most 8
    (balanced heights), column tiles fastest inside a group, row tiles fastest
    inside a column. Returns (column tile, row tile)."""
    groups = (mf + 7) // 8
    hg = -(-mf // groups)
    full = hg * n_tiles
    g = rel // full
    height = min(hg, mf - g * hg)
    r = rel - g * full
    n = r // height
    return n, g * hg + (r - n * height)


def test_phase1_tile_order_covers_each_tile_once_in_groups_of_eight():
    for mf in range(1, 70):
        for n_tiles in (1, 2, 3, 7, 8, 11, 16, 112):
            tiles = [phase1_tile(rel, mf, n_tiles) for rel in range(mf * n_tiles)]
            assert sorted(tiles) == [(n, m) for n in range(n_tiles) for m in range(mf)]
            if mf <= 8:  # the plain order: row tiles fastest
                assert tiles == [(rel // mf, rel % mf) for rel in range(mf * n_tiles)]
    # 32 row tiles, 11 column tiles (H=2048, I=1408 gate/up): any 32 consecutive
    # tiles span at most 8 row tiles (four groups of 8); the plain order spanned 32.
    tiles = [phase1_tile(rel, 32, 11) for rel in range(32 * 11)]
    for start in range(0, len(tiles) - 32, 32):
        window = tiles[start:start + 32]
        assert len({m for _, m in window}) <= 16 and len({n for n, _ in window}) >= 2
