"""The grouped GEMM's LDS ring schedule, simulated on the CPU.

ring_tile (cuda-moe-engine_amd/csrc/gemm.hip) keeps SA stages of A and SB >= SA
stages of B in LDS (equal depths of 3-4 for small tiles, 2 and 3 for the full
256 x 256 tile), issues per stage window the A loads of stage u+SA and then
the B loads of stage u+SB into the slots stage u freed, and before reading
stage u+1 waits until at most VM_STEADY loads are outstanding. Loads complete in
issue order, so the wait is right exactly when no load of stage u+1 is among the
VM_STEADY newest. This replays the issue order for every tile shape the kernels
instantiate and checks that each wait covers both matrices of the stage it
guards and that no refill lands in a slot a still-unread stage occupies. The
depth and wait formulas below are the kernel's; a wrong count (e.g. treating the
A loads as the newest when SA == SB) fails here for the affected shapes.
The wide tiles cap the ring at 4 stages; the decode kernel's small stages go
up to 8.
"""

import itertools

import pytest

KIB = 1024
ROW_BYTES = 128  # one 64-k stage of one row


def equal_stages(a_stage, b_stage, lds, cap):
    return min(lds // (a_stage + b_stage), cap)


def b_stages(a_stage, b_stage, lds, cap):
    if equal_stages(a_stage, b_stage, lds, cap) >= 3:
        return equal_stages(a_stage, b_stage, lds, cap)
    fit = 0 if lds < 2 * a_stage else (lds - 2 * a_stage) // b_stage
    return min(fit, cap)


def a_stages(a_stage, b_stage, lds, cap):
    if equal_stages(a_stage, b_stage, lds, cap) >= 3:
        return equal_stages(a_stage, b_stage, lds, cap)
    sb = b_stages(a_stage, b_stage, lds, cap)
    return min((lds - sb * b_stage) // a_stage, sb)


def replay(tm, bnt, lds, k_steps, cap=4):
    a_stage, b_stage = tm * ROW_BYTES, bnt * ROW_BYTES
    sb, sa = b_stages(a_stage, b_stage, lds, cap), a_stages(a_stage, b_stage, lds, cap)
    a_loads, b_loads = tm // 32, bnt // 32  # 8 rows per load, four waves
    loads = a_loads + b_loads
    vm_steady = (b_loads if sb > sa else 0) + (sa - 2) * loads
    vm_first = (b_loads if sb > sa else 0) + (sa - 1) * loads
    assert 2 <= sa <= sb and sa * a_stage + sb * b_stage <= lds
    assert vm_first < 64  # vmcnt field

    issued = []  # [matrix, stage, slot, done]

    def wait(n):
        for entry in issued[: max(len(issued) - n, 0)]:
            entry[3] = True

    def landed(matrix, stage):
        mine = [e for e in issued if e[0] == matrix and e[1] == stage]
        return bool(mine) and all(e[3] for e in mine)

    for v in range(-sb, 0):  # prologue windows
        if v + sa >= 0:
            issued += [["A", v + sa, (v + sa) % sa, False] for _ in range(a_loads)]
        issued += [["B", v + sb, (v + sb) % sb, False] for _ in range(b_loads)]
    wait(vm_first)
    assert landed("A", 0) and landed("B", 0)
    for u in range(k_steps - 1):
        wait(vm_steady)
        assert landed("A", u + 1) and landed("B", u + 1), f"stage {u + 1}"
        issued += [["A", u + sa, u % sa, False] for _ in range(a_loads)]
        issued += [["B", u + sb, u % sb, False] for _ in range(b_loads)]
        assert all(s % sa != u % sa for s in range(u + 1, u + sa))
        assert all(s % sb != u % sb for s in range(u + 1, u + sb))
    return sa, sb


def _shapes():
    # Wide tiles: at most 4 stages in 160 KiB.
    shapes = {(tm, bnt, 160 * KIB, 4) for tm, bnt in itertools.product((64, 128, 256), (64, 128, 256))}
    shapes.add((32, 256, 160 * KIB, 4))  # short tiles of at most 32 rows
    shapes |= {(tm, 256, 160 * KIB, 4) for tm in (160, 192, 224)}  # balanced row tiles
    # Decode tiles (grouped_gemm_decode_kernel): at most 8 stages in 160 KiB.
    for max_rows, bnt in ((64, 32), (128, 64), (128, 128)):  # down at 64 and 128 rows, gate/up at 128
        shapes |= {(64, bnt, 160 * KIB, 8), (max_rows, bnt, 160 * KIB, 8)}
    shapes.add((64, 128, 3 * (64 + 128) * ROW_BYTES, 8))  # gate/up at 64 rows: three stages, two per CU
    return sorted(shapes)


@pytest.mark.parametrize("tm,bnt,lds,cap", _shapes())
def test_ring_waits_cover_each_stage(tm, bnt, lds, cap):
    for k_steps in (1, 2, 3, 4, 5, 7, 9, 64, 224):
        replay(tm, bnt, lds, k_steps, cap)


def test_decode_rings_keep_32_kib_of_weights_in_flight():
    # Stages in flight while one is read: SB - 1 of B.
    for tm, bnt in ((64, 32), (64, 64), (128, 64), (128, 128)):
        sa, sb = replay(tm, bnt, 160 * KIB, 64, cap=8)
        assert (sb - 1) * bnt * ROW_BYTES >= 28 * KIB, (tm, bnt, sa, sb)


def test_full_tile_uses_all_lds_as_two_a_and_three_b_stages():
    assert replay(256, 256, 160 * KIB, 64) == (2, 3)


def test_small_tiles_get_equal_depths():
    assert replay(64, 64, 3 * 128 * ROW_BYTES, 8) == (3, 3)
    assert replay(64, 256, 160 * KIB, 8) == (4, 4)
    assert replay(64, 32, 160 * KIB, 8, cap=8) == (8, 8)


def replay_chain(tm, bnt, lds, k_steps, tiles=3, cap=4):
    """Consecutive tiles of one shape chained as the persistent kernel does.

    Tile t's stage s sits in slots (a0 + s) % SA and (b0 + s) % SB. Its last
    windows, which would reload its last stage, load the next tile's first
    stages into the slots that follow; after its k-loop (every wave done with
    the ring) the hook issues the prologue's last window of the next tile, which
    then waits for all loads before its first read. Checks that every read
    stage has landed, that no load overwrites a slot whose stage is still to be
    read, and that the next tile finds its stages where it looks for them.
    """
    a_stage, b_stage = tm * ROW_BYTES, bnt * ROW_BYTES
    sb, sa = b_stages(a_stage, b_stage, lds, cap), a_stages(a_stage, b_stage, lds, cap)
    assert k_steps >= sb
    a_loads, b_loads = tm // 32, bnt // 32
    loads = a_loads + b_loads
    vm_steady = (b_loads if sb > sa else 0) + (sa - 2) * loads
    issued = []  # [matrix, tile, stage, slot, done]
    slot_holds = {("A", i): None for i in range(sa)} | {("B", i): None for i in range(sb)}  # (tile, stage)

    def issue(matrix, tile, stage, slot, n):
        held = slot_holds[(matrix, slot)]
        # the slot's previous stage must already have been read (consumed)
        assert held is None or held in consumed, (matrix, tile, stage, slot, held)
        slot_holds[(matrix, slot)] = (tile, stage)
        issued.extend([[matrix, tile, stage, slot, False] for _ in range(n)])

    def wait(n):
        for entry in issued[: max(len(issued) - n, 0)]:
            entry[4] = True

    def landed(matrix, tile, stage, slot):
        # the loads of this stage into the slot it is read from (the last tile's
        # reloads of its last stage go to other slots and are never read)
        mine = [e for e in issued if e[:4] == [matrix, tile, stage, slot]]
        return bool(mine) and all(e[4] for e in mine) and slot_holds[(matrix, slot)] == (tile, stage)

    consumed = set()
    a0 = b0 = 0
    for v in range(-sb, 0):  # tile 0's full prologue at slots 0
        if v + sa >= 0:
            issue("A", 0, v + sa, (v + sa) % sa, a_loads)
        issue("B", 0, v + sb, (v + sb) % sb, b_loads)
    for t in range(tiles):
        chain = t + 1 < tiles
        wait(0)  # the first wait of a tile after an epilogue (or the kernel's first) takes everything
        assert landed("A", t, 0, a0 % sa) and landed("B", t, 0, b0 % sb)
        for u in range(k_steps - 1):
            if u > 0:
                wait(vm_steady)
            assert landed("A", t, u + 1, (a0 + u + 1) % sa) and landed("B", t, u + 1, (b0 + u + 1) % sb)
            consumed.add((t, u))  # stage u's last reads happen before this window's refills
            sa_slot, sb_slot = (a0 + u) % sa, (b0 + u) % sb
            for matrix, depth, slot, n in (("A", sa, sa_slot, a_loads), ("B", sb, sb_slot, b_loads)):
                stage = u + depth
                if stage < k_steps:
                    issue(matrix, t, stage, slot, n)
                elif chain:
                    issue(matrix, t + 1, stage - k_steps, slot, n)
                else:  # the last tile reloads its last stage into a freed slot (never read)
                    slot_holds[(matrix, slot)] = None
                    issued.extend([[matrix, t, k_steps - 1, slot, False] for _ in range(n)])
        consumed.add((t, k_steps - 1))
        if not chain:
            break
        a0, b0 = (a0 + k_steps) % sa, (b0 + k_steps) % sb
        # hook: the prologue's last window of the next tile (A stage SA-1, B stage SB-1)
        issue("A", t + 1, sa - 1, (a0 + sa - 1) % sa, a_loads)
        issue("B", t + 1, sb - 1, (b0 + sb - 1) % sb, b_loads)
        for s in range(sa):
            assert slot_holds[("A", (a0 + s) % sa)] == (t + 1, s)
        for s in range(sb):
            assert slot_holds[("B", (b0 + s) % sb)] == (t + 1, s)
    return sa, sb


@pytest.mark.parametrize("tm,bnt", [(256, 256), (224, 256), (192, 256), (160, 256), (128, 256), (64, 256), (32, 256),
                                    (256, 128), (128, 128), (64, 128), (256, 64), (128, 64), (64, 64)])
def test_chained_tiles_find_their_stages(tm, bnt):
    for k_steps in (4, 5, 7, 16, 64, 65):
        replay_chain(tm, bnt, 160 * KIB, k_steps)


def test_chained_start_slots_follow_the_k_chain():
    """k_steps = 5 on the full tile (SA = 2, SB = 3): the next tile starts at A slot 1
    and B slot 2, not 0; the replay above checks it finds its stages there."""
    sa, sb = replay_chain(256, 256, 160 * KIB, 5, tiles=2)
    assert (sa, sb) == (2, 3) and (0 + 5) % sa == 1 and (0 + 5) % sb == 2
