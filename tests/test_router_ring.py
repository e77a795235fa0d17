"""The fused router's LDS ring, replayed on the CPU.

router_ring_kernel (cuda-moe-engine_amd/csrc/router.hip) keeps STAGES = 4U
stages of 64 k in a ring (stage s in slot s % STAGES). It issues stages
0 .. STAGES-U-1 up front; then per iteration it waits until only STAGES-2U
stages' loads are outstanding, passes one barrier, refills the U slots the
previous iteration used with stages s0+STAGES-U .. s0+STAGES-1 (past the last
stage: the last one again) and computes stages s0 .. s0+U-1. Loads complete in
issue order. This replays that order for U = 1, 2, 4 and checks that each
wait covers every stage the iteration reads and that a refill only overwrites
a slot whose stage was read by an earlier iteration.
"""

import pytest


def replay(u, k_stages, wait_slack=0, refill_current=False):
    stages = 4 * u
    issued = []  # [stage, slot, landed]
    slot_of = {}  # slot -> index into issued of its latest load

    def issue(stage, slot):
        slot_of[slot] = len(issued)
        issued.append([stage, slot, False])

    for s in range(stages - u):
        issue(min(s, k_stages - 1), s)
    read = set()  # (stage, slot) pairs computed so far
    group = 0
    for s0 in range(0, k_stages, u):
        for entry in issued[: max(len(issued) - (stages - 2 * u) - wait_slack, 0)]:
            entry[2] = True
        refill = (group if refill_current else (3 if group == 0 else group - 1)) * u
        for j in range(u):
            slot = refill + j
            if slot in slot_of:
                old_stage = issued[slot_of[slot]][0]
                # A stage is read from slot stage % STAGES; that copy must be read before it is overwritten.
                assert old_stage % stages != slot or (old_stage, slot) in read, (u, k_stages, s0, slot)
            issue(min(s0 + stages - u + j, k_stages - 1), slot)
        for j in range(u):
            s = s0 + j
            if s >= k_stages:
                break
            slot = group * u + j
            latest = issued[slot_of[slot]]
            assert latest[0] == s and latest[2], (u, k_stages, s0, s)
            read.add((s, slot))
        group = 0 if group == 3 else group + 1
    assert {s for s, _ in read} == set(range(k_stages))


@pytest.mark.parametrize("u", [1, 2, 4])
def test_router_ring_waits_and_refills(u):
    for k_stages in (1, 2, 3, 4, 5, 7, 8, 9, 16, 17, 32, 64, 65):
        replay(u, k_stages)


@pytest.mark.parametrize("u", [1, 2, 4])
def test_replay_catches_a_short_wait_or_a_wrong_refill(u):
    with pytest.raises(AssertionError):
        replay(u, 64, wait_slack=1)
    with pytest.raises(AssertionError):
        replay(u, 64, refill_current=True)
