"""Pins the pager oracle (oracle/pager.py) with known-answer traces derived by
hand from the reference source text (src/wisp/integrations/vllm/
fused_moe.py:264-358, 1119-1140) and with the invariants of the reference's
own tests (tests/test_wisp_state.py)."""
import random

import pytest

from oracle.pager import PagerOracle, PagerOverflow, plan_groups


def run(E, cap, needs):
    p = PagerOracle(E, cap)
    return p, [p.ensure_resident(n) for n in needs]


def test_kat_lru_eviction_order():
    # E=8 cap=4: [0,1] -> 0->3, 1->2 (free.pop() takes the highest slot);
    # [2,3] -> 2->1, 3->0; [4] -> all four slots are candidates, ticks
    # [2,2,1,1], stable sort by tick -> slot 2 (expert 1) goes first.
    p, recs = run(8, 4, [[0, 1], [2, 3], [4]])
    assert recs[0]["loaded"] == [(0, 3), (1, 2)]
    assert recs[1]["loaded"] == [(2, 1), (3, 0)]
    assert recs[2]["evicted"] == [(1, 2)] and recs[2]["loaded"] == [(4, 2)]
    assert p.slot_to_expert == [3, 2, 4, 0]
    assert p.lru_tick == [2, 2, 3, 1]
    assert (p.stats_miss, p.stats_evict, p.stats_hits, p.lru_clock) == (5, 1, 0, 3)


def test_kat_cpython_set_order_drives_slots():
    # set([2, 9]) iterates 9 then 2 (9 & 7 == 1 < 2), so 9 takes slot 3.
    # set([3, 11]): 3 -> slot 3, 11 collides at 3 and lands in slot 0 -> [11, 3].
    # [9, 5]: 9 hits, 5 misses; candidates slot 2 (tick 1) before 0, 1 (tick 2).
    p, recs = run(16, 4, [[2, 9], [3, 11], [9, 5]])
    assert recs[0]["loaded"] == [(9, 3), (2, 2)]
    assert recs[1]["loaded"] == [(11, 1), (3, 0)]
    assert recs[2]["hits"] == 1
    assert recs[2]["evicted"] == [(2, 2)] and recs[2]["loaded"] == [(5, 2)]
    assert p.slot_to_expert == [3, 11, 5, 9]
    assert p.lru_tick == [2, 2, 3, 3]


def test_kat_free_then_evicted_slots_pop_from_end():
    # [0,1,2] fills slots 3,2,1; [3,4,5]: free=[0], evict slots 1,2 (ties,
    # ascending) -> free=[0,1,2]; pops give 3->2, 4->1, 5->0.
    p, recs = run(8, 4, [[0, 1, 2], [3, 4, 5]])
    assert recs[0]["loaded"] == [(0, 3), (1, 2), (2, 1)]
    assert recs[1]["evicted"] == [(2, 1), (1, 2)]
    assert recs[1]["loaded"] == [(3, 2), (4, 1), (5, 0)]
    assert p.slot_to_expert == [5, 4, 3, 0]
    assert p.lru_tick == [2, 2, 2, 1]


def test_kat_all_hit_touches_clock():
    p, recs = run(8, 4, [[0, 1], [1, 0, 1]])
    assert recs[1]["hits"] == 2 and recs[1]["loaded"] == [] and recs[1]["evicted"] == []
    assert p.lru_clock == 2 and p.lru_tick == [0, 0, 2, 2]
    assert p.stats_hits == 2 and p.stats_miss == 2


def test_kat_subbatch_groups_and_slots():
    # cap 4, three tokens x 2 experts: union 6 > 4, greedy -> [0,2), [2,3)
    p = PagerOracle(8, 4)
    res = p.forward([[0, 1], [2, 3], [4, 5]])
    assert res["groups"] == [(0, 2), (2, 3)]
    assert res["records"][0]["loaded"] == [(0, 3), (1, 2), (2, 1), (3, 0)]
    assert res["records"][1]["evicted"] == [(3, 0), (2, 1)]
    assert res["records"][1]["loaded"] == [(4, 1), (5, 0)]
    assert res["slots"] == [[3, 2], [1, 0], [1, 0]]
    assert p.slot_to_expert == [5, 4, 1, 0]
    assert (p.stats_forward, p.stats_miss, p.stats_evict, p.stats_hits) == (1, 6, 2, 0)


def test_kat_empty_call_ticks_clock():
    p = PagerOracle(8, 4)
    res = p.forward([])
    assert res["groups"] == [(0, 0)] and p.lru_clock == 1 and p.stats_forward == 1


def test_overflow_raises_subbatch_after_counting_hits():
    p = PagerOracle(8, 2)
    p.ensure_resident([0])
    with pytest.raises(RuntimeError, match="sub-batch"):
        p.ensure_resident([0, 1, 2])
    assert p.stats_hits == 1 and p.lru_clock == 1 and p.slot_to_expert == [-1, 0]
    with pytest.raises(PagerOverflow):
        PagerOracle(8, 2).forward([[0, 1, 2]])


def test_plan_groups_first_fit():
    assert plan_groups([[0, 1], [1, 2], [3, 4]], 3) == [(0, 2), (2, 3)]
    assert plan_groups([[0, 1], [0, 1]], 2) == [(0, 2)]
    # a token that alone exceeds cap still gets its own group
    assert plan_groups([[0, 1, 2], [3, 4, 5]], 2) == [(0, 1), (1, 2)]


def _consistent(p: PagerOracle):
    m = p.expert_map()
    for e, s in p.expert_to_slot.items():
        assert p.slot_to_expert[s] == e and m[e] == s
    for s, e in enumerate(p.slot_to_expert):
        if e != -1:
            assert p.expert_to_slot[e] == s


def test_invariants_random_walk():
    # reference tests/test_wisp_state.py:53-68, 96-103, 112-121
    rng = random.Random(0)
    for E, cap in [(8, 4), (16, 5), (128, 8), (128, 24)]:
        p = PagerOracle(E, cap)
        for _ in range(300):
            k = rng.randint(1, cap)
            need = rng.sample(range(E), k)
            before = dict(p.expert_to_slot)
            rec = p.ensure_resident(need)
            for e in need:
                assert e in p.expert_to_slot
            for victim, _s in rec["evicted"]:
                assert victim not in need and victim in before
            assert rec["hits"] + len(rec["loaded"]) == len(set(need))
            _consistent(p)


def test_resize_semantics():
    # reference tests/test_wisp_state.py:124-167
    p = PagerOracle(8, 4)
    p.ensure_resident([0, 1, 2, 3])
    p.resize_cap(6)
    assert p.cap_experts == 6 and p.slot_to_expert[4:] == [-1, -1]
    ev = p.stats_evict
    p.ensure_resident([4, 5])
    assert p.stats_evict == ev
    p.resize_cap(2)
    assert p.cap_experts == 2 and len(p.lru_tick) == 2
    _consistent(p)
    p.resize_cap(1)
    assert p.cap_experts == 2
    p.resize_cap(999)
    assert p.cap_experts == 8
