"""Pins the co-occurrence / prefetch oracle (oracle/cooccur.py,
PagerOracle.prefetch_async) with known answers derived by hand from the
reference source text, closed forms and an exact-arithmetic re-derivation."""
import random
from fractions import Fraction

import pytest

from oracle.cooccur import CooccurOracle, predict_layer, prefetch_glue
from oracle.pager import PagerOracle


def _table(steps):
    t = CooccurOracle()
    for st in steps:
        t.observe_step(st)
    return t


def test_observe_step_counts_forward_pairs_and_marginals():
    t = _table([{0: [1, 2], 1: [3], 2: [1]}])
    assert dict(t.layer_total) == {(0, 1): 1, (0, 2): 1, (1, 3): 1, (2, 1): 1}
    got = {(Ls, es, Ld, ed): n for (Ls, es), per in t.count.items()
           for Ld, row in per.items() for ed, n in row.items()}
    # only L_dst > L_src, every pair once
    assert got == {(0, 1, 1, 3): 1, (0, 2, 1, 3): 1, (0, 1, 2, 1): 1, (0, 2, 2, 1): 1,
                   (1, 3, 2, 1): 1}
    assert t.num_steps_observed == 1


def test_observe_step_pair_count_closed_form():
    rng = random.Random(3)
    for _ in range(20):
        step = {L: rng.sample(range(16), rng.randint(0, 5)) for L in range(6)}
        t = _table([step])
        n_pairs = sum(n for per in t.count.values() for row in per.values() for n in row.values())
        sizes = [len(step[L]) for L in range(6)]
        assert n_pairs == sum(sizes[a] * sizes[b] for a in range(6) for b in range(a + 1, 6))
        assert sum(t.layer_total.values()) == sum(sizes)


def test_predict_known_answer_normalised():
    # step A: layer0 {1}, layer1 {5, 6};  step B: layer0 {1, 2}, layer1 {6}
    t = _table([{0: [1], 1: [5, 6]}, {0: [1, 2], 1: [6]}])
    # P(6 | 1) = 2/2, P(5 | 1) = 1/2 ; from expert 2: P(6 | 2) = 1/1
    assert predict_layer(t, {0: {1}}, 1, k=8, normalize=True) == [6, 5]
    assert predict_layer(t, {0: {2}}, 1, k=8, normalize=True) == [6]
    # seen {1, 2}: 6 -> 1 + 1 = 2, 5 -> 0.5
    assert predict_layer(t, {0: {1, 2}}, 1, k=1) == [6]
    # without normalisation: raw counts 6 -> 2 + 1, 5 -> 1
    assert predict_layer(t, {0: {1, 2}}, 1, k=8, normalize=False) == [6, 5]


def test_predict_decay_and_only_prev_layer():
    # layer0 expert 0 points to 7 at layer 2; layer1 expert 3 points to 8 at layer 2
    t = _table([{0: [0], 1: [3], 2: [7]}, {1: [3], 2: [8]}, {1: [3], 2: [8]}])
    seen = {0: {0}, 1: {3}}
    # P(7|0@0) = 1 (weight decay^1), P(8|3@1) = 2/3, P(7|3@1) = 1/3 (weight 1)
    # decay 1.0: 7 -> 1 + 1/3, 8 -> 2/3
    assert predict_layer(t, seen, 2, decay=1.0) == [7, 8]
    # decay 0.25: 7 -> 0.25 + 1/3, 8 -> 2/3 ; 0.5833 < 0.6667
    assert predict_layer(t, seen, 2, decay=0.25) == [8, 7]
    assert predict_layer(t, seen, 2, only_prev_layer=True) == [8, 7]
    # sources at or above the target are ignored
    assert predict_layer(t, {2: {7}}, 2) == []


def test_predict_ties_go_to_lower_id_and_cold_is_empty():
    t = _table([{0: [4], 1: [9, 2, 5]}])
    assert predict_layer(t, {0: {4}}, 1, k=3) == [2, 5, 9]
    assert predict_layer(t, {0: {4}}, 1, k=2) == [2, 5]
    assert predict_layer(CooccurOracle(), {0: {4}}, 1) == []
    assert predict_layer(t, {0: {11}}, 1) == []


def test_scores_match_exact_rational_rederivation():
    rng = random.Random(7)
    steps = [{L: rng.sample(range(24), rng.randint(1, 6)) for L in range(5)} for _ in range(40)]
    t = _table(steps)
    for _ in range(50):
        seen = {L: set(rng.sample(range(24), rng.randint(1, 5))) for L in range(3)}
        target = rng.randint(1, 4)
        dec = rng.choice([1.0, 0.5, 0.25])
        # independent: exact rationals, destination-major
        exact = {}
        for ed in range(24):
            v, hit = Fraction(0), False
            for Ls, src in seen.items():
                if Ls >= target:
                    continue
                for es in src:
                    c = t.count.get((Ls, es), {}).get(target, {}).get(ed, 0)
                    if c:
                        v += Fraction(dec) ** (target - Ls - 1) * c / t.layer_total[(Ls, es)]
                        hit = True
            if hit:
                exact[ed] = v
        want = [e for e, _ in sorted(exact.items(), key=lambda x: (-x[1], x[0]))][:6]
        got = predict_layer(t, seen, target, k=6, decay=dec)
        # identical unless two exact scores are within float rounding of each other
        if got != want:
            vals = sorted(exact.values(), reverse=True)
            assert any(abs(float(a - b)) < 1e-12 for a, b in zip(vals, vals[1:]))


def test_json_round_trip():
    rng = random.Random(1)
    t = _table([{L: rng.sample(range(10), 3) for L in range(4)} for _ in range(5)])
    u = CooccurOracle.from_dict(t.to_dict())
    assert u.to_dict() == t.to_dict()
    assert u.num_steps_observed == 5
    with pytest.raises(ValueError):
        CooccurOracle.from_dict({"schema_version": 2})


def _state(cap, slots, ticks, clock, last):
    p = PagerOracle(32, cap)
    p.slot_to_expert = list(slots)
    p.expert_to_slot = {e: s for s, e in enumerate(slots) if e != -1}
    p.lru_tick = list(ticks)
    p.lru_clock = clock
    p.last_unique_experts = set(last)
    return p


def test_prefetch_loads_into_free_slots_in_set_order():
    p = _state(4, [10, 11, -1, -1], [1, 2, 0, 0], 2, {10})
    rec = p.prefetch_async({11, 12, 13})
    # set {11, 12, 13} iterates 11, 12, 13; 11 resident; free [2, 3] popped from the end
    assert rec == {"evicted": [], "loaded": [(12, 3), (13, 2)]}
    assert p.slot_to_expert == [10, 11, 13, 12] and p.lru_clock == 3
    assert p.lru_tick == [1, 2, 3, 3] and p.stats_evict == 0 and p.stats_miss == 0


def test_prefetch_evicts_lru_outside_history_and_prediction_and_truncates():
    p = _state(3, [10, 11, 14], [1, 2, 3], 3, {11})
    rec = p.prefetch_async({12, 13, 14})
    # candidates: slot 0 only (11 is history, 14 predicted); need 2 > 1 -> load only 12
    assert rec == {"evicted": [(10, 0)], "loaded": [(12, 0)]}
    assert p.slot_to_expert == [12, 11, 14] and p.lru_tick == [4, 2, 3]
    assert p.stats_evict == 1 and p.lru_clock == 4


def test_prefetch_noops():
    p = _state(2, [5, 6], [1, 1], 1, set())
    assert p.prefetch_async(set()) == {"evicted": [], "loaded": []}
    assert p.prefetch_async({5, 6}) == {"evicted": [], "loaded": []}
    assert p.lru_clock == 1
    # nothing can be evicted or placed: the clock still advances once
    q = _state(2, [5, 6], [1, 1], 1, {5, 6})
    assert q.prefetch_async({7}) == {"evicted": [], "loaded": []}
    assert q.lru_clock == 2


def test_prefetch_uses_set_iteration_order_for_slots():
    # {9, 2} in an 8-slot CPython table: 9 & 7 = 1 and 2 & 7 = 2, so it iterates 9 then 2
    p = _state(3, [-1, -1, -1], [0, 0, 0], 0, set())
    rec = p.prefetch_async(set([2, 9]))
    assert [e for e, _ in rec["loaded"]] == list({2, 9}) == [9, 2]


def test_prefetch_glue_steps_through_layers():
    # layer0 always {1,2} -> layer1 always {3,4}: after one learned step the
    # glue prefetches 3 and 4 (equal scores, ascending) into layer 1
    states = [PagerOracle(8, 4), PagerOracle(8, 4)]
    table, obs = CooccurOracle(), {}
    for step in range(2):
        states[0].forward([[1, 2]])
        pred = prefetch_glue(states, 0, table, obs, online=True)
        assert pred == ([] if step == 0 else [3, 4])
        if step == 1:
            assert states[1].last_unique_experts == {3, 4}
        states[1].forward([[3, 4]])
        prefetch_glue(states, 1, table, obs, online=True)
        assert obs == {}
    assert table.num_steps_observed == 2
    # step 1's prefetch found both experts already resident (the forward of
    # step 0 loaded them): counted as predicted, nothing loaded
    assert states[1].stats_pred_total == 2 and states[1].stats_evict == 0
