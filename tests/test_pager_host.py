"""The C++ pager (wisp_pager_decide_host, the specification the GPU kernel
is tested against) and its CPython set-order emulation, checked against the
oracle and live CPython sets on the CPU."""
import random

import numpy as np
import pytest

from oracle.pager import PagerOracle, PagerOverflow
from tests._util import HostPager, oracle_trace_matches
from wisp_amd import _lib


def test_set_order_matches_live_cpython(hiplib):
    rng = random.Random(1)
    cases = [[2, 9], [3, 11], [1, 9], [5, 37, 69, 101, 6, 7, 8, 9], list(range(128))]
    for E in (8, 16, 128, 512):
        for _ in range(400):
            n = rng.randint(0, min(E, 80 if rng.random() < 0.8 else E))
            cases.append(sorted(rng.sample(range(E), n)))
    for keys in cases:
        k = np.asarray(sorted(keys), dtype=np.int32)
        out = np.zeros(max(1, len(k)), dtype=np.int32)
        n = hiplib.wisp_cpython_set_order(k.ctypes.data if len(k) else None, len(k),
                                          out.ctypes.data)
        assert n == len(k)
        assert out[:n].tolist() == list(set(int(e) for e in k)), keys


def test_subbatch_plan_matches_oracle(hiplib):
    from oracle.pager import plan_groups
    rng = np.random.default_rng(2)
    for _ in range(200):
        E, K = int(rng.integers(4, 64)), int(rng.integers(1, 5))
        K = min(K, E)
        cap = int(rng.integers(K, E + 1))
        T = int(rng.integers(1, 40))
        ids = np.stack([rng.choice(E, K, replace=False) for _ in range(T)]).astype(np.int32)
        ends = np.zeros(T + 1, dtype=np.int32)
        ng = hiplib.wisp_subbatch_plan(ids.ctypes.data, T, K, cap, ends.ctypes.data)
        want = plan_groups(ids.tolist(), cap)
        assert ends[:ng].tolist() == [e for _, e in want]


def _random_calls(rng, E, K, cap, steps, tmax):
    for _ in range(steps):
        T = int(rng.integers(0, tmax + 1))
        yield [rng.choice(E, K, replace=False).tolist() for _ in range(T)]


@pytest.mark.parametrize("E,K,cap,tmax", [(8, 2, 4, 3), (16, 2, 4, 4), (128, 8, 8, 1),
                                           (128, 8, 24, 6), (128, 8, 32, 40), (8, 2, 2, 16),
                                           (512, 8, 64, 8), (256, 8, 100, 20), (512, 16, 300, 40)])
def test_host_pager_matches_oracle(E, K, cap, tmax):
    rng = np.random.default_rng(E * 1000 + cap)
    ora, hp = PagerOracle(E, cap), HostPager(E, cap)
    for ids in _random_calls(rng, E, K, cap, 120, tmax):
        res = ora.forward(ids)
        rec = hp.call(ids, K=K)
        assert rec["rc"] == 0 and rec["status"] == 0
        oracle_trace_matches(res, rec)
        assert rec["slots"] == res["slots"]
        assert hp.s2e.tolist() == ora.slot_to_expert
        assert hp.tick.tolist() == ora.lru_tick
        assert hp.map.tolist() == ora.expert_map()
        assert hp.ctr[:5].tolist() == [ora.lru_clock, ora.stats_forward, ora.stats_miss,
                                       ora.stats_evict, ora.stats_hits]


def test_host_pager_single_group_and_overflow():
    ora, hp = PagerOracle(8, 4), HostPager(8, 4)
    for need in ([0, 1], [2, 3], [4], [1, 1, 4], [5, 6, 7, 0]):
        ora.ensure_resident(need)
        rec = hp.call(need, single_group=True)
        assert rec["rc"] == 0
        assert hp.s2e.tolist() == ora.slot_to_expert and hp.tick.tolist() == ora.lru_tick
    assert hp.ctr[1] == 0   # ensure_resident does not count layer calls
    with pytest.raises(PagerOverflow):
        ora.ensure_resident([0, 1, 2, 3, 4])
    rec = hp.call([0, 1, 2, 3, 4], single_group=True)
    assert rec["rc"] == _lib.WISP_ERR_SUBBATCH and rec["fail_group"] == 0
    assert rec["fail_unique"] == 5
    assert hp.ctr[4] == ora.stats_hits and hp.s2e.tolist() == ora.slot_to_expert


def test_host_pager_overflow_mid_call_keeps_earlier_groups():
    # token 1 routes to 3 experts with cap 2: group 0 completes, group 1 fails
    ora, hp = PagerOracle(8, 2), HostPager(8, 2)
    ids = [[0, 1, 1], [2, 3, 4]]
    with pytest.raises(PagerOverflow):
        ora.forward(ids)
    rec = hp.call(ids)
    assert rec["rc"] == _lib.WISP_ERR_SUBBATCH and rec["fail_group"] == 1
    assert len(rec["groups"]) == 1
    assert hp.s2e.tolist() == ora.slot_to_expert and hp.ctr[4] == ora.stats_hits


def test_host_pager_rejects_bad_ids():
    hp = HostPager(8, 4)
    rec = hp.call([[0, 9]])
    assert rec["rc"] == _lib.WISP_ERR_INVALID
