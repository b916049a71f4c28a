"""Live scratch resize and the process-wide registry helpers the MV-WSA
controller drives (reference fused_moe.py:439-490, 537-593): pager decisions
across resizes bit-exact with the oracle, outputs byte-identical to
resident, and the helpers' sums, clamps and resets."""
import random

import pytest
import torch

from oracle.moe import route
from oracle.pager import PagerOracle
from wisp_amd import workloads as W
from wisp.integrations.vllm import fused_moe as fm

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


@pytest.fixture(scope="module")
def toy():
    return W.toy(steps=48, pin=True)


def _check(st, ora, t):
    assert st.slot_to_expert == ora.slot_to_expert, t
    assert st.lru_tick == ora.lru_tick and st.lru_clock == ora.lru_clock, t
    assert (st.stats_miss, st.stats_hits, st.stats_evict, st.stats_forward) == \
        (ora.stats_miss, ora.stats_hits, ora.stats_evict, ora.stats_forward), t


def test_resize_trace_matches_oracle_and_resident(toy):
    w13, w2 = toy.views()
    E, K = toy.shape.experts, toy.shape.top_k
    st = fm.WispMoEState(w13, w2, 4, "paged", DEV, 0)
    res = fm.WispMoEState(w13, w2, E, "resident", DEV, 1)
    res.prime_identity()
    ora = PagerOracle(E, 4)
    plan = {6: 7, 12: 2, 18: 2, 24: 1, 30: 999, 36: 5}   # grow, shrink, no-op, clamps
    for t in range(toy.steps):
        if t in plan:
            torch.cuda.synchronize()
            st.resize_cap(plan[t])
            ora.resize_cap(plan[t])
            assert st.cap_experts == ora.cap_experts
            assert len(st.slot_to_expert) == st.cap_experts == len(st.lru_tick)
            emap = st.expert_map_device.tolist()
            for e in range(E):  # the map agrees with the slot table after a resize
                assert emap[e] == st.expert_to_slot.get(e, -1), (t, e)
        x, lg = toy.x[t].to(DEV), toy.logits[t].to(DEV)
        out = st.forward(x, lg, K, True)
        ref = res.forward(x, lg, K, True)
        ora.forward(route(toy.logits[t], K)[1].tolist())
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int32), ref.view(torch.int32)), t
        _check(st, ora, t)
    assert st.cap_experts == 5


def test_registry_helpers(monkeypatch, toy):
    w13, w2 = toy.views()
    E, K, H, I = toy.shape.experts, toy.shape.top_k, toy.shape.hidden, toy.shape.inter
    monkeypatch.setattr(fm, "_LAYER_STATES", [])
    assert fm.num_registered_layers() == 0 and fm.current_layer_cap() is None
    assert fm.num_experts_per_layer() is None and fm.resize_layer_caps(6) == 0
    assert fm.expert_bytes_per_cap() == 0
    assert fm.snapshot_expert_stats() == {"miss": 0, "hit": 0, "forward": 0, "ws": 0}

    states = [fm.WispMoEState(w13, w2, 4, "paged", DEV, L) for L in range(3)]
    oras = [PagerOracle(E, 4) for _ in range(3)]
    monkeypatch.setattr(fm, "_LAYER_STATES", states)
    assert fm.num_registered_layers() == 3 and fm.current_layer_cap() == 4
    assert fm.num_experts_per_layer() == E
    assert fm.expert_bytes_per_cap() == 3 * 3 * I * H * 4  # fp32 w13 + w2 of one slot

    rng = random.Random(0)
    last_sets = []
    for t in range(10):
        for L, (st, ora) in enumerate(zip(states, oras)):
            s = rng.randrange(toy.steps)
            st.forward(toy.x[s].to(DEV), toy.logits[s].to(DEV), K, True)
            ids = route(toy.logits[s], K)[1].tolist()
            ora.forward(ids)
            if t == 9:
                last_sets.append(len({e for row in ids for e in row}))
    torch.cuda.synchronize()
    snap = fm.snapshot_expert_stats(reset=False)
    assert snap == {"miss": sum(o.stats_miss for o in oras), "hit": sum(o.stats_hits for o in oras),
                    "forward": sum(o.stats_forward for o in oras), "ws": max(last_sets)}
    snap2 = fm.snapshot_expert_stats()          # reset=True by default
    assert snap2 == snap
    assert fm.snapshot_expert_stats() == {"miss": 0, "hit": 0, "forward": 0, "ws": max(last_sets)}
    # evictions and the LRU clock are not telemetry: they survive the reset
    assert [st.stats_evict for st in states] == [o.stats_evict for o in oras]

    assert fm.resize_layer_caps(6) == 3
    for o in oras:
        o.resize_cap(6)
    assert fm.current_layer_cap() == 6 and all(st.cap_experts == 6 for st in states)
    assert fm.expert_bytes_per_cap() == 3 * 3 * I * H * 4  # per slot, independent of cap
    for st, o in zip(states, oras):
        st.forward(toy.x[0].to(DEV), toy.logits[0].to(DEV), K, True)
        o.forward(route(toy.logits[0], K)[1].tolist())
        torch.cuda.synchronize()
        assert st.slot_to_expert == o.slot_to_expert and st.lru_tick == o.lru_tick
    assert fm.resize_layer_caps(1) == 3 and fm.current_layer_cap() == 2
