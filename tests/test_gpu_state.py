"""WispMoEState on the GPU: the reference's own state tests
(tests/test_wisp_state.py) restated against this implementation, plus
decision traces checked against the oracle."""
import pytest
import torch

from oracle.pager import PagerOracle
from wisp.integrations.vllm.fused_moe import WispMoEState

pytestmark = pytest.mark.gpu

E, CAP, DEV = 8, 4, "cuda:0"


def make_state(cap: int = CAP, mode: str = "paged") -> WispMoEState:
    # every expert filled with its own id so content checks are exact
    w13 = torch.empty((E, 4, 2), dtype=torch.float32)
    w2 = torch.empty((E, 2, 4), dtype=torch.float32)
    for e in range(E):
        w13[e].fill_(float(e))
        w2[e].fill_(float(e))
    return WispMoEState(w13.pin_memory(), w2.pin_memory(), cap, mode, torch.device(DEV), 0)


def need(st, experts):
    st.ensure_resident(torch.tensor(experts, dtype=torch.long, device=DEV))


def emap(st):
    torch.cuda.synchronize()
    return st.expert_map_device.cpu().tolist()


def assert_consistent(st):
    torch.cuda.synchronize()
    m = emap(st)
    s2e = st.slot_to_expert
    e2s = st.expert_to_slot
    for e, s in e2s.items():
        assert s2e[s] == e and m[e] == s
        assert torch.all(st.scratch_w13[s].cpu() == float(e)), (e, s)
        assert torch.all(st.scratch_w2[s].cpu() == float(e)), (e, s)
    for e in range(st.num_experts):
        if e not in e2s:
            assert m[e] == -1


def test_miss_then_hit():
    st = make_state()
    need(st, [0, 1])
    assert st.stats_miss == 2 and st.stats_hits == 0
    assert_consistent(st)
    need(st, [0, 1])
    assert st.stats_miss == 2 and st.stats_hits == 2 and st.stats_evict == 0
    assert_consistent(st)


def test_lru_eviction_order_exact():
    st = make_state()
    need(st, [0, 1])
    need(st, [2, 3])
    need(st, [4])
    # exact victim and slot, as derived from the reference source
    assert st.slot_to_expert == [3, 2, 4, 0] and st.lru_tick == [2, 2, 3, 1]
    assert st.stats_evict == 1
    assert_consistent(st)


def test_needed_set_never_evicted():
    st = make_state()
    need(st, [0, 1, 2, 3])
    need(st, [0, 1, 4])
    e2s = st.expert_to_slot
    assert 0 in e2s and 1 in e2s and 4 in e2s
    assert (2 in e2s) != (3 in e2s)
    assert_consistent(st)


def test_working_set_overflow_raises():
    st = make_state()
    with pytest.raises(RuntimeError, match="sub-batch"):
        need(st, [0, 1, 2, 3, 4])


def test_map_consistency_random_walk_matches_oracle():
    torch.manual_seed(0)
    st, ora = make_state(), PagerOracle(E, CAP)
    for _ in range(50):
        k = int(torch.randint(1, CAP + 1, ()).item())
        experts = torch.randperm(E)[:k].tolist()
        need(st, experts)
        ora.ensure_resident(experts)
        assert st.slot_to_expert == ora.slot_to_expert
        assert st.lru_tick == ora.lru_tick
    assert_consistent(st)


def test_resize_grow_preserves_residents():
    st = make_state()
    need(st, [0, 1, 2, 3])
    st.resize_cap(6)
    assert st.cap_experts == 6 and len(st.slot_to_expert) == 6 and len(st.lru_tick) == 6
    assert st.slot_to_expert[4] == -1 and st.slot_to_expert[5] == -1
    assert_consistent(st)
    before = st.stats_evict
    need(st, [4, 5])
    assert st.stats_evict == before
    assert_consistent(st)


def test_resize_shrink_drops_tail_and_repages():
    st = make_state()
    need(st, [0, 1, 2, 3])
    tail = [e for e in st.slot_to_expert[2:] if e != -1]
    st.resize_cap(2)
    assert st.cap_experts == 2 and len(st.slot_to_expert) == 2
    m = emap(st)
    for e in tail:
        assert e not in st.expert_to_slot and m[e] == -1
    assert_consistent(st)
    need(st, [tail[0]])
    assert tail[0] in st.expert_to_slot
    assert_consistent(st)


def test_resize_noop_and_clamps():
    st = make_state()
    need(st, [0, 1])
    st.resize_cap(CAP)
    assert st.cap_experts == CAP
    st.resize_cap(1)
    assert st.cap_experts == 2
    st.resize_cap(999)
    assert st.cap_experts == E
    assert_consistent(st)


def test_prime_identity_resident_mode():
    st = make_state(cap=E, mode="resident")
    st.prime_identity()
    torch.cuda.synchronize()
    assert emap(st) == list(range(E))
    assert_consistent(st)
