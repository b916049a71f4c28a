"""Oracle: restatement of the reference expert pager — TEST INFRASTRUCTURE ONLY.

Follows ``src/wisp/integrations/vllm/fused_moe.py`` of the reference:

* ``PagerOracle.ensure_resident``  <- ``WispMoEState.ensure_resident`` (264-358)
* ``PagerOracle.prime_identity``   <- ``WispMoEState.prime_identity`` (242-258)
* ``PagerOracle.resize_cap``       <- ``WispMoEState.resize_cap`` (439-490)
* ``PagerOracle.prefetch_async``   <- ``WispMoEState.prefetch_async`` (360-433)
* ``plan_groups``                  <- greedy first-fit sub-batching (1119-1140)
* ``PagerOracle.forward``          <- working-set check + fast path / sub-batch
                                      loop of ``_wisp_forward_cuda_paged``
                                      (1017, 1102-1168)

Only the bookkeeping is restated (no tensors, no copies): every call returns a
trace record ``{needed, hits, evicted, loaded, clock, slot_to_expert, lru_tick}``
with ``evicted`` / ``loaded`` as ``(expert, slot)`` pairs in issue order.

Set order.  ``missing`` is formed by iterating a CPython ``set`` built from the
ascending unique ids (fused_moe.py:279-283); this module runs on CPython, so it
gets that order natively.  The library's C++ emulation of that order is checked
against live ``set()`` in the tests.

Pinning.  ``ensure_resident`` / ``plan_groups`` / ``forward`` are pinned by the
hand-derived known-answer traces in ``tests/test_oracle_pager.py`` (worked
from the reference source text, not by running this module) and by the
invariants asserted in the reference's ``tests/test_wisp_state.py`` (three
residency views agree, needed never evicted, overflow raises "sub-batch",
hit/miss/evict counters).  ``resize_cap`` is pinned by the reference's resize
tests (``tests/test_wisp_state.py:124-167``).
"""
from __future__ import annotations

from typing import Iterable, Sequence

SUBBATCH_MSG = (
    "wisp: per-kernel-call working set ({u} unique experts) exceeds "
    "cap_experts ({cap}); the forward path must sub-batch"
)


class PagerOverflow(RuntimeError):
    """Raised where the reference raises its "sub-batch" RuntimeError
    (fused_moe.py:315-327)."""


class PagerOracle:
    """Host-side LRU pager state for one MoE layer (fused_moe.py:161-236)."""

    def __init__(self, num_experts: int, cap_experts: int) -> None:
        self.num_experts = int(num_experts)
        self.cap_experts = int(cap_experts)
        self.slot_to_expert: list[int] = [-1] * self.cap_experts
        self.expert_to_slot: dict[int, int] = {}
        self.lru_tick: list[int] = [0] * self.cap_experts
        self.lru_clock = 0
        self.stats_forward = 0
        self.stats_miss = 0
        self.stats_evict = 0
        self.stats_hits = 0
        # post-forward bookkeeping (fused_moe.py:1173-1177) and prefetch count
        self.last_unique_experts: set[int] = set()
        self.stats_pred_total = 0

    # -- expert_map_device view (fused_moe.py:196-204, 333, 353) -----------
    def expert_map(self) -> list[int]:
        m = [-1] * self.num_experts
        for e, s in self.expert_to_slot.items():
            m[e] = s
        return m

    def snapshot(self) -> dict:
        return {
            "clock": self.lru_clock,
            "slot_to_expert": list(self.slot_to_expert),
            "lru_tick": list(self.lru_tick),
        }

    # -- fused_moe.py:242-258 ---------------------------------------------
    def prime_identity(self) -> None:
        assert self.cap_experts == self.num_experts
        for i in range(self.num_experts):
            self.slot_to_expert[i] = i
            self.expert_to_slot[i] = i

    # -- fused_moe.py:264-358 ---------------------------------------------
    def ensure_resident(self, ids: Iterable[int]) -> dict:
        needed = sorted({int(e) for e in ids})      # torch.unique: sorted
        needed_set = set(int(e) for e in needed)     # inserted ascending
        missing = [e for e in needed_set if e not in self.expert_to_slot]
        hits = len(needed_set) - len(missing)
        self.stats_hits += hits
        rec = {"needed": needed, "hits": hits, "evicted": [], "loaded": []}
        if not missing:
            self.lru_clock += 1
            for e in needed_set:
                self.lru_tick[self.expert_to_slot[e]] = self.lru_clock
            rec.update(self.snapshot())
            return rec

        free_slots = [s for s in range(self.cap_experts) if self.slot_to_expert[s] == -1]
        candidates = sorted(
            (
                (self.lru_tick[s], s)
                for s in range(self.cap_experts)
                if self.slot_to_expert[s] != -1 and self.slot_to_expert[s] not in needed_set
            ),
            key=lambda ts: ts[0],
        )
        shortfall = len(missing) - len(free_slots)
        if shortfall > 0:
            if shortfall > len(candidates):
                raise PagerOverflow(SUBBATCH_MSG.format(u=len(needed_set), cap=self.cap_experts))
            for _tick, s in candidates[:shortfall]:
                victim = self.slot_to_expert[s]
                self.expert_to_slot.pop(victim, None)
                self.slot_to_expert[s] = -1
                free_slots.append(s)
                self.stats_evict += 1
                rec["evicted"].append((victim, s))

        self.lru_clock += 1
        for e in missing:
            s = free_slots.pop()
            self.slot_to_expert[s] = e
            self.expert_to_slot[e] = s
            self.lru_tick[s] = self.lru_clock
            self.stats_miss += 1
            rec["loaded"].append((e, s))
        for e in needed_set:
            self.lru_tick[self.expert_to_slot[e]] = self.lru_clock
        rec.update(self.snapshot())
        return rec

    # -- fused_moe.py:360-433 ---------------------------------------------
    def prefetch_async(self, predicted_experts: set) -> dict:
        """Speculative load of ``predicted_experts`` (a set; its iteration
        order fixes which slot each expert takes).  Evicts by LRU tick among
        slots whose expert is neither in ``last_unique_experts`` nor
        predicted; loads what fits; bumps the clock once if anything was
        missing.  Returns ``{"evicted": [(e, s)], "loaded": [(e, s)]}``."""
        rec = {"evicted": [], "loaded": []}
        if not predicted_experts:
            return rec
        to_load = [e for e in predicted_experts if e not in self.expert_to_slot]
        if not to_load:
            return rec
        free_slots = [s for s in range(self.cap_experts) if self.slot_to_expert[s] == -1]
        candidates = sorted(
            (
                (self.lru_tick[s], s)
                for s in range(self.cap_experts)
                if self.slot_to_expert[s] != -1
                and self.slot_to_expert[s] not in self.last_unique_experts
                and self.slot_to_expert[s] not in predicted_experts
            ),
            key=lambda ts: ts[0],
        )
        need = len(to_load) - len(free_slots)
        if need > 0:
            if need > len(candidates):
                # speculative: load only what fits (first in set order)
                to_load = to_load[: len(candidates) + len(free_slots)]
                need = len(to_load) - len(free_slots)
            for _tick, s in candidates[:need]:
                victim = self.slot_to_expert[s]
                self.expert_to_slot.pop(victim, None)
                self.slot_to_expert[s] = -1
                free_slots.append(s)
                self.stats_evict += 1
                rec["evicted"].append((victim, s))
        self.lru_clock += 1
        for e in to_load:
            if not free_slots:
                break
            s = free_slots.pop()
            self.slot_to_expert[s] = int(e)
            self.expert_to_slot[int(e)] = s
            self.lru_tick[s] = self.lru_clock
            rec["loaded"].append((int(e), s))
        return rec

    # -- fused_moe.py:439-490 ---------------------------------------------
    def resize_cap(self, new_cap: int) -> None:
        new_cap = max(2, min(int(new_cap), self.num_experts))
        old_cap = self.cap_experts
        if new_cap == old_cap:
            return
        if new_cap < old_cap:
            for s in range(new_cap, old_cap):
                e = self.slot_to_expert[s]
                if e != -1:
                    self.expert_to_slot.pop(e, None)
            del self.slot_to_expert[new_cap:]
            del self.lru_tick[new_cap:]
        else:
            self.slot_to_expert.extend([-1] * (new_cap - old_cap))
            self.lru_tick.extend([0] * (new_cap - old_cap))
        self.cap_experts = new_cap

    # -- fused_moe.py:1017, 1102-1168 -------------------------------------
    def forward(self, topk_ids: Sequence[Sequence[int]]) -> dict:
        """One paged layer call: returns ``{"groups": [[t0, t1), ...],
        "records": [...]}`` (one record per ``ensure_resident`` call) and the
        per-(token, k) slot each routed expert was read from."""
        self.stats_forward += 1
        ids = [[int(e) for e in row] for row in topk_ids]
        groups = plan_groups(ids, self.cap_experts)
        records, slots = [], []
        for (t0, t1) in groups:
            rec = self.ensure_resident(e for row in ids[t0:t1] for e in row)
            records.append(rec)
            for row in ids[t0:t1]:
                slots.append([self.expert_to_slot[e] for e in row])
        # post-forward (fused_moe.py:1173-1177): built from the sorted unique ids
        self.last_unique_experts = {int(e) for e in sorted({e for row in ids for e in row})}
        return {"groups": groups, "records": records, "slots": slots}


def plan_groups(topk_ids: Sequence[Sequence[int]], cap: int) -> list[tuple[int, int]]:
    """Greedy first-fit over tokens in index order (fused_moe.py:1102, 1124-1140).

    A token joins the open group iff the union stays within ``cap`` or the
    group is empty; groups are therefore contiguous token ranges, returned
    as ``(start, end)``.  When the whole batch's union fits (the reference's
    fast path at 1103-1118) this yields one group, which is the same call."""
    T = len(topk_ids)
    if len({int(e) for row in topk_ids for e in row}) <= cap:
        # includes T == 0: the reference still makes one (empty) call, which
        # advances the LRU clock (fused_moe.py:1102-1105, 285-289)
        return [(0, T)]
    groups: list[tuple[int, int]] = []
    start, cur = 0, set()
    for t in range(T):
        tok = {int(e) for e in topk_ids[t]}
        merged = cur | tok
        if len(merged) <= cap or t == start:
            cur = merged
        else:
            groups.append((start, t))
            start, cur = t, tok
    groups.append((start, T))
    return groups
