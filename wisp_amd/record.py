"""Decoding of the pager's decision record (layout in wisp_amd/csrc/pager_core.h).

A record is one int32 array per layer call: an 8-word header, one 8-word
entry per token group, then the evicted and the loaded (expert, slot) pairs
in issue order.  ``parse_record`` turns it into the per-call trace the
reference's pager would produce: for every ``ensure_resident`` call its
token range, unique-expert count, hits, evictions and loads.
"""
from __future__ import annotations

import numpy as np

STATUS, GROUPS_DONE, GROUPS_PLANNED, FAIL_GROUP, FAIL_UNIQUE, N_EVICTED, N_LOADED = range(7)


def layout(T: int, K: int) -> tuple[int, int, int]:
    max_groups = T if T > 0 else 1
    max_pairs = T * K if T * K > 0 else 1
    ev_base = 8 + 8 * max_groups
    ld_base = ev_base + 2 * max_pairs
    return max_groups, ev_base, ld_base


def parse_record(rec, T: int, K: int) -> dict:
    r = np.asarray(rec, dtype=np.int64)
    _, ev_base, ld_base = layout(T, K)
    groups = []
    for g in range(int(r[GROUPS_DONE])):
        t0, t1, n_needed, hits, ev_off, n_ev, ld_off, n_ld = (int(v) for v in r[8 + 8 * g: 16 + 8 * g])
        ev = r[ev_base + 2 * ev_off: ev_base + 2 * (ev_off + n_ev)].reshape(-1, 2)
        ld = r[ld_base + 2 * ld_off: ld_base + 2 * (ld_off + n_ld)].reshape(-1, 2)
        groups.append({
            "tokens": (t0, t1), "n_needed": n_needed, "hits": hits,
            "evicted": [tuple(int(v) for v in p) for p in ev],
            "loaded": [tuple(int(v) for v in p) for p in ld],
        })
    return {
        "status": int(r[STATUS]), "groups_planned": int(r[GROUPS_PLANNED]),
        "fail_group": int(r[FAIL_GROUP]), "fail_unique": int(r[FAIL_UNIQUE]),
        "groups": groups,
    }
