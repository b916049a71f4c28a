"""Shared helpers of the test suite."""
from __future__ import annotations

import ctypes as C

import numpy as np

from wisp_amd import _lib
from wisp_amd.record import parse_record


class HostPager:
    """Drives ``wisp_pager_decide_host`` (the C++ specification of the GPU
    pager) with host-side state arrays."""

    def __init__(self, E: int, cap: int) -> None:
        self.E, self.cap = E, cap
        self.map = np.full(E, -1, dtype=np.int32)
        self.s2e = np.full(cap, -1, dtype=np.int32)
        self.tick = np.zeros(cap, dtype=np.int64)
        self.ctr = np.zeros(8, dtype=np.int64)

    def call(self, ids, single_group: bool = False, K: int | None = None):
        """``ids``: [T][K] routed ids of one layer call (or a flat list of
        needed experts with single_group=True)."""
        if single_group:
            ids = np.asarray(ids, dtype=np.int32).reshape(-1, 1)
        else:
            K = K if K is not None else (len(ids[0]) if len(ids) else 1)
            ids = np.asarray(ids, dtype=np.int32).reshape(len(ids), K)
        ids = np.ascontiguousarray(ids)
        T, K = ids.shape
        words = _lib.lib().wisp_record_words(T, K)
        rec = np.zeros(words, dtype=np.int32)
        slots = np.full(max(1, T * K), -7, dtype=np.int32)
        rc = _lib.lib().wisp_pager_decide_host(
            ids.ctypes.data if ids.size else None, T, K, self.E, self.cap, int(single_group),
            self.map.ctypes.data, self.s2e.ctypes.data, self.tick.ctypes.data,
            self.ctr.ctypes.data, slots.ctypes.data, rec.ctypes.data, words)
        out = parse_record(rec, T, K)
        out["rc"] = rc
        out["slots"] = slots[: T * K].reshape(T, K).tolist() if T * K else []
        return out

    @property
    def clock(self):
        return int(self.ctr[0])


def oracle_trace_matches(ora_res: dict, rec: dict) -> None:
    """Assert a parsed record equals the oracle's forward() result."""
    assert [g["tokens"] for g in rec["groups"]] == [tuple(g) for g in ora_res["groups"]]
    for g, o in zip(rec["groups"], ora_res["records"]):
        assert g["n_needed"] == len(o["needed"])
        assert g["hits"] == o["hits"]
        assert g["evicted"] == [tuple(p) for p in o["evicted"]]
        assert g["loaded"] == [tuple(p) for p in o["loaded"]]


def load_golden(name: str) -> dict:
    import gzip
    import json
    import os
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", name)
    with gzip.open(path, "rt") as f:
        return json.load(f)


def fixture_matches(entry: dict, rec: dict, s2e, tick, clock) -> None:
    """Assert a parsed decision record plus the pager state after the call
    equal one fixture trace entry."""
    assert [list(g["tokens"]) for g in rec["groups"]] == entry["groups"]
    for g, r in zip(rec["groups"], entry["records"]):
        assert g["n_needed"] == r["n"] and g["hits"] == r["hits"]
        assert [list(p) for p in g["evicted"]] == r["evicted"]
        assert [list(p) for p in g["loaded"]] == r["loaded"]
    assert list(s2e) == entry["s2e"] and list(tick) == entry["tick"] and clock == entry["clock"]
