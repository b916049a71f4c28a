"""Writes the golden fixtures of this directory from the oracle.

    python tests/golden/make_golden.py

Fixtures (all routing from the seeded generators in wisp_amd/workloads.py):

* ``toy.json.gz`` / ``toy_out.npz`` - fp32 toy layer (H512 I256 E16 k2 cap4),
  64 bs=1 steps: routing ids and weights, the pager trace of every call and
  the float64 oracle output of every step.
* ``qwen3.json.gz`` - Qwen3-shaped layer, 256 bs=1 steps, cap 8: routing ids
  and pager traces.
* ``batch.json.gz`` - 512-token prefill chunk then 8 batch-32 decode steps,
  cap 32: routing ids and pager traces (greedy token groups).
* ``mixtral.json.gz`` - Mixtral-shaped layer, 256 bs=1 steps then 16 bs=16
  steps, cap 4.
* ``stack.json.gz`` - first 32 tokens of the 48-layer stack, cap 24 per layer.

A trace entry per layer call: token groups, per group the unique-expert
count, hits, evicted and loaded (expert, slot) pairs; then the clock, slot
table and LRU ticks after the call.
"""
from __future__ import annotations

import gzip
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle.moe import moe_forward, route  # noqa: E402
from oracle.pager import PagerOracle  # noqa: E402
from wisp_amd import workloads as W  # noqa: E402


def trace_call(pager: PagerOracle, ids) -> dict:
    res = pager.forward(ids)
    return {
        "groups": [list(g) for g in res["groups"]],
        "records": [{"n": len(r["needed"]), "hits": r["hits"],
                     "evicted": [list(p) for p in r["evicted"]],
                     "loaded": [list(p) for p in r["loaded"]]} for r in res["records"]],
        "clock": pager.lru_clock,
        "s2e": list(pager.slot_to_expert),
        "tick": list(pager.lru_tick),
    }


def run_sequence(E, cap, calls):
    pager = PagerOracle(E, cap)
    return [trace_call(pager, ids) for ids in calls], {
        "forward": pager.stats_forward, "miss": pager.stats_miss,
        "evict": pager.stats_evict, "hits": pager.stats_hits}


def routed(logits, k):
    ids_all, w_all = [], []
    for t in range(logits.shape[0]):
        w, ids = route(logits[t], k)
        ids_all.append(ids.tolist())
        w_all.append(w.tolist())
    return ids_all, w_all


def dump(name, obj):
    with gzip.open(os.path.join(HERE, name), "wt") as f:
        json.dump(obj, f, separators=(",", ":"))


def main() -> None:
    # toy fp32 layer
    wl = W.toy()
    sh = wl.shape
    ids, ws = routed(wl.logits, sh.top_k)
    traces, stats = run_sequence(sh.experts, sh.cap, ids)
    dump("toy.json.gz", {"shape": [sh.hidden, sh.inter, sh.experts, sh.top_k, sh.cap],
                         "ids": ids, "weights": ws, "trace": traces, "stats": stats})
    w13, w2 = wl.views()
    outs = np.stack([moe_forward(wl.x[t], np.asarray(ws[t]), np.asarray(ids[t]), w13, w2).numpy()
                     for t in range(wl.steps)])
    np.savez_compressed(os.path.join(HERE, "toy_out.npz"), out=outs)

    # qwen3 decode
    wl = W.qwen3_decode(weights=False)
    ids, _ = routed(wl.logits, 8)
    traces, stats = run_sequence(128, 8, ids)
    dump("qwen3.json.gz", {"ids": ids, "trace": traces, "stats": stats})

    # batched: prefill chunk then batch-32 decode
    pre = W.batch_prefill(weights=False)
    dec = W.batch_decode(weights=False, steps=8)
    calls = [routed(pre.logits, 8)[0][0]] + [routed(dec.logits, 8)[0][t] for t in range(8)]
    traces, stats = run_sequence(128, 32, calls)
    dump("batch.json.gz", {"ids": calls, "trace": traces, "stats": stats})

    # mixtral: bs=1 then bs=16
    m1 = W.mixtral(weights=False)
    m16 = W.mixtral(seed=1, steps=16, tokens=16, weights=False)
    calls = [r for r in routed(m1.logits, 2)[0]] + [r for r in routed(m16.logits, 2)[0]]
    traces, stats = run_sequence(8, 4, calls)
    dump("mixtral.json.gz", {"ids": calls, "trace": traces, "stats": stats})

    # 48-layer stack: layer L's pager sees token t's layer-L routing
    lg = W.stack_routing(tokens=32)
    layers = []
    for L in range(lg.shape[0]):
        ids = [route(lg[L, t:t + 1], 8)[1].tolist() for t in range(lg.shape[1])]
        traces, stats = run_sequence(128, 24, ids)
        layers.append({"ids": ids, "trace": traces, "stats": stats})
    dump("stack.json.gz", {"layers": layers})


if __name__ == "__main__":
    main()
