"""Cross-layer speculative prefetch on the GPU: co-occurrence table, predictor
and prefetch decisions bit-exact with the oracle (oracle/cooccur.py,
PagerOracle.prefetch_async), and layer outputs unchanged by prefetching."""
import json
import random

import numpy as np
import pytest
import torch

from oracle.cooccur import CooccurOracle, predict_layer as predict_oracle, prefetch_glue
from oracle.moe import route
from oracle.pager import PagerOracle
from wisp_amd import workloads as W
from wisp.integrations.vllm import fused_moe as fm
from wisp.integrations.vllm.cooccur import CooccurTable, predict_layer

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _steps(rng, layers, experts, n, kmax=5):
    return [{L: rng.sample(range(experts), rng.randint(1, kmax)) for L in range(layers)}
            for _ in range(n)]


def _as_sets(d):
    return ({tuple(p) for p in d["pairs"]}, {tuple(m) for m in d["marginals"]},
            d["num_steps_observed"])


def test_gpu_table_counts_match_oracle():
    rng = random.Random(0)
    steps = _steps(rng, 5, 24, 30)
    o, g = CooccurOracle(), CooccurTable(5, 24, DEV)
    for st in steps:
        o.observe_step(st)
        g.observe_step(st)
    assert _as_sets(g.to_dict()) == _as_sets(o.to_dict())


@pytest.mark.parametrize("decay,normalize,only_prev", [(0.5, True, False), (1.0, True, False),
                                                        (0.3, True, False), (0.5, False, False),
                                                        (0.5, True, True)])
def test_gpu_predict_matches_oracle(decay, normalize, only_prev):
    rng = random.Random(1)
    L, E = 6, 40
    steps = _steps(rng, L, E, 60, kmax=8)
    o, g = CooccurOracle(), CooccurTable(L, E, DEV)
    for st in steps:
        o.observe_step(st)
        g.observe_step(st)
    for _ in range(60):
        seen = {Ls: set(rng.sample(range(E), rng.randint(1, 8)))
                for Ls in rng.sample(range(L), rng.randint(1, L))}
        target = rng.randint(0, L - 1)
        k = rng.randint(1, 20)
        want = predict_oracle(o, seen, target, k=k, normalize=normalize, decay=decay,
                              only_prev_layer=only_prev)
        got = predict_layer(g, seen, target, k=k, normalize=normalize, decay=decay,
                            only_prev_layer=only_prev)
        assert got == want, (seen, target, k)


def test_gpu_table_json_round_trip(tmp_path):
    rng = random.Random(2)
    o = CooccurOracle()
    for st in _steps(rng, 4, 16, 20):
        o.observe_step(st)
    path = tmp_path / "table.json.gz"
    g = CooccurTable.from_dict(o.to_dict(), 4, 16, DEV)
    g.save(path)
    h = CooccurTable.load(path, 4, 16, DEV)
    assert _as_sets(h.to_dict()) == _as_sets(o.to_dict())
    assert CooccurOracle.from_dict(json.loads(json.dumps(h.to_dict()))).to_dict()["pairs"]


def _toy_state(wl, cap):
    w13, w2 = wl.views()
    return fm.WispMoEState(w13, w2, cap, "paged", DEV, 0)


def test_prefetch_decisions_and_outputs_match_oracle():
    wl = W.toy(steps=40, pin=True)
    K = wl.shape.top_k
    st = _toy_state(wl, 4)
    w13, w2 = wl.views()
    res = fm.WispMoEState(w13, w2, wl.shape.experts, "resident", DEV, 1)
    res.prime_identity()
    ora = PagerOracle(wl.shape.experts, 4)
    rng = random.Random(5)
    for t in range(wl.steps):
        x, lg = wl.x[t].to(DEV), wl.logits[t].to(DEV)
        out = st.forward(x, lg, K, True)
        ref = res.forward(x, lg, K, True)
        ora.forward(route(wl.logits[t], K)[1].tolist())
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int32), ref.view(torch.int32)), t
        pred = set(rng.sample(range(wl.shape.experts), rng.randint(0, 5)))
        st.prefetch_async(pred)
        want = ora.prefetch_async(pred)
        got = st.last_prefetch
        assert (got["evicted"], got["loaded"]) == (want["evicted"], want["loaded"]), t
        assert st.slot_to_expert == ora.slot_to_expert and st.lru_tick == ora.lru_tick, t
        assert st.lru_clock == ora.lru_clock and st.stats_evict == ora.stats_evict, t


def _stack(wl, layers, cap):
    w13, w2 = wl.views()
    return [fm.WispMoEState(w13, w2, cap, "paged", DEV, L) for L in range(layers)]


@pytest.mark.parametrize("warm", [False, True], ids=["online-cold", "warm-file"])
def test_prefetch_glue_stack_matches_oracle(monkeypatch, tmp_path, warm):
    layers, cap = 4, 4
    wl = W.toy(steps=1, pin=True)
    E, K = wl.shape.experts, wl.shape.top_k
    tokens = 24
    lg = torch.from_numpy(W.stack_routing(seed=3, layers=layers, tokens=tokens, experts=E, k=K))
    xs = torch.randn((tokens, 1, wl.shape.hidden), generator=torch.Generator().manual_seed(4))
    table_o = CooccurOracle()
    if warm:
        rng = random.Random(9)
        for st in _steps(rng, layers, E, 50, kmax=K):
            table_o.observe_step(st)
        path = tmp_path / "warm.json"
        path.write_text(json.dumps(table_o.to_dict()))
        monkeypatch.setenv("WISP_COOCCUR_PATH", str(path))
        monkeypatch.delenv("WISP_COOCCUR_ONLINE", raising=False)
    else:
        monkeypatch.setenv("WISP_COOCCUR_ONLINE", "1")
        monkeypatch.delenv("WISP_COOCCUR_PATH", raising=False)
    monkeypatch.setenv("WISP_PREFETCH", "1")
    fm._reset_cooccur()
    states = _stack(wl, layers, cap)
    monkeypatch.setattr(fm, "_LAYER_STATES", states)
    w13, w2 = wl.views()
    res = fm.WispMoEState(w13, w2, E, "resident", DEV, layers)
    res.prime_identity()
    oras = [PagerOracle(E, cap) for _ in range(layers)]
    obs = {}
    try:
        for t in range(tokens):
            h = xs[t].to(DEV)
            for L in range(layers):
                logit = lg[L, t:t + 1].to(DEV)
                out = states[L].forward(h, logit, K, True)
                fm._prefetch_after_forward(states[L])
                ref = res.forward(h, logit, K, True)
                oras[L].forward(route(lg[L, t:t + 1], K)[1].tolist())
                prefetch_glue(oras, L, table_o, obs, online=not warm)
                torch.cuda.synchronize()
                assert torch.equal(out.view(torch.int32), ref.view(torch.int32)), (t, L)
                h = out
            for L in range(layers):
                s, o = states[L], oras[L]
                assert s.slot_to_expert == o.slot_to_expert, (t, L)
                assert s.lru_tick == o.lru_tick and s.lru_clock == o.lru_clock, (t, L)
                assert (s.stats_evict, s.stats_miss, s.stats_pred_total) == \
                    (o.stats_evict, o.stats_miss, o.stats_pred_total), (t, L)
        assert sum(o.stats_pred_total for o in oras) > 0  # the prefetch path ran
        tab = fm._COOCCUR_TABLE
        assert tab.num_steps_observed == table_o.num_steps_observed
        assert _as_sets(tab.to_dict())[:2] == _as_sets(table_o.to_dict())[:2]
    finally:
        fm._reset_cooccur()
