"""Stream fences of side-stream page-in, proved under a stalled caller's stream.

Prefetch copies run on a layer's side stream (src/wisp/integrations/vllm/
fused_moe.py:360-433 issues them on copy_stream with copy_event); here the
side stream waits for the prefetch decisions queued on the caller's stream
(read-after-write, and, through stream order, after every earlier kernel that
read the slots: write-after-read), and the layer's next call waits for the
copies before its own page-in and expert kernels (read-after-write).

The test queues a whole 4-layer stack for many tokens with no host
synchronisation and a long, bounded spin kernel before every layer call, so
the caller's stream runs far behind the host and the side stream would race
ahead of it wherever a fence were missing: a copy would then use a stale
decision record or overwrite a slot still being read, and the chained layer
outputs would leave the resident layer's bytes.
"""
import pytest
import torch

from oracle.cooccur import CooccurOracle, prefetch_glue
from oracle.moe import route
from oracle.pager import PagerOracle
from wisp_amd import workloads as W
from wisp.integrations.vllm import fused_moe as fm

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
SPIN_CYCLES = 2_000_000  # a bounded busy loop on the caller's stream


@pytest.mark.parametrize("engine", ["kernel", "memcpy"])
def test_prefetch_fences_hold_under_a_stalled_stream(monkeypatch, engine):
    if not hasattr(torch.cuda, "_sleep"):
        pytest.skip("torch.cuda._sleep is not available")
    monkeypatch.setenv("WISP_PAGEIN_ENGINE", engine)
    monkeypatch.setenv("WISP_PREFETCH", "1")
    monkeypatch.setenv("WISP_COOCCUR_ONLINE", "1")
    monkeypatch.delenv("WISP_COOCCUR_PATH", raising=False)
    layers, cap, tokens = 4, 4, 16
    wl = W.toy(steps=1, pin=True)
    E, K = wl.shape.experts, wl.shape.top_k
    lg = torch.from_numpy(W.stack_routing(seed=11, layers=layers, tokens=tokens, experts=E, k=K))
    xs = torch.randn((tokens, 1, wl.shape.hidden), generator=torch.Generator().manual_seed(12))
    w13, w2 = wl.views()
    fm._reset_cooccur()
    states = [fm.WispMoEState(w13, w2, cap, "paged", DEV, L) for L in range(layers)]
    monkeypatch.setattr(fm, "_LAYER_STATES", states)
    assert all(s.pagein_engine == engine for s in states)
    lgd, xsd = lg.to(DEV), xs.to(DEV)
    torch.cuda.synchronize()
    print(f"queueing {tokens} tokens x {layers} layers, engine={engine}", flush=True)
    outs = []
    try:
        for t in range(tokens):
            h = xsd[t]
            for L in range(layers):
                torch.cuda._sleep(SPIN_CYCLES)
                h = states[L].forward(h, lgd[L, t:t + 1], K, True)
                fm._prefetch_after_forward(states[L])
                outs.append(h)
        torch.cuda.synchronize()
    finally:
        fm._reset_cooccur()

    # the same chain through a resident layer, one call at a time
    res = fm.WispMoEState(w13, w2, E, "resident", DEV, layers)
    res.prime_identity()
    i = 0
    for t in range(tokens):
        h = xsd[t]
        for L in range(layers):
            h = res.forward(h, lgd[L, t:t + 1], K, True)
            torch.cuda.synchronize()
            assert torch.equal(outs[i].view(torch.int32), h.view(torch.int32)), (t, L)
            i += 1

    # and the pager states the oracle's prefetch glue reaches
    oras = [PagerOracle(E, cap) for _ in range(layers)]
    table = CooccurOracle()
    obs = {}
    for t in range(tokens):
        for L in range(layers):
            oras[L].forward(route(lg[L, t:t + 1], K)[1].tolist())
            prefetch_glue(oras, L, table, obs, online=True)
    for L in range(layers):
        s, o = states[L], oras[L]
        assert s.slot_to_expert == o.slot_to_expert, L
        assert s.lru_tick == o.lru_tick and s.lru_clock == o.lru_clock, L
        assert (s.stats_evict, s.stats_miss, s.stats_hits, s.stats_pred_total) == \
            (o.stats_evict, o.stats_miss, o.stats_hits, o.stats_pred_total), L
    assert sum(s.stats_pred_total for s in states) > 0  # prefetch really ran


def test_queued_decode_holds_under_a_stalled_stream(monkeypatch):
    """Sub-batched calls with side-stream hipMemcpyAsync page-in (two copy
    streams) between spins on the caller's stream.  The host waits for each
    call's pager decisions, which drains the spin before it; within the call
    each group's copies wait for the previous group's kernels and the group's
    kernels wait for its copies, through events only.  Every output equals
    the resident layer's bytes and the pager state the oracle's."""
    if not hasattr(torch.cuda, "_sleep"):
        pytest.skip("torch.cuda._sleep is not available")
    monkeypatch.setenv("WISP_PAGEIN_ENGINE", "memcpy")
    monkeypatch.setenv("WISP_PAGEIN_STREAMS", "2")
    wl = W.gaussian_logits("batch", seed=5, steps=4, tokens=16, pin=True)
    w13, w2 = wl.views()
    K = wl.shape.top_k
    paged = fm.WispMoEState(w13, w2, 32, "paged", DEV, 0)
    res = fm.WispMoEState(w13, w2, wl.shape.experts, "resident", DEV, 1)
    res.prime_identity()
    xs = [wl.x[t].to(DEV) for t in range(wl.steps)]
    lgs = [wl.logits[t].to(DEV) for t in range(wl.steps)]
    torch.cuda.synchronize()
    outs = []
    for t in range(wl.steps):
        torch.cuda._sleep(SPIN_CYCLES)
        outs.append(paged.forward(xs[t], lgs[t], K, True))
        torch.cuda._sleep(SPIN_CYCLES)  # behind the call's last group
    torch.cuda.synchronize()
    ora = PagerOracle(wl.shape.experts, 32)
    for t in range(wl.steps):
        ref = res.forward(xs[t], lgs[t], K, True)
        torch.cuda.synchronize()
        assert torch.equal(outs[t].view(torch.int16), ref.view(torch.int16)), t
        ora.forward(route(wl.logits[t], K)[1].tolist())
    assert paged.slot_to_expert == ora.slot_to_expert and paged.lru_tick == ora.lru_tick
    assert paged.stats_miss == ora.stats_miss and paged.stats_evict == ora.stats_evict
