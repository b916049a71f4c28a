"""Golden fixtures (tests/golden/, written by make_golden.py from the oracle):
the oracle and the generators still reproduce them, and the C++ pager
specification reproduces every trace bit for bit."""
import numpy as np
import pytest
import torch

from oracle.moe import moe_forward, route
from tests._util import HostPager, fixture_matches, load_golden
from wisp_amd import workloads as W

TRACES = {"toy.json.gz": (16, 4), "qwen3.json.gz": (128, 8), "batch.json.gz": (128, 32),
          "mixtral.json.gz": (8, 4)}


@pytest.mark.parametrize("name", sorted(TRACES))
def test_host_pager_reproduces_fixture(name):
    E, cap = TRACES[name]
    g = load_golden(name)
    hp = HostPager(E, cap)
    for ids, entry in zip(g["ids"], g["trace"]):
        rec = hp.call(ids, K=len(ids[0]))
        assert rec["rc"] == 0
        fixture_matches(entry, rec, hp.s2e.tolist(), hp.tick.tolist(), hp.clock)
    st = g["stats"]
    assert hp.ctr[1:5].tolist() == [st["forward"], st["miss"], st["evict"], st["hits"]]


def test_host_pager_reproduces_stack_fixture():
    g = load_golden("stack.json.gz")
    for layer in g["layers"]:
        hp = HostPager(128, 24)
        for ids, entry in zip(layer["ids"], layer["trace"]):
            rec = hp.call(ids, K=8)
            fixture_matches(entry, rec, hp.s2e.tolist(), hp.tick.tolist(), hp.clock)


def test_generators_reproduce_fixture_routing():
    wl = W.toy()
    g = load_golden("toy.json.gz")
    for t in range(wl.steps):
        w, ids = route(wl.logits[t], 2)
        assert ids.tolist() == g["ids"][t]
        assert np.allclose(w, g["weights"][t], rtol=1e-12)
    q = W.qwen3_decode(weights=False)
    gq = load_golden("qwen3.json.gz")
    for t in range(q.steps):
        assert route(q.logits[t], 8)[1].tolist() == gq["ids"][t]
    m = W.mixtral(weights=False)
    gm = load_golden("mixtral.json.gz")
    for t in range(m.steps):
        assert route(m.logits[t], 2)[1].tolist() == gm["ids"][t]


def test_toy_outputs_fixture():
    wl = W.toy()
    g = load_golden("toy.json.gz")
    out = np.load(__import__("os").path.join(__import__("os").path.dirname(__file__), "golden",
                                             "toy_out.npz"))["out"]
    w13, w2 = wl.views()
    for t in (0, 17, 63):
        ref = moe_forward(wl.x[t], np.asarray(g["weights"][t]), np.asarray(g["ids"][t]), w13, w2)
        assert np.allclose(ref.numpy(), out[t], rtol=1e-12, atol=1e-14)


@pytest.mark.parametrize("name,k", [("toy", 2), ("qwen3", 8), ("mixtral", 2)])
def test_logit_order_equals_probability_order(name, k):
    # The oracle ranks by logit; vLLM ranks by float32 softmax probability.
    # On the fixture workloads the two agree at every routed position.
    wl = {"toy": W.toy, "qwen3": lambda: W.qwen3_decode(weights=False),
          "mixtral": lambda: W.mixtral(weights=False)}[name]()
    lg = wl.logits.reshape(-1, wl.shape.experts)
    p = torch.softmax(lg.float(), -1)
    for t in range(lg.shape[0]):
        by_logit = np.lexsort((np.arange(lg.shape[1]), -lg[t].numpy()))[: k + 1]
        by_prob = np.lexsort((np.arange(lg.shape[1]), -p[t].numpy()))[: k + 1]
        assert by_logit[:k].tolist() == by_prob[:k].tolist()
