"""The 48-layer stack configuration through the full layer call on the GPU.

Qwen3-30B-A3B-shaped layers (H 2048, I 768, 128 experts, top-8, bf16) with a
cap-24 scratch and pager each, sharing one set of pinned masters, routed by
the layer-conditioned Dirichlet(0.3) co-occurrence logits of
``workloads.stack_routing`` (the first 32 tokens, which
``tests/golden/stack.json.gz`` holds).  Each token runs through the 48 layers
in order, layer L's output being layer L+1's input, with routing fused into
the pager kernel and page-in by the copy kernel.

Checked for every one of the 48 x 32 layer calls: the routed ids, the
decision record, slot table, ticks and clock against the fixture, and the
output against the resident layer's bytes (one resident state serves every
layer, since they share the masters).  One call per layer, at rotating
tokens, is checked against the float64 oracle within 1e-2.
"""
import pytest
import torch

from oracle.moe import moe_forward, route
from tests._util import fixture_matches, load_golden
from tests.test_gpu_layer import bits, rel_err
from wisp_amd import workloads as W
from wisp_amd.record import parse_record
from wisp.integrations.vllm.fused_moe import WispMoEState

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def test_stack_48_layers_cap24_through_the_layer_call():
    g = load_golden("stack.json.gz")
    layers, tokens, K, cap = 48, 32, 8, 24
    base = W.qwen3_decode(steps=1, pin=True)
    w13, w2 = base.views()
    sh = base.shape
    lg = torch.from_numpy(W.stack_routing(seed=0, layers=layers, tokens=tokens))
    x0 = torch.randn((tokens, 1, sh.hidden), generator=torch.Generator().manual_seed(1)) \
        .to(sh.dtype)
    paged = [WispMoEState(w13, w2, cap, "paged", DEV, L) for L in range(layers)]
    res = WispMoEState(w13, w2, sh.experts, "resident", DEV, layers)
    res.prime_identity()
    lgd, x0d = lg.to(DEV), x0.to(DEV)
    torch.cuda.synchronize()
    checked = 0
    for t in range(tokens):
        print(f"token {t}", flush=True)
        h = hr = x0d[t]
        for L in range(layers):
            hin = h
            h = paged[L].forward(hin, lgd[L, t:t + 1], K, True)
            hr = res.forward(hr, lgd[L, t:t + 1], K, True)
            torch.cuda.synchronize()
            assert torch.equal(bits(h), bits(hr)), (t, L)
            st = paged[L]
            _, ids = st.last_topk
            assert ids.cpu().tolist() == g["layers"][L]["ids"][t], (t, L)
            rec = parse_record(st.last_record.numpy(), 1, K)
            fixture_matches(g["layers"][L]["trace"][t], rec, st.slot_to_expert, st.lru_tick,
                            st.lru_clock)
            if t == L % tokens:  # one oracle check per layer, rotating over tokens
                w_ref, ids_ref = route(lg[L, t:t + 1], K)
                ref = moe_forward(hin.cpu(), w_ref, ids_ref, w13, w2)
                assert rel_err(h, ref) < 1e-2, (t, L)
                checked += 1
    assert checked == layers
    for L in range(layers):
        s = g["layers"][L]["stats"]
        st = paged[L]
        assert (st.stats_forward, st.stats_miss, st.stats_evict, st.stats_hits) == \
            (s["forward"], s["miss"], s["evict"], s["hits"]), L
