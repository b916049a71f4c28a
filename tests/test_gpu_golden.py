"""The GPU path against the committed golden fixtures: routing ids from the
route kernel, decision traces from the pager kernel, and the toy layer's
outputs through the full paged layer call."""
import os

import numpy as np
import pytest
import torch

from tests._util import fixture_matches, load_golden
from tests.test_gpu_kernels import DevPager, gpu_route
from wisp_amd import workloads as W
from wisp.integrations.vllm.fused_moe import WispMoEState

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name,E,cap", [("toy.json.gz", 16, 4), ("qwen3.json.gz", 128, 8),
                                        ("batch.json.gz", 128, 32), ("mixtral.json.gz", 8, 4)])
def test_gpu_pager_reproduces_fixture(name, E, cap):
    g = load_golden(name)
    dp = DevPager(E, cap)
    for ids, entry in zip(g["ids"], g["trace"]):
        rec = dp.call(ids, len(ids[0]))
        fixture_matches(entry, rec, dp.s2e.tolist(), dp.tick.tolist(), int(dp.ctr[0]))


def test_gpu_pager_reproduces_stack_fixture():
    g = load_golden("stack.json.gz")
    for layer in g["layers"][:12]:
        dp = DevPager(128, 24)
        for ids, entry in zip(layer["ids"], layer["trace"]):
            rec = dp.call(ids, 8)
            fixture_matches(entry, rec, dp.s2e.tolist(), dp.tick.tolist(), int(dp.ctr[0]))


@pytest.mark.parametrize("name,make,k", [
    ("qwen3.json.gz", lambda: W.qwen3_decode(weights=False), 8),
    ("mixtral.json.gz", lambda: W.mixtral(weights=False), 2),
    ("toy.json.gz", W.toy, 2)])
def test_gpu_routing_reproduces_fixture(name, make, k):
    wl = make()
    g = load_golden(name)
    lg = wl.logits.reshape(-1, wl.shape.experts)
    _, ids = gpu_route(lg, k)
    assert ids.numpy().tolist() == [row for call in g["ids"][: wl.steps] for row in call]


def test_toy_layer_outputs_fixture():
    wl = W.toy(pin=True)
    g = load_golden("toy.json.gz")
    out_ref = np.load(os.path.join(os.path.dirname(__file__), "golden", "toy_out.npz"))["out"]
    w13, w2 = wl.views()
    st = WispMoEState(w13, w2, 4, "paged", torch.device("cuda:0"), 0)
    for t in range(wl.steps):
        out = st.forward(wl.x[t].cuda(), wl.logits[t].cuda(), 2, True)
        torch.cuda.synchronize()
        ref = torch.from_numpy(out_ref[t])
        err = float((out.double().cpu() - ref).abs().max() / ref.abs().max())
        assert err < 1e-5, (t, err)
        entry = g["trace"][t]
        assert st.slot_to_expert == entry["s2e"] and st.lru_tick == entry["tick"]
