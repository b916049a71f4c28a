"""Ordering hazards and kernel coverage of the layer call on the GPU.

* Two prefetches of one layer with no layer call between them (allowed by the
  reference API, fused_moe.py:360-433): the second one's decisions must not
  rewrite the record the first one's side-stream copies still read.
* A workspace that grows between queued calls (bs=1, then a larger batch,
  with no host synchronisation): the old pinned decision record must not be
  released while a queued pager kernel still writes it.
* Shapes the decode GEMV pair does not cover are decided before the pager
  runs: bf16 takes the MFMA path, fp32 fails with the pager state untouched.

Every case runs behind bounded spin kernels on the caller's stream, so the
host is far ahead of the GPU wherever it does not wait.
"""
import random

import pytest
import torch

from oracle.moe import moe_forward, route
from oracle.pager import PagerOracle
from tests.test_gpu_layer import bits, drive, rel_err
from wisp_amd import workloads as W
from wisp.integrations.vllm.fused_moe import WispMoEState

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
SPIN_CYCLES = 2_000_000


def _spin():
    if hasattr(torch.cuda, "_sleep"):
        torch.cuda._sleep(SPIN_CYCLES)


def _resident(w13, w2, E):
    res = WispMoEState(w13, w2, E, "resident", DEV, 99)
    res.prime_identity()
    return res


@pytest.mark.parametrize("engine", ["kernel", "memcpy"])
def test_back_to_back_prefetches_without_a_layer_call(monkeypatch, engine):
    monkeypatch.setenv("WISP_PAGEIN_ENGINE", engine)
    wl = W.toy(steps=12, pin=True)
    w13, w2 = wl.views()
    E, K, cap = wl.shape.experts, wl.shape.top_k, 6
    paged = WispMoEState(w13, w2, cap, "paged", DEV, 0)
    assert paged.pagein_engine == engine
    res = _resident(w13, w2, E)
    rng = random.Random(3)
    preds = [[set(rng.sample(range(E), 3)), set(rng.sample(range(E), 4))]
             for _ in range(wl.steps)]
    xs = [wl.x[t].to(DEV) for t in range(wl.steps)]
    lgs = [wl.logits[t].to(DEV) for t in range(wl.steps)]
    torch.cuda.synchronize()
    print(f"queueing {wl.steps} calls with two prefetches each, engine={engine}", flush=True)
    outs = []
    for t in range(wl.steps):
        _spin()
        outs.append(paged.forward(xs[t], lgs[t], K, True))
        for p in preds[t]:  # back to back: no layer call between them
            paged.prefetch_async(p)
    torch.cuda.synchronize()
    ora = PagerOracle(E, cap)
    for t in range(wl.steps):
        ref = res.forward(xs[t], lgs[t], K, True)
        torch.cuda.synchronize()
        assert torch.equal(bits(outs[t]), bits(ref)), t
        ora.forward(route(wl.logits[t], K)[1].tolist())
        for p in preds[t]:
            ora.prefetch_async(p)
    assert paged.slot_to_expert == ora.slot_to_expert
    assert paged.lru_tick == ora.lru_tick and paged.lru_clock == ora.lru_clock
    assert (paged.stats_miss, paged.stats_evict, paged.stats_hits) == \
        (ora.stats_miss, ora.stats_evict, ora.stats_hits)


@pytest.mark.parametrize("engine", ["kernel", "memcpy"])
def test_workspace_grows_between_queued_calls(monkeypatch, engine):
    """Token counts 1, 1, 16, 1, 40, 2 in a row, each call queued behind a
    spin with no host synchronisation: every growth of the workspace (and of
    its pinned decision record) lands while earlier calls are still queued.
    Decisions match the oracle and outputs equal the resident layer's bytes."""
    monkeypatch.setenv("WISP_PAGEIN_ENGINE", engine)
    sizes = [1, 1, 16, 1, 40, 2]
    wl = W.toy(steps=sum(sizes), pin=True)
    w13, w2 = wl.views()
    E, K, H, cap = wl.shape.experts, wl.shape.top_k, wl.shape.hidden, 4
    paged = WispMoEState(w13, w2, cap, "paged", DEV, 0)
    res = _resident(w13, w2, E)
    calls, a = [], 0
    for T in sizes:
        calls.append((wl.x[a:a + T].reshape(T, H), wl.logits[a:a + T].reshape(T, E)))
        a += T
    dev_calls = [(x.to(DEV), lg.to(DEV)) for x, lg in calls]
    torch.cuda.synchronize()
    print(f"queueing calls of {sizes} tokens, engine={engine}", flush=True)
    outs = []
    for x, lg in dev_calls:
        _spin()
        outs.append(paged.forward(x, lg, K, True))
    torch.cuda.synchronize()
    ora = PagerOracle(E, cap)
    for i, ((x, lg), (xc, lgc)) in enumerate(zip(dev_calls, calls)):
        ref = res.forward(x, lg, K, True)
        torch.cuda.synchronize()
        assert torch.equal(bits(outs[i]), bits(ref)), i
        w, ids = route(lgc, K)
        ora.forward(ids.tolist())
        o = moe_forward(xc, w, ids, w13, w2)
        assert rel_err(outs[i], o) < 1e-5, i
    assert paged.slot_to_expert == ora.slot_to_expert and paged.lru_tick == ora.lru_tick
    assert (paged.stats_forward, paged.stats_miss, paged.stats_evict, paged.stats_hits) == \
        (ora.stats_forward, ora.stats_miss, ora.stats_evict, ora.stats_hits)


@pytest.mark.parametrize("T", [1, 3])
def test_bf16_rows_longer_than_the_gemv_take_the_mfma_path(monkeypatch, T):
    """Hidden 6144 (Mixtral-8x22B's) is past the GEMV w13 kernel's registers:
    the decode call runs on the MFMA path, decisions match the oracle and
    paged bytes equal resident bytes."""
    monkeypatch.setitem(W.SHAPES, "h6144", W.LayerShape(6144, 256, 16, 2, 4, torch.bfloat16))
    wl = W.gaussian_logits("h6144", seed=T, steps=4, tokens=T, pin=True)
    drive(wl, 4, wl.steps, tol=1e-2)


@pytest.mark.parametrize("H,K", [(256, 17), (4096, 2)])
def test_fp32_shapes_no_kernel_covers_fail_before_the_pager(monkeypatch, H, K):
    """fp32 has only the GEMV pair (up to 16 experts per token, rows up to
    2048 elements): the call raises NotImplementedError and leaves every
    piece of pager state as it was; a covered call afterwards is exact."""
    E = 32
    monkeypatch.setitem(W.SHAPES, "f32wide", W.LayerShape(H, 128, E, K, E, torch.float32))
    wl = W.gaussian_logits("f32wide", seed=H + K, steps=2, tokens=1, pin=True)
    w13, w2 = wl.views()
    st = WispMoEState(w13, w2, E, "paged", DEV, 0)
    x, lg = wl.x[0].to(DEV), wl.logits[0].to(DEV)
    with pytest.raises(NotImplementedError, match="no expert kernel covers"):
        st.forward(x, lg, K, True)
    torch.cuda.synchronize()
    assert st.stats_forward == 0 and st.stats_miss == 0 and st.lru_clock == 0
    assert st.slot_to_expert == [-1] * E
    assert st.expert_map_device.tolist() == [-1] * E
    if H > 2048:
        return
    # top_k 2 on the same layer is covered and starts from the untouched state
    out = st.forward(x, lg, 2, True)
    torch.cuda.synchronize()
    ora = PagerOracle(E, E)
    w, ids = route(wl.logits[0], 2)
    ora.forward(ids.tolist())
    assert st.slot_to_expert == ora.slot_to_expert and st.lru_tick == ora.lru_tick
    assert rel_err(out, moe_forward(wl.x[0], w, ids, w13, w2)) < 1e-5
