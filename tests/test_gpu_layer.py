"""Layer calls on the GPU: decision traces bit-exact with the oracle, outputs
within tolerance of the float64 oracle, paged bytes == resident bytes."""
import numpy as np
import pytest
import torch

from oracle.moe import moe_forward, route
from oracle.pager import PagerOracle
from tests._util import oracle_trace_matches
from wisp_amd import workloads as W
from wisp_amd.integrations.vllm.fused_moe import WispMoEState
from wisp_amd.record import parse_record

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def rel_err(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return float((a - b).abs().max() / b.abs().max().clamp_min(1e-30))


def states(wl, cap, modes=("paged", "resident")):
    w13, w2 = wl.views()
    out = {}
    for m in modes:
        st = WispMoEState(w13, w2, wl.shape.experts if m == "resident" else cap, m, DEV, 0)
        if m == "resident":
            st.prime_identity()
        out[m] = st
    return out


def bits(t):
    return t.view(torch.int16) if t.dtype == torch.bfloat16 else t.view(torch.int32)


def drive(wl, cap, steps, check_out_every=1, tol=None, act_round=None, algo=0):
    sts = states(wl, cap)
    ora = PagerOracle(wl.shape.experts, cap)
    w13, w2 = wl.views()
    K = wl.shape.top_k
    for t in range(steps):
        x = wl.x[t].to(DEV)
        lg = wl.logits[t].to(DEV)
        outs = {m: st.forward(x, lg, K, True, algo=algo) for m, st in sts.items()}
        torch.cuda.synchronize()
        assert torch.equal(bits(outs["paged"]), bits(outs["resident"])), t
        w_ref, ids_ref = route(wl.logits[t], K)
        res = ora.forward(ids_ref.tolist())
        pst = sts["paged"]
        w_gpu, ids_gpu = pst.last_topk
        assert ids_gpu.cpu().numpy().tolist() == ids_ref.tolist()
        assert np.allclose(w_gpu.cpu().numpy(), w_ref, rtol=2e-6, atol=1e-7)
        rec = parse_record(pst.last_record.numpy(), wl.tokens, K)
        oracle_trace_matches(res, rec)
        assert pst.last_slots.cpu().tolist() == res["slots"]
        assert pst.slot_to_expert == ora.slot_to_expert and pst.lru_tick == ora.lru_tick
        if tol is not None and t % check_out_every == 0:
            ref = moe_forward(wl.x[t], w_ref, ids_ref, w13, w2, act_round=act_round)
            assert rel_err(outs["paged"], ref) < tol, t
    st = sts["paged"]
    assert (st.stats_forward, st.stats_miss, st.stats_evict, st.stats_hits) == \
        (ora.stats_forward, ora.stats_miss, ora.stats_evict, ora.stats_hits)
    return sts


def test_toy_fp32_layer_all_steps():
    wl = W.toy(pin=True)
    drive(wl, 4, wl.steps, tol=1e-5)


@pytest.mark.parametrize("streams", ["0", "1", "2"])
def test_qwen3_bf16_layer_decode(monkeypatch, streams):
    # page-in on the caller's stream (default) or on side streams with events
    monkeypatch.setenv("WISP_PAGEIN_STREAMS", streams)
    wl = W.qwen3_decode(steps=48, pin=True)
    sts = drive(wl, 8, wl.steps, check_out_every=8, tol=1e-2)
    ms, nbytes = sts["paged"].pagein_stats()
    assert nbytes > 0 and ms > 0


@pytest.mark.parametrize("streams", ["0", "2"])
def test_batched_subbatching_matches_resident_bytes(monkeypatch, streams):
    monkeypatch.setenv("WISP_PAGEIN_STREAMS", streams)
    # 16 tokens, cap 32 of 128 experts: several greedy groups per call
    wl = W.gaussian_logits("batch", seed=3, steps=3, tokens=16, pin=True)
    drive(wl, 32, wl.steps, check_out_every=1, tol=1e-2)


def test_mixtral_shape_decode_small_steps():
    wl = W.mixtral(steps=6, pin=True)
    drive(wl, 4, wl.steps, check_out_every=3, tol=1e-2)


def test_overflow_token_raises_subbatch():
    wl = W.toy(steps=2, pin=True)
    w13, w2 = wl.views()
    st = WispMoEState(w13, w2, 2, "paged", DEV, 0)
    x = wl.x[0].to(DEV)
    with pytest.raises(RuntimeError, match="sub-batch"):
        st.forward(x, wl.logits[0].to(DEV), 3, True)

