"""Layer calls on the GPU: decision traces bit-exact with the oracle, outputs
within tolerance of the float64 oracle, paged bytes == resident bytes."""
import numpy as np
import pytest
import torch

from oracle.moe import moe_forward, route
from oracle.pager import PagerOracle
from tests._util import oracle_trace_matches
from wisp_amd import workloads as W
from wisp.integrations.vllm.fused_moe import WispMoEState
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


def drive(wl, cap, steps, check_out_every=1, tol=None, act_round=None, algo=0, timed=False):
    sts = states(wl, cap)
    if timed:
        sts["paged"].profile(True)
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


def test_toy_fp32_layer_cap_equals_top_k():
    # cap == top_k: every one-token call fills every slot, so the decode
    # kernels lay their waves out by slot (a miss on most calls here)
    wl = W.toy(pin=True)
    drive(wl, wl.shape.top_k, wl.steps, tol=1e-5)


@pytest.mark.parametrize("engine,streams", [("kernel", "0"), ("memcpy", "0"), ("memcpy", "1"),
                                            ("memcpy", "2")])
def test_qwen3_bf16_layer_decode(monkeypatch, engine, streams):
    # copy kernel (default), or hipMemcpyAsync on the caller's stream or on
    # side streams with events
    monkeypatch.setenv("WISP_PAGEIN_ENGINE", engine)
    monkeypatch.setenv("WISP_PAGEIN_STREAMS", streams)
    wl = W.qwen3_decode(steps=48, pin=True)
    sts = drive(wl, 8, wl.steps, check_out_every=1, tol=1e-2, timed=True)
    assert sts["paged"].pagein_engine == engine
    ms, nbytes = sts["paged"].pagein_stats()
    assert ms > 0 and nbytes == sts["paged"].stats_miss * wl.shape.expert_bytes
    # timing off (the default): the same calls count nothing
    sts["paged"].profile(False)
    for t in range(4):
        sts["paged"].forward(wl.x[t].to(DEV), wl.logits[t].to(DEV), wl.shape.top_k, True)
    torch.cuda.synchronize()
    assert sts["paged"].pagein_stats() == (0.0, 0.0)


@pytest.mark.parametrize("engine,streams", [("kernel", "0"), ("memcpy", "0"), ("memcpy", "2")])
def test_batched_subbatching_matches_resident_bytes(monkeypatch, engine, streams):
    monkeypatch.setenv("WISP_PAGEIN_ENGINE", engine)
    monkeypatch.setenv("WISP_PAGEIN_STREAMS", streams)
    # 16 tokens, cap 32 of 128 experts: several greedy groups per call
    wl = W.gaussian_logits("batch", seed=3, steps=3, tokens=16, pin=True)
    sts = drive(wl, 32, wl.steps, check_out_every=1, tol=1e-2)
    assert sts["paged"].pagein_engine == engine


@pytest.mark.parametrize("engine", ["kernel", "memcpy"])
def test_queued_decode_over_layers_matches_resident(monkeypatch, engine):
    # Four layers share the masters and are called round-robin with no host
    # synchronisation between calls, as a decode loop runs: every call's
    # output must still equal the resident layer's bytes, and each layer's
    # final pager state must equal its own oracle's.
    monkeypatch.setenv("WISP_PAGEIN_ENGINE", engine)
    wl = W.qwen3_decode(steps=40, pin=True)
    w13, w2 = wl.views()
    K, nl = wl.shape.top_k, 4
    paged = [WispMoEState(w13, w2, 8, "paged", DEV, i) for i in range(nl)]
    res = WispMoEState(w13, w2, wl.shape.experts, "resident", DEV, nl)
    res.prime_identity()
    oras = [PagerOracle(wl.shape.experts, 8) for _ in range(nl)]
    xs = [wl.x[t].to(DEV) for t in range(wl.steps)]
    lgs = [wl.logits[t].to(DEV) for t in range(wl.steps)]
    torch.cuda.synchronize()
    outs, refs = [], []
    for t in range(wl.steps):
        outs.append(paged[t % nl].forward(xs[t], lgs[t], K, True))
    for t in range(wl.steps):
        refs.append(res.forward(xs[t], lgs[t], K, True))
    torch.cuda.synchronize()
    for t in range(wl.steps):
        assert torch.equal(bits(outs[t]), bits(refs[t])), t
        oras[t % nl].forward(route(wl.logits[t], K)[1].tolist())
    for st, ora in zip(paged, oras):
        assert st.pagein_engine == engine
        assert st.slot_to_expert == ora.slot_to_expert and st.lru_tick == ora.lru_tick
        assert (st.stats_forward, st.stats_miss, st.stats_evict, st.stats_hits) == \
            (ora.stats_forward, ora.stats_miss, ora.stats_evict, ora.stats_hits)


def test_kernel_engine_needs_pinned_masters():
    # The copy kernel reads masters through their device mapping; a layer
    # whose masters are pageable (or whose range leaves the pinned
    # allocation) must be created with the hipMemcpyAsync engine instead.
    import ctypes as C
    from wisp_amd import _lib
    wl = W.toy(steps=1, pin=True)
    w13, w2 = wl.views()
    st = WispMoEState(w13, w2, 4, "paged", DEV, 0)
    assert st.pagein_engine == "kernel"
    pageable = wl.slabs.clone()
    assert not pageable.is_pinned()
    cases = [(pageable.data_ptr(), pageable.data_ptr() + st._w13_elems * 4),
             # starts where the pinned masters end, so the range runs past
             # their allocation (the allocator rounds sizes up to at most 2x)
             (wl.slabs.data_ptr() + wl.slabs.numel() * 4,
              wl.slabs.data_ptr() + wl.slabs.numel() * 4 + st._w13_elems * 4)]
    for m13, m2 in cases:
        d = st._make_desc()
        d.pagein_engine = _lib.WISP_PAGEIN_KERNEL
        d.master_w13, d.master_w2 = m13, m2
        h = C.c_void_p()
        _lib.check(_lib.lib().wisp_layer_create(C.byref(d), C.byref(h)), "create")
        try:
            assert _lib.lib().wisp_layer_pagein_engine(h) == _lib.WISP_PAGEIN_MEMCPY
        finally:
            _lib.lib().wisp_layer_destroy(h)


def test_kernel_engine_with_masters_in_a_large_pinned_allocation():
    """Masters at the end of one pinned allocation of more than 2 GiB (the
    allocator rounds it up to 4 GiB, a size whose range attribute does not
    read back on this runtime) still take the copy kernel; decisions match the
    oracle and paged bytes equal resident bytes.  A range that crosses the
    allocation's end is still refused."""
    import ctypes as C
    from wisp_amd import _lib
    wl = W.toy(steps=8)
    n = wl.slabs.numel() * wl.slabs.element_size()
    big = torch.empty(9 << 28, dtype=torch.uint8, pin_memory=True)  # 2.25 GiB
    off = (big.numel() - n) & ~255
    slabs = big[off:off + n].view(wl.slabs.dtype).view(wl.slabs.shape)
    slabs.copy_(wl.slabs)
    wl.slabs = slabs
    sts = drive(wl, 4, wl.steps, tol=1e-5)
    st = sts["paged"]
    assert st.pagein_engine == "kernel"
    alloc_end = big.data_ptr() + (4 << 30)  # the rounded allocation
    d = st._make_desc()
    d.pagein_engine = _lib.WISP_PAGEIN_KERNEL
    d.master_w13 = alloc_end - st._w13_elems * 4 // 2
    d.master_w2 = d.master_w13 + st._w13_elems * 4
    h = C.c_void_p()
    _lib.check(_lib.lib().wisp_layer_create(C.byref(d), C.byref(h)), "create")
    try:
        assert _lib.lib().wisp_layer_pagein_engine(h) == _lib.WISP_PAGEIN_MEMCPY
    finally:
        _lib.lib().wisp_layer_destroy(h)
    del sts, st
    torch.cuda.synchronize()


def test_empty_calls_tick_the_clock_like_the_reference():
    """A zero-token call between decode steps returns an empty output and
    moves the pager as the reference's empty ensure_resident does (the
    clock and the call count tick); later calls keep matching the oracle and
    the resident layer's bytes."""
    wl = W.toy(steps=8, pin=True)
    sh, K = wl.shape, wl.shape.top_k
    sts = states(wl, 4)
    paged, res = sts["paged"], sts["resident"]
    ora = PagerOracle(sh.experts, 4)
    x0 = torch.empty((0, sh.hidden), dtype=wl.x.dtype, device=DEV)
    lg0 = torch.empty((0, sh.experts), dtype=torch.float32, device=DEV)
    for t in range(wl.steps):
        if t % 2:
            out0 = paged.forward(x0, lg0, K, True)
            torch.cuda.synchronize()
            assert tuple(out0.shape) == (0, sh.hidden)
            ora.forward([])
        x, lg = wl.x[t].to(DEV), wl.logits[t].to(DEV)
        out = paged.forward(x, lg, K, True)
        ref = res.forward(x, lg, K, True)
        torch.cuda.synchronize()
        assert torch.equal(bits(out), bits(ref)), t
        ora.forward(route(wl.logits[t], K)[1].tolist())
        assert paged.slot_to_expert == ora.slot_to_expert, t
        assert paged.lru_tick == ora.lru_tick and paged.lru_clock == ora.lru_clock, t
    assert (paged.stats_forward, paged.stats_miss, paged.stats_evict, paged.stats_hits) == \
        (ora.stats_forward, ora.stats_miss, ora.stats_evict, ora.stats_hits)


@pytest.mark.parametrize("E,T", [(200, 1), (200, 8), (512, 1), (512, 4), (512, 8)])
def test_wide_expert_counts_with_fused_routing(monkeypatch, E, T):
    """Routing fused into the pager for E above 128 (4 and 8 logits per lane,
    with the layer state read into registers before routing): decisions match
    the oracle bit for bit and paged bytes equal resident bytes, one-group and
    sub-batched (T * K above cap)."""
    monkeypatch.setitem(W.SHAPES, "wide", W.LayerShape(256, 128, E, 8, 48, torch.bfloat16))
    wl = W.gaussian_logits("wide", seed=E + T, steps=6, tokens=T, pin=True)
    drive(wl, 48, wl.steps, tol=1e-2)


@pytest.mark.parametrize("T", [1, 3])
def test_top_k_above_the_gemv_limit_takes_the_mfma_path(monkeypatch, T):
    """20 routed experts per token (the decode GEMV pair handles up to 16):
    the automatic choice runs the MFMA path even for a one-token call, with
    decisions matching the oracle and paged bytes equal to resident bytes."""
    monkeypatch.setitem(W.SHAPES, "topk20", W.LayerShape(512, 256, 64, 20, 24, torch.bfloat16))
    wl = W.gaussian_logits("topk20", seed=T, steps=4, tokens=T, pin=True)
    drive(wl, 24, wl.steps, tol=1e-2)


def test_forward_refuses_tensors_off_the_device_and_bad_out():
    """Tensors in host memory would reach the kernels as raw pointers, and a
    wrong out buffer would be overrun: both are refused before any launch."""
    wl = W.toy(steps=2, pin=True)
    sh, K = wl.shape, wl.shape.top_k
    st = states(wl, 4, modes=("paged",))["paged"]
    x, lg = wl.x[0].to(DEV), wl.logits[0].to(DEV)
    with pytest.raises(ValueError, match="x is on"):
        st.forward(wl.x[0], lg, K, True)
    with pytest.raises(ValueError, match="router_logits is on"):
        st.forward(x, wl.logits[0], K, True)
    for bad in (torch.empty((2, sh.hidden), dtype=x.dtype, device=DEV),
                torch.empty((1, sh.hidden), dtype=torch.bfloat16, device=DEV),
                torch.empty((sh.hidden, 2), dtype=x.dtype, device=DEV)[:, :1].t(),
                torch.empty((1, sh.hidden), dtype=x.dtype)):
        with pytest.raises(ValueError, match="out"):
            st.forward(x, lg, K, True, out=bad)
    assert st.stats_forward == 0  # nothing reached the pager
    good = torch.empty_like(x)
    assert st.forward(x, lg, K, True, out=good).data_ptr() == good.data_ptr()


def test_prefill_chunk_layer_mfma():
    # 96-token chunk at the Qwen3 shape, cap 32 of 128 experts: the call is
    # split into greedy token groups and runs on the MFMA grouped GEMM
    wl = W.batch_prefill(tokens=96, pin=True)
    drive(wl, 32, 1, tol=1e-2)


def test_batched_config_at_full_size_against_the_fixture():
    """The batched configuration at its real sizes on one layer state (Qwen3
    shape, cap 32, router logits N(0,1)): the 512-token prefill chunk, then
    bs=32 decode steps, the sequence of tests/golden/batch.json.gz.  Every
    call's decisions, slot table and ticks equal the fixture's; every output
    equals the resident layer's bytes and is within 1e-2 of the float64
    oracle."""
    from tests._util import fixture_matches, load_golden
    g = load_golden("batch.json.gz")
    pre = W.batch_prefill(pin=True)
    dec = W.batch_decode(steps=8, weights=False)  # the fixture's draw; 3 steps run
    calls = [(pre.x[0], pre.logits[0])] + [(dec.x[t], dec.logits[t]) for t in range(3)]
    w13, w2 = pre.views()
    K, E, cap = 8, pre.shape.experts, 32
    paged = WispMoEState(w13, w2, cap, "paged", DEV, 0)
    res = WispMoEState(w13, w2, E, "resident", DEV, 1)
    res.prime_identity()
    for i, (x, lg) in enumerate(calls):
        print(f"call {i}: {x.shape[0]} tokens", flush=True)
        xd, lgd = x.to(DEV), lg.to(DEV)
        out = paged.forward(xd, lgd, K, True)
        ref = res.forward(xd, lgd, K, True)
        torch.cuda.synchronize()
        assert torch.equal(bits(out), bits(ref)), i
        _, ids_gpu = paged.last_topk
        assert ids_gpu.cpu().tolist() == g["ids"][i]
        rec = parse_record(paged.last_record.numpy(), x.shape[0], K)
        fixture_matches(g["trace"][i], rec, paged.slot_to_expert, paged.lru_tick,
                        paged.lru_clock)
        w_ref, ids_ref = route(lg, K)
        o = moe_forward(x, w_ref, ids_ref, w13, w2)
        assert rel_err(out, o) < 1e-2, i


@pytest.mark.parametrize("algo", [1, 2], ids=["gemv", "mfma"])
def test_batched_decode_explicit_algo(algo):
    wl = W.batch_decode(steps=2, tokens=8, pin=True)
    drive(wl, 32, wl.steps, tol=1e-2, algo=algo)


def test_mixtral_shape_decode_small_steps():
    wl = W.mixtral(steps=6, pin=True)
    drive(wl, 4, wl.steps, check_out_every=3, tol=1e-2)


def test_mixtral_shape_batch16_mfma():
    # bs=16 at the Mixtral shape (8 experts, top-2, cap 4): sub-batched groups
    # on the MFMA path
    wl = W.mixtral(steps=2, tokens=16, pin=True)
    drive(wl, 4, wl.steps, check_out_every=2, tol=1e-2)


def test_overflow_token_raises_subbatch():
    wl = W.toy(steps=2, pin=True)
    w13, w2 = wl.views()
    st = WispMoEState(w13, w2, 2, "paged", DEV, 0)
    x = wl.x[0].to(DEV)
    with pytest.raises(RuntimeError, match="sub-batch"):
        st.forward(x, wl.logits[0].to(DEV), 3, True)
