"""Layer calls on the GPU: decision traces bit-exact with the oracle, outputs
within tolerance of the float64 oracle, paged bytes == resident bytes."""
import numpy as np
import pytest
import torch

from oracle.moe import moe_forward, route
from oracle.pager import PagerOracle
from tests._util import fixture_matches, load_golden, oracle_trace_matches
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


def oracle_check(x, logits, outs, K, w13, w2, tol, act_round=None, label=""):
    """Every row of ``outs`` (a list of [T_i, H] outputs of calls with inputs
    ``x[i]`` / ``logits[i]``) within ``tol`` of the float64 oracle, each call
    measured as max|gpu - oracle| / max|oracle|.  The oracle evaluates every
    token independently, so all calls go through it in one batch (one float64
    conversion per expert instead of one per call)."""
    xs = torch.cat([torch.as_tensor(a).reshape(-1, a.shape[-1]) for a in x])
    lgs = torch.cat([torch.as_tensor(a).reshape(-1, a.shape[-1]) for a in logits])
    w_ref, ids_ref = route(lgs, K)
    ref = moe_forward(xs, w_ref, ids_ref, w13, w2, act_round=act_round)
    r0 = 0
    for i, o in enumerate(outs):
        n = o.shape[0]
        err = rel_err(o, ref[r0:r0 + n])
        assert err < tol, (label, i, err)
        r0 += n
    return r0


def drive(wl, cap, steps, check_out_every=1, tol=None, act_round=None, algo=0, timed=False,
          fixture=None):
    """Run ``steps`` calls of ``wl`` through a paged (cap) and a resident state:
    paged bytes == resident bytes, routing and every decision bit-exact with
    the oracle pager (and with ``fixture``'s trace when given), and the
    outputs of every ``check_out_every``-th call within ``tol`` of the float64
    oracle."""
    sts = states(wl, cap)
    if timed:
        sts["paged"].profile(True)
    ora = PagerOracle(wl.shape.experts, cap)
    w13, w2 = wl.views()
    K = wl.shape.top_k
    checked = []
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
        if fixture is not None:
            assert ids_gpu.cpu().tolist() == fixture["ids"][t]
            fixture_matches(fixture["trace"][t], rec, pst.slot_to_expert, pst.lru_tick,
                            pst.lru_clock)
        if tol is not None and t % check_out_every == 0:
            checked.append((t, outs["paged"].cpu()))
    st = sts["paged"]
    assert (st.stats_forward, st.stats_miss, st.stats_evict, st.stats_hits) == \
        (ora.stats_forward, ora.stats_miss, ora.stats_evict, ora.stats_hits)
    if checked:
        idx = [t for t, _ in checked]
        oracle_check([wl.x[t] for t in idx], [wl.logits[t] for t in idx],
                     [o for _, o in checked], K, w13, w2, tol, act_round, wl.name)
    return sts


def test_toy_fp32_layer_all_steps():
    wl = W.toy(pin=True)
    drive(wl, 4, wl.steps, tol=1e-5)


@pytest.mark.parametrize("fused", ["0", "1"])
def test_toy_fp32_layer_cap_equals_top_k(monkeypatch, fused):
    # cap == top_k: every one-token call fills every slot, so the decode
    # kernels lay their waves out by slot (a miss on most calls here); with
    # WISP_DECODE_FUSED=1 the pager, page-in and w13 run as one launch
    monkeypatch.setenv("WISP_DECODE_FUSED", fused)
    wl = W.toy(pin=True)
    drive(wl, wl.shape.top_k, wl.steps, tol=1e-5)


@pytest.mark.parametrize("fused", ["0", "1"])
def test_qwen3_decode_fused_launch_equals_two_launches(monkeypatch, fused):
    """The Qwen3 decode sequence at cap 8 == top-k: with WISP_DECODE_FUSED=1
    the pager wave, the page-in copies (started by the pager's epoch word)
    and w13 per slot share one launch; the decisions, slot tables and ticks
    equal the fixture's, outputs equal the resident layer's bytes and the
    oracle's within 1e-2, and the timing counts the same calls and bytes."""
    monkeypatch.setenv("WISP_DECODE_FUSED", fused)
    wl = W.qwen3_decode(pin=True)  # the fixture's 256-step draw; 64 steps run
    sts = drive(wl, 8, 64, tol=1e-2, timed=True, fixture=load_golden("qwen3.json.gz"))
    st = sts["paged"]
    ms, nbytes = st.pagein_stats()
    assert ms > 0 and nbytes == st.stats_miss * wl.shape.expert_bytes
    prof = st.profile(False)
    assert prof["calls"] == 64 and prof["w2_noload_calls"] == prof["w13_calls"] > 0


@pytest.mark.parametrize("engine,streams", [("kernel", "0"), ("memcpy", "0"), ("memcpy", "1"),
                                            ("memcpy", "2")])
def test_qwen3_bf16_layer_decode(monkeypatch, engine, streams):
    # copy kernel (default), or hipMemcpyAsync on the caller's stream or on
    # side streams with events
    # The copy-kernel engine runs the whole 256-step sequence of
    # tests/golden/qwen3.json.gz: every call's decisions, slot table and
    # ticks equal the fixture's and every output is checked against the
    # oracle; the other engines run its first 48 steps.
    monkeypatch.setenv("WISP_PAGEIN_ENGINE", engine)
    monkeypatch.setenv("WISP_PAGEIN_STREAMS", streams)
    full = engine == "kernel"
    wl = W.qwen3_decode(steps=256 if full else 48, pin=True)
    sts = drive(wl, 8, wl.steps, check_out_every=1, tol=1e-2, timed=True,
                fixture=load_golden("qwen3.json.gz") if full else None)
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


@pytest.mark.parametrize("engine", ["kernel", "memcpy", "fused"])
def test_queued_decode_over_layers_matches_resident(monkeypatch, engine):
    # Four layers share the masters and are called round-robin with no host
    # synchronisation between calls, as a decode loop runs: every call's
    # output must still equal the resident layer's bytes, and each layer's
    # final pager state must equal its own oracle's.
    # (fused: the copy-kernel engine with WISP_DECODE_FUSED=1)
    monkeypatch.setenv("WISP_PAGEIN_ENGINE", "kernel" if engine == "fused" else engine)
    monkeypatch.setenv("WISP_DECODE_FUSED", "1" if engine == "fused" else "0")
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
        assert st.pagein_engine == ("kernel" if engine == "fused" else engine)
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
    the resident layer's bytes.  The resident layer takes the same empty
    calls (a regression case: its routing launch read row 0 of the empty
    logits buffer, a null pointer, and faulted)."""
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
            # the resident layer too: its routing launch only ticks the
            # call count and must not read the (empty) logits
            n0 = res.stats_forward
            assert tuple(res.forward(x0, lg0, K, True).shape) == (0, sh.hidden)
            torch.cuda.synchronize()
            assert res.stats_forward == n0 + 1
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


@pytest.mark.parametrize("E,K,cap", [(3, 1, 1), (17, 2, 5), (64, 8, 8), (64, 5, 64),
                                     (100, 7, 30), (128, 1, 1), (128, 16, 16), (128, 8, 64)])
def test_one_token_pager_instance(monkeypatch, E, K, cap):
    """One-token calls routed in the pager on the register path (E <= 128,
    cap <= 64) run the instance compiled for that case: E below a wave
    (invalid lanes), K == cap (every call fills the scratch), cap = 1 and
    cap = 64 (every lane a slot).  Ids, weights, decisions and state
    bit-exact with the oracle over 40 calls, paged bytes equal to resident."""
    monkeypatch.setitem(W.SHAPES, "one", W.LayerShape(256, 128, E, K, cap, torch.bfloat16))
    wl = W.gaussian_logits("one", seed=E * 3 + K + cap, steps=40, tokens=1, pin=True)
    drive(wl, cap, wl.steps, check_out_every=8, tol=1e-2)


@pytest.mark.parametrize("E,T", [(128, 1), (128, 8), (512, 1), (512, 4)])
def test_fused_routing_with_tied_logits(monkeypatch, E, T):
    """Routing fused into the pager (the one-token register-path instance at
    E = 128, T = 1; the general instances otherwise) on logits full of exact
    ties, -0.0 and -inf: ids and decisions bit-exact with the oracle, paged
    bytes equal resident bytes."""
    from tests.test_gpu_kernels import tie_logits
    monkeypatch.setitem(W.SHAPES, "ties", W.LayerShape(256, 128, E, 8, 8 * T, torch.bfloat16))
    wl = W.gaussian_logits("ties", seed=E + T, steps=12, tokens=T, pin=True)
    rng = np.random.default_rng(E * 5 + T)
    wl.logits = torch.stack([tie_logits(rng, T, E, 8) for _ in range(wl.steps)])
    drive(wl, 8 * T, wl.steps, tol=1e-2)


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
    all 8 bs=32 decode steps of tests/golden/batch.json.gz.  Every call's
    decisions, slot table and ticks equal the fixture's; every output equals
    the resident layer's bytes and every row is within 1e-2 of the float64
    oracle."""
    g = load_golden("batch.json.gz")
    pre = W.batch_prefill(pin=True)
    dec = W.batch_decode(steps=8, weights=False)  # the fixture's draw
    calls = [(pre.x[0], pre.logits[0])] + [(dec.x[t], dec.logits[t]) for t in range(8)]
    w13, w2 = pre.views()
    K, E, cap = 8, pre.shape.experts, 32
    paged = WispMoEState(w13, w2, cap, "paged", DEV, 0)
    res = WispMoEState(w13, w2, E, "resident", DEV, 1)
    res.prime_identity()
    outs = []
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
        outs.append(out.cpu())
    # per-row bound: every token of every call, each row against its own max
    xs = [c[0][t:t + 1] for c in calls for t in range(c[0].shape[0])]
    lgs = [c[1][t:t + 1] for c in calls for t in range(c[0].shape[0])]
    rows = [o[t:t + 1] for o in outs for t in range(o.shape[0])]
    assert oracle_check(xs, lgs, rows, K, w13, w2, 1e-2, label="batch") == 512 + 8 * 32


@pytest.mark.parametrize("tokens", [600, 1024])
@pytest.mark.parametrize("cap", [32, 128])
def test_prefill_chunk_above_the_staged_id_limit(tokens, cap):
    """Prefill chunks of more than 4096 (token, k) pairs at the Qwen3 shape
    (router logits N(0,1)): the pager reads the routed ids from global memory
    and writes its decision record in device memory, mirrored to the host
    record at its end.  At cap 32 the chunk splits into ~tokens/4 greedy
    token groups; at cap = E it is one group.  Decisions, slot table and
    ticks bit-exact with the oracle, paged bytes == resident bytes, then a
    bs=32 step on the same state; sampled rows within 1e-2 of the float64
    oracle."""
    wl = W.gaussian_logits("batch", seed=11 + tokens, steps=1, tokens=tokens, pin=True)
    w13, w2 = wl.views()
    K, E = 8, wl.shape.experts
    assert tokens * K > 4096
    paged = WispMoEState(w13, w2, cap, "paged", DEV, 0)
    res = WispMoEState(w13, w2, E, "resident", DEV, 1)
    res.prime_identity()
    ora = PagerOracle(E, cap)
    x, lg = wl.x[0], wl.logits[0]
    calls = [(x, lg), (x[tokens - 32:], lg[tokens - 32:])]
    for i, (xc, lgc) in enumerate(calls):
        print(f"chunk {tokens} cap {cap} call {i}: {xc.shape[0]} tokens", flush=True)
        out = paged.forward(xc.to(DEV), lgc.to(DEV), K, True)
        ref = res.forward(xc.to(DEV), lgc.to(DEV), K, True)
        torch.cuda.synchronize()
        assert torch.equal(bits(out), bits(ref)), i
        w_ref, ids_ref = route(lgc, K)
        r = ora.forward(ids_ref.tolist())
        _, ids_gpu = paged.last_topk
        assert ids_gpu.cpu().numpy().tolist() == ids_ref.tolist()
        rec = parse_record(paged.last_record.numpy(), xc.shape[0], K)
        assert rec["status"] == 0
        oracle_trace_matches(r, rec)
        assert paged.last_slots.cpu().tolist() == r["slots"]
        assert paged.slot_to_expert == ora.slot_to_expert and paged.lru_tick == ora.lru_tick
        assert paged.lru_clock == ora.lru_clock
        if i == 0:
            assert (len(r["groups"]) > tokens // 8) == (cap < E)
            pick = [0, 1, 2, 63, 64, 255, 256, 511, 512, tokens // 2 + 3, tokens - 2,
                    tokens - 1]
            oracle_check([xc[pick]], [lgc[pick]], [out[pick].cpu()], K, w13, w2, 1e-2,
                         label=f"chunk{tokens}")
    assert (paged.stats_forward, paged.stats_miss, paged.stats_evict, paged.stats_hits) == \
        (ora.stats_forward, ora.stats_miss, ora.stats_evict, ora.stats_hits)


@pytest.mark.parametrize("algo", [1, 2], ids=["gemv", "mfma"])
def test_batched_decode_explicit_algo(algo):
    wl = W.batch_decode(steps=2, tokens=8, pin=True)
    drive(wl, 32, wl.steps, tol=1e-2, algo=algo)


def test_mixtral_config_against_the_fixture():
    """The Mixtral configuration at its real sizes (8 experts, top-2, cap 4,
    ~352 MB per expert): the 256 bs=1 decode steps, then the 16 bs=16 calls of
    tests/golden/mixtral.json.gz, in one pager sequence.  Every call's
    decisions, slot table and ticks equal the fixture's, every output equals
    the resident layer's bytes, and every output row is within 1e-2 of the
    float64 oracle (bs=1 on the GEMV pair, bs=16 sub-batched on the MFMA
    grouped GEMM)."""
    g = load_golden("mixtral.json.gz")
    m1 = W.mixtral(pin=True)
    m16 = W.mixtral(seed=1, steps=16, tokens=16, weights=False)
    calls = [(m1.x[t], m1.logits[t]) for t in range(m1.steps)] + \
            [(m16.x[t], m16.logits[t]) for t in range(m16.steps)]
    assert len(calls) == len(g["ids"]) == 272
    w13, w2 = m1.views()
    K, E, cap = 2, 8, 4
    paged = WispMoEState(w13, w2, cap, "paged", DEV, 0)
    res = WispMoEState(w13, w2, E, "resident", DEV, 1)
    res.prime_identity()
    outs = []
    for i, (x, lg) in enumerate(calls):
        if i % 64 == 0 or i >= 256:
            print(f"mixtral call {i}: {x.shape[0]} tokens", flush=True)
        xd, lgd = x.to(DEV), lg.to(DEV)
        out = paged.forward(xd, lgd, K, True)
        ref = res.forward(xd, lgd, K, True)
        torch.cuda.synchronize()
        assert torch.equal(bits(out), bits(ref)), i
        _, ids_gpu = paged.last_topk
        assert ids_gpu.cpu().tolist() == g["ids"][i], i
        rec = parse_record(paged.last_record.numpy(), x.shape[0], K)
        fixture_matches(g["trace"][i], rec, paged.slot_to_expert, paged.lru_tick,
                        paged.lru_clock)
        outs.append(out.cpu())
    assert paged.stats_miss == g["stats"]["miss"] and paged.stats_hits == g["stats"]["hits"]
    del paged, res
    torch.cuda.empty_cache()
    xs = [c[0][t:t + 1] for c in calls for t in range(c[0].shape[0])]
    lgs = [c[1][t:t + 1] for c in calls for t in range(c[0].shape[0])]
    rows = [o[t:t + 1] for o in outs for t in range(o.shape[0])]
    assert oracle_check(xs, lgs, rows, K, w13, w2, 1e-2, label="mixtral") == 256 + 16 * 16


def test_overflow_token_raises_subbatch():
    wl = W.toy(steps=2, pin=True)
    w13, w2 = wl.views()
    st = WispMoEState(w13, w2, 2, "paged", DEV, 0)
    x = wl.x[0].to(DEV)
    with pytest.raises(RuntimeError, match="sub-batch"):
        st.forward(x, wl.logits[0].to(DEV), 3, True)


@pytest.mark.parametrize("engine,streams", [("kernel", "0"), ("memcpy", "0"), ("memcpy", "2")])
def test_calls_of_mixed_sizes_on_one_state(monkeypatch, engine, streams):
    """One paged state (E 128, top-8, cap 32) driven by calls of 0 to 70
    tokens in a seeded order, so consecutive calls take different pager
    instances on the same layer state: one token routed in the kernel, up to 8
    tokens routed in the kernel, more tokens routed first (one group or
    several); on both page-in engines.  Every call: routing and decisions
    bit-exact with the oracle, the device state equal to the oracle's, paged
    bytes equal to a resident state's; every output within 1e-2 of the
    float64 oracle."""
    monkeypatch.setenv("WISP_PAGEIN_ENGINE", engine)
    monkeypatch.setenv("WISP_PAGEIN_STREAMS", streams)
    sh = W.LayerShape(256, 128, 128, 8, 32, torch.bfloat16)
    g = torch.Generator().manual_seed(11)
    slabs = W.alloc_slabs(sh, pin=True)
    W.fill_expert_weights(slabs, sh, g)
    w13, w2 = W.slab_views(slabs, sh)
    sts = {m: WispMoEState(w13, w2, sh.experts if m == "resident" else sh.cap, m, DEV, 0)
           for m in ("paged", "resident")}
    sts["resident"].prime_identity()
    ora = PagerOracle(sh.experts, sh.cap)
    K = sh.top_k
    rng = np.random.default_rng(5)
    bias = torch.from_numpy(rng.normal(0.0, 1.5, sh.experts).astype(np.float32))
    sizes = [1, 1, 8, 3, 70, 1, 0, 4, 40, 1, 12, 2, 1, 64, 5, 1, 9, 1, 33, 6]
    xs, lgs, outs = [], [], []
    for t, T in enumerate(sizes):
        x = torch.randn((T, sh.hidden), generator=g).to(sh.dtype)
        lg = torch.randn((T, sh.experts), generator=g) + bias
        o = {m: st.forward(x.to(DEV), lg.to(DEV), K, True) for m, st in sts.items()}
        torch.cuda.synchronize()
        assert torch.equal(bits(o["paged"]), bits(o["resident"])), (t, T)
        w_ref, ids_ref = route(lg, K)
        res = ora.forward(ids_ref.tolist())
        pst = sts["paged"]
        if T:
            w_gpu, ids_gpu = pst.last_topk
            assert ids_gpu.cpu().numpy().tolist() == ids_ref.tolist(), (t, T)
            assert np.allclose(w_gpu.cpu().numpy(), w_ref, rtol=2e-6, atol=1e-7), (t, T)
            rec = parse_record(pst.last_record.numpy(), T, K)
            oracle_trace_matches(res, rec)
            assert pst.last_slots.cpu().tolist() == res["slots"], (t, T)
            xs.append(x)
            lgs.append(lg)
            outs.append(o["paged"].cpu())
        assert pst.slot_to_expert == ora.slot_to_expert and pst.lru_tick == ora.lru_tick, (t, T)
    assert (pst.stats_forward, pst.stats_miss, pst.stats_evict, pst.stats_hits) == \
        (ora.stats_forward, ora.stats_miss, ora.stats_evict, ora.stats_hits)
    oracle_check(xs, lgs, outs, K, w13, w2, 1e-2, label="mixed sizes")


def test_mixed_sizes_with_resizes_and_prefetches():
    """Calls of 0 to 70 tokens on one paged layer whose scratch is resized
    between calls (32 -> 48 -> 70 -> 16 -> 64 -> 8 slots: the pager's register
    path up to 64 slots, its LDS path above) and which takes speculative
    prefetches between calls: after every call and prefetch the slot table,
    ticks, clock and counters equal the oracle's, and every output's bytes
    equal a resident layer's."""
    sh = W.LayerShape(256, 128, 128, 8, 32, torch.bfloat16)
    g = torch.Generator().manual_seed(23)
    slabs = W.alloc_slabs(sh, pin=True)
    W.fill_expert_weights(slabs, sh, g)
    w13, w2 = W.slab_views(slabs, sh)
    st = WispMoEState(w13, w2, sh.cap, "paged", DEV, 0)
    res = WispMoEState(w13, w2, sh.experts, "resident", DEV, 1)
    res.prime_identity()
    ora = PagerOracle(sh.experts, sh.cap)
    K = sh.top_k
    rng = np.random.default_rng(29)
    bias = torch.from_numpy(rng.normal(0.0, 1.5, sh.experts).astype(np.float32))
    sizes = [1, 3, 8, 1, 40, 1, 0, 12, 1, 70, 2, 1, 33, 1, 5, 64, 1, 9, 1, 20, 1, 4]
    resizes = {5: 48, 9: 70, 13: 16, 17: 64, 20: 8}
    prefetches = {3, 8, 12, 16, 19, 21}

    def check(label):
        assert st.slot_to_expert == ora.slot_to_expert, label
        assert st.lru_tick == ora.lru_tick and st.lru_clock == ora.lru_clock, label
        assert (st.stats_forward, st.stats_miss, st.stats_evict, st.stats_hits) == \
            (ora.stats_forward, ora.stats_miss, ora.stats_evict, ora.stats_hits), label

    for t, T in enumerate(sizes):
        if t in resizes:
            torch.cuda.synchronize()
            st.resize_cap(resizes[t])
            ora.resize_cap(resizes[t])
            assert st.cap_experts == ora.cap_experts
            check(("resize", t))
        if t in prefetches:
            pred = set(int(e) for e in rng.choice(sh.experts, 6, replace=False))
            st.prefetch_async(list(pred))
            ora.prefetch_async(pred)
            torch.cuda.synchronize()
            check(("prefetch", t))
        x = torch.randn((T, sh.hidden), generator=g).to(sh.dtype)
        lg = torch.randn((T, sh.experts), generator=g) + bias
        out = st.forward(x.to(DEV), lg.to(DEV), K, True)
        ref = res.forward(x.to(DEV), lg.to(DEV), K, True)
        ora.forward(route(lg, K)[1].tolist() if T else [])
        torch.cuda.synchronize()
        assert torch.equal(bits(out), bits(ref)), (t, T)
        check((t, T))


@pytest.mark.parametrize("fused", ["0", "1"])
def test_bfloat16_router_logits(monkeypatch, fused):
    """Router logits in bfloat16, as a bf16 model hands them over: the routing
    fused into the pager (one-token instance, general instance, and with
    WISP_DECODE_FUSED=1 the fused decode launch at cap == top-k) and the
    routing kernel (more than 8 tokens) read them as their exact float32
    values, so ids, weights and decisions equal the oracle's on those values
    and paged bytes equal a resident layer's."""
    monkeypatch.setenv("WISP_DECODE_FUSED", fused)
    # H = 1024: rows of two 16-byte chunks per lane, a shape the fused decode
    # launch serves
    sh = W.LayerShape(1024, 128, 128, 8, 8, torch.bfloat16)
    g = torch.Generator().manual_seed(31)
    slabs = W.alloc_slabs(sh, pin=True)
    W.fill_expert_weights(slabs, sh, g)
    w13, w2 = W.slab_views(slabs, sh)
    caps = {"decode": sh.cap, "batch": 32}
    sts = {k: WispMoEState(w13, w2, c, "paged", DEV, 0) for k, c in caps.items()}
    res = WispMoEState(w13, w2, sh.experts, "resident", DEV, 1)
    res.prime_identity()
    oras = {k: PagerOracle(sh.experts, c) for k, c in caps.items()}
    K = sh.top_k
    sizes = {"decode": [1] * 12, "batch": [1, 5, 1, 8, 20, 1, 3, 40]}
    for key, seq in sizes.items():
        st, ora = sts[key], oras[key]
        for t, T in enumerate(seq):
            x = torch.randn((T, sh.hidden), generator=g).to(sh.dtype)
            lg = (torch.randn((T, sh.experts), generator=g) * 2.0).to(torch.bfloat16)
            out = st.forward(x.to(DEV), lg.to(DEV), K, True)
            ref = res.forward(x.to(DEV), lg.to(DEV), K, True)
            w_ref, ids_ref = route(lg.float(), K)
            ora_res = ora.forward(ids_ref.tolist())
            torch.cuda.synchronize()
            assert torch.equal(bits(out), bits(ref)), (key, t, T)
            w_gpu, ids_gpu = st.last_topk
            assert ids_gpu.cpu().numpy().tolist() == ids_ref.tolist(), (key, t, T)
            assert np.allclose(w_gpu.cpu().numpy(), w_ref, rtol=2e-6, atol=1e-7), (key, t, T)
            assert st.last_slots.cpu().tolist() == ora_res["slots"], (key, t, T)
            assert st.slot_to_expert == ora.slot_to_expert and st.lru_tick == ora.lru_tick
