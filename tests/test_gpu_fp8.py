"""Block-FP8 paged path on the GPU: the activation quantiser bit-exact with the
oracle, the expert kernels within the bf16 tolerance of the oracle's
restatement of vLLM's w8a8 block math (oracle/fp8.py), outputs independent
of slot placement and batching (byte-identical), pager decisions of the FP8
state bit-exact with the reference pager, and the FP8 plug-in surface."""
import ctypes as C

import numpy as np
import pytest
import torch

from oracle import fp8 as F
from oracle.moe import route
from oracle.pager import PagerOracle
from wisp_amd import _lib
from wisp_amd import workloads as W
from wisp.integrations.vllm import fused_moe_fp8 as f8m
from wisp.integrations.vllm.fused_moe_fp8 import WispMoEStateFP8, fp8_slab_masters

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
# bf16 outputs: the tolerance the paged path is held to
REL_TOL = 1e-2


def _rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def _experts(E, H, I, block, seed=0, gain=True):
    """Host slabs of E block-FP8 experts with block scales that differ by up
    to 16x between blocks."""
    buf, w13, w2, s13, s2 = fp8_slab_masters(E, H, I, block, pin=False)
    g = torch.Generator().manual_seed(seed)
    bn, bk = block
    for e in range(E):
        for dst, sdst, shape in ((w13, s13, (2 * I, H)), (w2, s2, (H, I))):
            w = torch.randn(shape, generator=g) * 0.05
            if gain:
                gb = 2.0 ** (torch.rand((shape[0] // bn, shape[1] // bk), generator=g) * 4 - 2)
                w = w * gb.repeat_interleave(bn, 0).repeat_interleave(bk, 1)
            q, s = W.block_quant_fp8(w, block)
            dst[e].copy_(q)
            sdst[e].copy_(s)
    return buf, w13, w2, s13, s2


def _rows(t, idx):
    """Rows ``idx`` of a CPU tensor (fp8 through its bytes)."""
    idx = torch.as_tensor(np.asarray(idx, dtype=np.int64))
    if t.dtype == torch.float8_e4m3fn:
        return t.view(torch.uint8)[idx].view(t.dtype)
    return t[idx]


def _routing(T, E, K, seed):
    rng = np.random.default_rng(seed)
    ids = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int32)
    w = rng.uniform(0.05, 1.0, (T, K)).astype(np.float32)
    return ids, w


def _run_experts(x, ids, tw, w13, w2, s13, s2, block, slots=None, nslots=None,
                 algo=_lib.WISP_ALGO_GEMV):
    """wisp_moe_experts_fp8 through the C ABI on device copies; returns
    (out, act) as float32 CPU tensors."""
    T, H = x.shape
    K = ids.shape[1]
    E, I = w13.shape[0], w2.shape[2]
    d13, d2 = w13.to(DEV), w2.to(DEV)
    ds13, ds2 = s13.to(DEV), s2.to(DEV)
    sl = torch.from_numpy(ids if slots is None else slots).to(DEV).contiguous()
    twd = torch.from_numpy(tw).to(DEV).contiguous()
    xd = x.to(DEV).contiguous()
    act = torch.full((max(1, T * K), I), float("nan"), dtype=torch.bfloat16, device=DEV)
    out = torch.empty((T, H), dtype=torch.bfloat16, device=DEV)
    ns = E if nslots is None else nslots
    nbytes = _lib.lib().wisp_moe_fp8_work_bytes(max(1, T), K, H, I, ns)
    work = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
    rc = _lib.lib().wisp_moe_experts_fp8(
        xd.data_ptr(), T, H, I, K, twd.data_ptr(), sl.data_ptr(), ns,
        d13.data_ptr(), d13.stride(0), ds13.data_ptr(), ds13.stride(0), d2.data_ptr(),
        d2.stride(0), ds2.data_ptr(), ds2.stride(0), block[0], block[1], act.data_ptr(),
        out.data_ptr(), work.data_ptr(), nbytes, algo, _lib.stream_handle())
    _lib.check(rc, "wisp_moe_experts_fp8")
    torch.cuda.synchronize()
    return out.float().cpu(), act.float().cpu().view(T, K, I)


def test_quant_groups_bit_exact():
    g = torch.Generator().manual_seed(1)
    x = torch.randn((37, 1024), generator=g) * torch.logspace(-3, 3, 37).view(37, 1)
    x[5, 256:384] = 0.0
    x[6, :128] = 448.0
    for dt, code in ((torch.bfloat16, _lib.WISP_BF16), (torch.float32, _lib.WISP_F32)):
        xd = x.to(dt).to(DEV).contiguous()
        q = torch.empty((37, 1024), dtype=torch.uint8, device=DEV)
        s = torch.empty((37, 8), dtype=torch.float32, device=DEV)
        _lib.check(_lib.lib().wisp_quant_fp8_groups(xd.data_ptr(), code, 37, 1024, 128,
                                                    q.data_ptr(), s.data_ptr(),
                                                    _lib.stream_handle()), "quant")
        torch.cuda.synchronize()
        wq, ws = F.quant_groups(xd.float().cpu().numpy(), 128)
        assert np.array_equal(q.cpu().numpy(), wq), dt
        assert np.array_equal(s.cpu().numpy(), ws), dt


SHAPES = [  # T, H, I, E, K, block
    (1, 2048, 768, 12, 8, (128, 128)),   # Qwen3-30B-A3B-FP8 decode shape, fewer experts
    (3, 256, 256, 8, 2, (128, 128)),     # K = 2: bf16 adds in moe_sum
    (4, 1024, 384, 10, 3, (64, 128)),    # block_n 64, K = 3
    (2, 4096, 256, 6, 1, (128, 128)),    # eight w13 waves, K = 1
    (9, 512, 256, 12, 6, (128, 128)),    # batch of 9, shared experts
]


@pytest.mark.parametrize("T,H,I,E,K,block", SHAPES)
def test_experts_fp8_match_oracle(T, H, I, E, K, block):
    _, w13, w2, s13, s2 = _experts(E, H, I, block, seed=T * 31 + K)
    ids, tw = _routing(T, E, K, seed=T + H)
    x = (torch.randn((T, H), generator=torch.Generator().manual_seed(5)) * 2).to(torch.bfloat16)
    out, act = _run_experts(x, ids, tw, w13, w2, s13, s2, block)
    want, want_act = F.moe_forward_fp8(x, tw, ids, w13, w2, s13, s2, block, return_act=True)
    assert _rel(act, want_act) < REL_TOL
    # the MFMA's own rounding moves a few bf16 ulps; most act values are equal
    same = float(np.mean(act.numpy() == want_act))
    assert same > 0.95, same
    assert _rel(out, want) < REL_TOL, _rel(out, want)


ALGOS = [pytest.param(_lib.WISP_ALGO_GEMV, id="decode"),
         pytest.param(_lib.WISP_ALGO_MFMA, id="grouped")]


@pytest.mark.parametrize("algo", ALGOS)
def test_experts_fp8_absent_slot_and_slot_placement(algo):
    T, H, I, E, K, block = 4, 512, 256, 10, 4, (128, 128)
    _, w13, w2, s13, s2 = _experts(E, H, I, block, seed=3)
    ids, tw = _routing(T, E, K, seed=4)
    x = torch.randn((T, H), generator=torch.Generator().manual_seed(6)).to(torch.bfloat16)
    base, _ = _run_experts(x, ids, tw, w13, w2, s13, s2, block, algo=algo)
    # the same experts at other slots: byte-identical
    perm = np.random.default_rng(7).permutation(E)
    inv = np.argsort(perm)
    moved, _ = _run_experts(x, ids, tw, _rows(w13, perm), _rows(w2, perm), _rows(s13, perm),
                            _rows(s2, perm), block, slots=inv[ids].astype(np.int32), algo=algo)
    assert torch.equal(base.view(torch.int32), moved.view(torch.int32))
    # a slot of -1 contributes nothing (vLLM's expert_map == -1)
    sl = ids.copy()
    sl[1, 2] = -1
    sl[3, 0] = -1
    got, _ = _run_experts(x, ids, tw, w13, w2, s13, s2, block, slots=sl, algo=algo)
    # oracle: the absent pairs route to an extra expert the map marks absent
    ext = list(range(E)) + [0]
    emap = np.concatenate([np.zeros(E, np.int32), [-1]])
    want = F.moe_forward_fp8(x, tw, np.where(sl < 0, E, ids), _rows(w13, ext), _rows(w2, ext),
                             _rows(s13, ext), _rows(s2, ext), block, expert_map=emap)
    assert _rel(got, want) < REL_TOL


def test_experts_fp8_one_token_absent_slots():
    """One-token calls run their own w13 kernel: a slot of -1 or past the
    scratch contributes nothing there too, with the act rows of those pairs
    zero, and the other pairs keep the bytes of the full call."""
    T, H, I, E, K, block = 1, 1024, 384, 10, 5, (128, 128)
    _, w13, w2, s13, s2 = _experts(E, H, I, block, seed=11)
    ids, tw = _routing(T, E, K, seed=12)
    x = torch.randn((T, H), generator=torch.Generator().manual_seed(13)).to(torch.bfloat16)
    full, full_act = _run_experts(x, ids, tw, w13, w2, s13, s2, block)
    sl = ids.copy()
    sl[0, 1] = -1
    sl[0, 3] = E + 2  # past the nslots = E slots of the scratch
    got, act = _run_experts(x, ids, tw, w13, w2, s13, s2, block, slots=sl)
    assert torch.count_nonzero(act[0, 1]) == 0 and torch.count_nonzero(act[0, 3]) == 0
    for k in (0, 2, 4):
        assert torch.equal(act[0, k].view(torch.int32), full_act[0, k].view(torch.int32)), k
    ext = list(range(E)) + [0]
    emap = np.concatenate([np.zeros(E, np.int32), [-1]])
    absent = (sl < 0) | (sl >= E)
    want = F.moe_forward_fp8(x, tw, np.where(absent, E, ids), _rows(w13, ext), _rows(w2, ext),
                             _rows(s13, ext), _rows(s2, ext), block, expert_map=emap)
    assert _rel(got, want) < REL_TOL


@pytest.mark.parametrize("algo", ALGOS)
def test_experts_fp8_batching_is_byte_invariant(algo):
    """A token's output does not depend on the other tokens of the launch
    (MFMA columns are independent), so grouping never changes bytes."""
    T, H, I, E, K, block = 6, 1024, 512, 8, 4, (128, 128)
    _, w13, w2, s13, s2 = _experts(E, H, I, block, seed=8)
    ids, tw = _routing(T, E, K, seed=9)
    x = torch.randn((T, H), generator=torch.Generator().manual_seed(10)).to(torch.bfloat16)
    full, _ = _run_experts(x, ids, tw, w13, w2, s13, s2, block, algo=algo)
    for t in range(T):
        one, _ = _run_experts(x[t:t + 1], ids[t:t + 1], tw[t:t + 1], w13, w2, s13, s2, block,
                              algo=algo)
        assert torch.equal(one[0].view(torch.int32), full[t].view(torch.int32)), t
    halves = [_run_experts(x[a:b], ids[a:b], tw[a:b], w13, w2, s13, s2, block, algo=algo)[0]
              for a, b in ((0, 2), (2, 6))]
    assert torch.equal(torch.cat(halves).view(torch.int32), full.view(torch.int32))


GROUPED = [  # T, H, I, E, K, block: tile widths 1, 2 and 4 per pass, odd k-block counts;
    # w2 blocks of 4 (H a multiple of 512), 2 (H = 768) and 1 (H = 384) panels
    (16, 2048, 768, 32, 8, (128, 128)),
    (70, 1024, 384, 16, 4, (64, 128)),
    (200, 512, 256, 24, 8, (128, 128)),
    (40, 384, 640, 12, 2, (128, 128)),
    (33, 768, 256, 10, 4, (128, 128)),
]


@pytest.mark.parametrize("T,H,I,E,K,block", GROUPED)
def test_experts_fp8_grouped_match_oracle(T, H, I, E, K, block):
    _, w13, w2, s13, s2 = _experts(E, H, I, block, seed=T + 1)
    ids, tw = _routing(T, E, K, seed=T + 2)
    x = torch.randn((T, H), generator=torch.Generator().manual_seed(T)).to(torch.bfloat16)
    out, act = _run_experts(x, ids, tw, w13, w2, s13, s2, block, algo=_lib.WISP_ALGO_MFMA)
    want, want_act = F.moe_forward_fp8(x, tw, ids, w13, w2, s13, s2, block, return_act=True)
    assert _rel(act, want_act) < REL_TOL
    assert float(np.mean(act.numpy() == want_act)) > 0.95
    assert _rel(out, want) < REL_TOL, _rel(out, want)


@pytest.mark.parametrize("H,I,block", [(1024, 384, (64, 128)), (768, 256, (128, 128)),
                                         (384, 640, (128, 128))])
def test_experts_fp8_grouped_bytes_equal_across_kernel_families(H, I, block):
    """Above 16 tokens the grouped path runs the LDS-staged kernels, up to 16
    the register-streaming ones; both take each output through the same
    k-block steps, so one call over 48 tokens, two of 24 and chunks of 8 or
    16 give the same bytes for every token (w2 blocks of 4, 2 and 1 panels
    for H = 1024, 768 and 384)."""
    T, E, K = 48, 12, 4
    _, w13, w2, s13, s2 = _experts(E, H, I, block, seed=21)
    ids, tw = _routing(T, E, K, seed=22)
    x = torch.randn((T, H), generator=torch.Generator().manual_seed(23)).to(torch.bfloat16)
    mfma = _lib.WISP_ALGO_MFMA
    full, full_act = _run_experts(x, ids, tw, w13, w2, s13, s2, block, algo=mfma)
    for step in (24, 16, 8):
        parts = [_run_experts(x[a:a + step], ids[a:a + step], tw[a:a + step], w13, w2, s13, s2,
                              block, algo=mfma)[0] for a in range(0, T, step)]
        assert torch.equal(torch.cat(parts).view(torch.int32), full.view(torch.int32)), step
    want, want_act = F.moe_forward_fp8(x, tw, ids, w13, w2, s13, s2, block, return_act=True)
    assert _rel(full_act, want_act) < REL_TOL and _rel(full, want) < REL_TOL


def test_experts_fp8_decode_kernels_over_256_pairs():
    """The decode kernels' in-memory slot scan (launches of more than 256
    pairs) against the oracle."""
    T, H, I, E, K, block = 40, 512, 256, 16, 8, (128, 128)
    _, w13, w2, s13, s2 = _experts(E, H, I, block, seed=21)
    ids, tw = _routing(T, E, K, seed=22)
    x = torch.randn((T, H), generator=torch.Generator().manual_seed(23)).to(torch.bfloat16)
    out, _ = _run_experts(x, ids, tw, w13, w2, s13, s2, block, algo=_lib.WISP_ALGO_GEMV)
    want = F.moe_forward_fp8(x, tw, ids, w13, w2, s13, s2, block)
    assert _rel(out, want) < REL_TOL


def _fp8_state(wl, cap):
    w13, w2, s13, s2 = wl.views()
    return WispMoEStateFP8(w13, w2, s13, s2, cap, DEV, 0)


@pytest.fixture(scope="module")
def small_fp8():
    """Qwen3-shaped block-FP8 layer with 32 experts, 48 decode steps, pinned."""
    base = W.qwen3_decode(seed=2, steps=48, weights=False)
    base.logits = base.logits[:, :, :32].contiguous()
    return W.fp8_layer(base, pin=True, experts=32)


@pytest.mark.parametrize("engine,cap", [("kernel", 8), ("memcpy", 8), ("kernel", 12)])
def test_fp8_state_decode_matches_oracle(monkeypatch, small_fp8, engine, cap):
    """Decode steps through cap slots: decisions equal the oracle's, outputs
    the bytes of a cap=E state and, sampled, the oracle's within tolerance.
    On the copy-kernel engine one launch pages in and runs w13: loaded
    experts computed by the copy blocks from the codes they copy, the others
    by w13 blocks laid out by slot (cap == top-k) or by pair (cap 12)."""
    monkeypatch.setenv("WISP_PAGEIN_ENGINE", engine)
    wl = small_fp8
    E, K = 32, wl.shape.top_k
    st = _fp8_state(wl, cap)
    assert st.pagein_engine == engine
    full = _fp8_state(wl, E)
    ora = PagerOracle(E, cap)
    w13, w2, s13, s2 = wl.views()
    for t in range(wl.steps):
        x, lg = wl.x[t].to(DEV), wl.logits[t].to(DEV)
        out = st.forward(x, lg, K, True)
        ref = full.forward(x, lg, K, True)
        res = ora.forward(route(wl.logits[t], K)[1].tolist())
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), t
        assert st.slot_to_expert == ora.slot_to_expert and st.lru_tick == ora.lru_tick, t
        assert (st.stats_miss, st.stats_evict, st.stats_hits) == \
            (ora.stats_miss, ora.stats_evict, ora.stats_hits), t
        if t % 16 == 0:
            tw, ids = route(wl.logits[t], K)
            want = F.moe_forward_fp8(wl.x[t], tw.astype(np.float32), ids, w13, w2, s13, s2)
            assert _rel(out.float().cpu(), want) < REL_TOL, t
    assert ora.stats_miss > cap  # the trace pages


def test_fp8_state_empty_calls_tick_the_clock(small_fp8):
    """Zero-token calls between decode steps: empty output, the pager moves
    as the reference's empty call does, and the next calls still match the
    oracle and the resident layer's bytes."""
    wl = small_fp8
    E, K, cap = 32, wl.shape.top_k, 8
    st, full = _fp8_state(wl, cap), _fp8_state(wl, E)
    ora = PagerOracle(E, cap)
    x0 = torch.empty((0, wl.shape.hidden), dtype=torch.bfloat16, device=DEV)
    lg0 = torch.empty((0, E), dtype=torch.float32, device=DEV)
    for t in range(8):
        if t % 2:
            out0 = st.forward(x0, lg0, K, True)
            torch.cuda.synchronize()
            assert tuple(out0.shape) == (0, wl.shape.hidden)
            ora.forward([])
        x, lg = wl.x[t].to(DEV), wl.logits[t].to(DEV)
        out = st.forward(x, lg, K, True)
        ref = full.forward(x, lg, K, True)
        ora.forward(route(wl.logits[t], K)[1].tolist())
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), t
        assert st.slot_to_expert == ora.slot_to_expert and st.lru_tick == ora.lru_tick, t
        assert st.lru_clock == ora.lru_clock and st.stats_forward == ora.stats_forward, t


def test_fp8_state_subbatches_like_the_reference(small_fp8):
    """A batch whose experts overflow cap runs as greedy token groups."""
    wl = small_fp8
    E, K, cap = 32, wl.shape.top_k, 12
    st = _fp8_state(wl, cap)
    full = _fp8_state(wl, E)
    ora = PagerOracle(E, cap)
    x = wl.x[:6, 0].to(DEV)
    lg = wl.logits[:6, 0].to(DEV)
    out = st.forward(x, lg, K, True)
    ref = full.forward(x, lg, K, True)
    res = ora.forward(route(wl.logits[:6, 0], K)[1].tolist())
    torch.cuda.synchronize()
    assert len(res["groups"]) > 1
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    assert st.slot_to_expert == ora.slot_to_expert and st.lru_tick == ora.lru_tick


@pytest.fixture(scope="module")
def full_fp8():
    """The Qwen3-30B-A3B-FP8 layer at full size (128 experts), one 512-token
    chunk with router logits ~N(0, 1), pinned masters."""
    return W.fp8_layer(W.gaussian_logits("batch", seed=5, steps=1, tokens=512, weights=False),
                       pin=True)


def test_fp8_state_full_size_chunk_and_batches(full_fp8):
    """At the full Qwen3-FP8 shape: the 512-token chunk through cap=32 (~4-token
    groups on the register-streaming kernels) and through cap=E (one group on
    the LDS-staged kernels, w2 blocks of four 128-row panels) give the same
    bytes; decisions equal the reference pager's; sampled tokens match the
    oracle.  Then two bs=32 steps, from the chunk's tokens, the same way."""
    wl = full_fp8
    E, K, cap = 128, wl.shape.top_k, 32
    st = _fp8_state(wl, cap)
    full = _fp8_state(wl, E)
    ora = PagerOracle(E, cap)
    w13, w2, s13, s2 = wl.views()
    x, lg = wl.x[0].to(DEV), wl.logits[0].to(DEV)
    out = st.forward(x, lg, K, True)
    ref = full.forward(x, lg, K, True)
    res = ora.forward(route(wl.logits[0], K)[1].tolist())
    torch.cuda.synchronize()
    assert len(res["groups"]) > 100
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    assert st.slot_to_expert == ora.slot_to_expert and st.lru_tick == ora.lru_tick
    tw, ids = route(wl.logits[0], K)
    pick = [0, 1, 77, 200, 311, 450, 510, 511]
    want = F.moe_forward_fp8(wl.x[0][pick], tw[pick].astype(np.float32), ids[pick],
                             w13, w2, s13, s2)
    assert _rel(out[pick].float().cpu(), want) < REL_TOL
    for a in (0, 32):
        out = st.forward(x[a:a + 32], lg[a:a + 32], K, True)
        ref = full.forward(x[a:a + 32], lg[a:a + 32], K, True)
        ora.forward(route(wl.logits[0][a:a + 32], K)[1].tolist())
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), a
        assert st.slot_to_expert == ora.slot_to_expert and st.lru_tick == ora.lru_tick, a
        assert (st.stats_miss, st.stats_evict, st.stats_hits) == \
            (ora.stats_miss, ora.stats_evict, ora.stats_hits), a


def _max_rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


@pytest.mark.parametrize("tokens", [600, 1024])
def test_fp8_state_chunk_above_the_staged_id_limit(tokens):
    """Block-FP8 prefill chunks of more than 4096 (token, k) pairs at the full
    Qwen3-FP8 shape: the pager reads the routed ids from global memory and
    mirrors its device record to the host record.  Cap 32 (~tokens/4 token
    groups) and cap = E (one group): each state's decisions, slot table and
    ticks equal its own oracle pager's, the two give the same bytes, and
    sampled rows are within 1e-2 of oracle/fp8.py in both the L2 and the max
    norm.  A bs=32 call follows on both states."""
    wl = W.fp8_layer(W.gaussian_logits("batch", seed=21 + tokens, steps=1, tokens=tokens,
                                       weights=False), pin=True)
    E, K = 128, wl.shape.top_k
    assert tokens * K > 4096
    sts = {cap: _fp8_state(wl, cap) for cap in (32, E)}
    oras = {cap: PagerOracle(E, cap) for cap in (32, E)}
    w13, w2, s13, s2 = wl.views()
    x, lg = wl.x[0], wl.logits[0]
    for i, (xc, lgc) in enumerate([(x, lg), (x[:32], lg[:32])]):
        print(f"fp8 chunk {tokens} call {i}: {xc.shape[0]} tokens", flush=True)
        outs = {cap: st.forward(xc.to(DEV), lgc.to(DEV), K, True) for cap, st in sts.items()}
        torch.cuda.synchronize()
        assert torch.equal(outs[32].view(torch.int16), outs[E].view(torch.int16)), i
        if i == 0:
            first = outs[32].float().cpu()
        ids = route(lgc, K)[1].tolist()
        for cap, st in sts.items():
            res = oras[cap].forward(ids)
            ora = oras[cap]
            if i == 0:
                assert (len(res["groups"]) > tokens // 8) == (cap < E)
            assert st.slot_to_expert == ora.slot_to_expert and st.lru_tick == ora.lru_tick
            assert (st.stats_miss, st.stats_evict, st.stats_hits) == \
                (ora.stats_miss, ora.stats_evict, ora.stats_hits), (i, cap)
    tw, ids = route(lg, K)
    pick = [0, 1, 63, 64, 255, 256, 511, 512, tokens // 2 + 3, tokens - 1]
    want = F.moe_forward_fp8(x[pick], tw[pick].astype(np.float32), ids[pick], w13, w2, s13, s2)
    got = first[pick]
    assert _rel(got, want) < REL_TOL
    for r in range(len(pick)):
        assert _max_rel(got[r], want[r]) < REL_TOL, pick[r]


def test_fp8_state_prefill_paged_equals_full(small_fp8):
    """A 64-token prefill chunk (grouped path) through cap=16: token groups,
    each group's experts paged in; bytes equal the cap=E run and decisions
    equal the reference pager's."""
    wl = small_fp8
    E, K, cap = 32, wl.shape.top_k, 16
    st = _fp8_state(wl, cap)
    full = _fp8_state(wl, E)
    ora = PagerOracle(E, cap)
    x = wl.x[:, 0].repeat(2, 1)[:64].contiguous().to(DEV)    # 48 steps, twice
    lg = wl.logits[:, 0].repeat(2, 1)[:64].contiguous().to(DEV)
    out = st.forward(x, lg, K, True)
    ref = full.forward(x, lg, K, True)
    res = ora.forward(route(lg.cpu(), K)[1].tolist())
    torch.cuda.synchronize()
    assert len(res["groups"]) > 1
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    assert st.slot_to_expert == ora.slot_to_expert and st.lru_tick == ora.lru_tick
    w13, w2, s13, s2 = wl.views()
    tw, ids = route(lg.cpu(), K)
    want = F.moe_forward_fp8(x.cpu(), tw.astype(np.float32), ids, w13, w2, s13, s2)
    assert _rel(out.float().cpu(), want) < REL_TOL


def test_fp8_cap_clamp_above_num_experts(monkeypatch):
    """WISP_CAP_EXPERTS=2 with E=4 clamps to 8 slots (> E); the misses take
    the top free slots, as in the reference."""
    H, I, E, K = 256, 256, 4, 2
    _, w13, w2, s13, s2 = _experts(E, H, I, (128, 128), seed=11)
    monkeypatch.setenv("WISP_CAP_EXPERTS", "2")
    cap = f8m._resolve_cap_experts(E)
    assert cap == 8
    st = WispMoEStateFP8(w13, w2, s13, s2, cap, DEV, 0)
    ora = PagerOracle(E, cap)
    g = torch.Generator().manual_seed(12)
    for t in range(6):
        lg = torch.randn((1, E), generator=g)
        x = torch.randn((1, H), generator=g).to(torch.bfloat16)
        st.forward(x.to(DEV), lg.to(DEV), K, True)
        ora.forward(route(lg, K)[1].tolist())
        torch.cuda.synchronize()
        assert st.slot_to_expert == ora.slot_to_expert, t
    n = sum(e >= 0 for e in st.slot_to_expert)
    assert n >= K and st.slot_to_expert[:cap - n] == [-1] * (cap - n)


def test_install_wisp_fp8_standin_layer_matches_resident():
    from wisp.integrations.vllm.layer import Fp8FusedMoE, Fp8MoEMethod
    E, H, I, K, block = 16, 512, 256, 4, (128, 128)
    _, w13, w2, s13, s2 = _experts(E, H, I, block, seed=13)
    g = torch.Generator().manual_seed(14)
    x = torch.randn((3, H), generator=g).to(torch.bfloat16).to(DEV)
    lg = torch.randn((3, E), generator=g).to(DEV)
    names = ("create_weights", "process_weights_after_loading", "apply")
    saved = {n: Fp8MoEMethod.__dict__[n] for n in names}
    was_patched = getattr(Fp8MoEMethod, f8m._PATCHED_FLAG, False)
    if was_patched:  # an earlier install_wisp_moe() also patched the FP8 method
        for n in names:
            setattr(Fp8MoEMethod, n, getattr(Fp8MoEMethod, "_wisp_original_" + n))
        delattr(Fp8MoEMethod, f8m._PATCHED_FLAG)
    try:
        plain = Fp8FusedMoE(E, K, H, I, block)  # unpatched: every expert on the GPU
        plain.load_weights(w13, w2, s13, s2)
        plain.process_weights_after_loading()
        ref = plain(x, lg)
        assert f8m.install_wisp_fp8() and f8m.is_fp8_installed()
        assert not f8m.install_wisp_fp8()  # idempotent
        paged = Fp8FusedMoE(E, K, H, I, block)
        assert paged.w13_weight.device.type == "cpu" and paged.w13_weight.is_pinned()
        paged.load_weights(w13, w2, s13, s2)
        paged.process_weights_after_loading()
        st = paged._wisp_fp8_state
        assert st.cap_experts == min(E, 24) and st.pagein_engine == "kernel"
        assert paged.w13_weight.numel() == 0  # device placeholder
        out = paged(x, lg)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
        with pytest.raises(NotImplementedError):
            paged.quant_method.apply(paged, x, lg, K, True, expert_map=torch.zeros(E))
    finally:
        for n, f in saved.items():
            setattr(Fp8MoEMethod, n, f)
        if was_patched:
            setattr(Fp8MoEMethod, f8m._PATCHED_FLAG, True)
        elif hasattr(Fp8MoEMethod, f8m._PATCHED_FLAG):
            delattr(Fp8MoEMethod, f8m._PATCHED_FLAG)
        f8m._FP8_LAYER_STATES.clear()


def test_fp8_state_from_weights_loaded_outside_the_slab():
    """A block-FP8 layer whose parameters were created by the unpatched
    create_weights (four separate tensors) gets its masters copied into one
    pinned slab by the patched process_weights_after_loading; its outputs
    equal the unpatched resident layer's bytes."""
    from wisp.integrations.vllm.layer import Fp8FusedMoE, Fp8MoEMethod
    E, H, I, K, block = 16, 512, 256, 4, (128, 128)
    _, w13, w2, s13, s2 = _experts(E, H, I, block, seed=17)
    g = torch.Generator().manual_seed(18)
    x = torch.randn((3, H), generator=g).to(torch.bfloat16).to(DEV)
    lg = torch.randn((3, E), generator=g).to(DEV)
    names = ("create_weights", "process_weights_after_loading", "apply")
    saved = {n: Fp8MoEMethod.__dict__[n] for n in names}
    if getattr(Fp8MoEMethod, f8m._PATCHED_FLAG, False):  # build the layers unpatched
        for n in names:
            setattr(Fp8MoEMethod, n, getattr(Fp8MoEMethod, "_wisp_original_" + n))
    try:
        ref_layer = Fp8FusedMoE(E, K, H, I, block)  # every expert on the GPU
        ref_layer.load_weights(w13, w2, s13, s2)
        ref_layer.process_weights_after_loading()
        ref = ref_layer(x, lg)
        plain = Fp8FusedMoE(E, K, H, I, block)
        plain.load_weights(w13, w2, s13, s2)
        assert not hasattr(plain, "_wisp_fp8_slab")
        f8m._patched_process_weights_after_loading(plain.quant_method, plain)
        st = plain._wisp_fp8_state
        assert plain._wisp_fp8_slab.is_pinned() and st.pagein_engine == "kernel"
        assert plain.w13_weight.numel() == 0
        out = f8m._patched_apply(plain.quant_method, plain, x, lg, K, True)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    finally:
        for n, fn in saved.items():
            setattr(Fp8MoEMethod, n, fn)
        f8m._FP8_LAYER_STATES.clear()


@pytest.mark.parametrize("engine,logits_dtype", [("kernel", torch.float32),
                                                  ("memcpy", torch.float32),
                                                  ("kernel", torch.bfloat16)])
def test_fp8_state_calls_of_mixed_sizes(monkeypatch, small_fp8, engine, logits_dtype):
    """Calls of 0 to 64 tokens in a seeded order on one block-FP8 state (cap 8,
    every one-token call fills the scratch) and on a cap=E state: the
    one-token fused page-in launch, the decode kernels and the grouped
    kernels follow each other on the same scratch and pager (both page-in
    engines; float32 and bfloat16 router logits).  Every call: bytes equal to
    the cap=E state's, decisions and state equal to the oracle's; sampled
    outputs within the bf16 tolerance of the oracle."""
    monkeypatch.setenv("WISP_PAGEIN_ENGINE", engine)
    wl = small_fp8
    E, K, cap, H = 32, wl.shape.top_k, 8, wl.shape.hidden
    st, full = _fp8_state(wl, cap), _fp8_state(wl, E)
    ora = PagerOracle(E, cap)
    w13, w2, s13, s2 = wl.views()
    g = torch.Generator().manual_seed(17)
    bias = torch.randn((E,), generator=g) * 1.5
    sizes = [1, 1, 8, 3, 40, 0, 1, 20, 5, 1, 64, 2, 1, 0, 13, 1]
    for t, T in enumerate(sizes):
        x = torch.randn((T, H), generator=g).to(torch.bfloat16)
        lg = (torch.randn((T, E), generator=g) + bias).to(logits_dtype)
        out = st.forward(x.to(DEV), lg.to(DEV), K, True)
        ref = full.forward(x.to(DEV), lg.to(DEV), K, True)
        lg = lg.float()
        ids = route(lg, K)[1].tolist() if T else []
        ora.forward(ids)
        torch.cuda.synchronize()
        assert tuple(out.shape) == (T, H), (t, T)
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), (t, T)
        assert st.slot_to_expert == ora.slot_to_expert and st.lru_tick == ora.lru_tick, (t, T)
        assert (st.stats_forward, st.stats_miss, st.stats_evict, st.stats_hits) == \
            (ora.stats_forward, ora.stats_miss, ora.stats_evict, ora.stats_hits), (t, T)
        if T and t % 3 == 0:
            tw, rid = route(lg, K)
            want = F.moe_forward_fp8(x, tw.astype(np.float32), rid, w13, w2, s13, s2)
            assert _rel(out.float().cpu(), want) < REL_TOL, (t, T)
