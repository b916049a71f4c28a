"""GPU parity of the HIP kernels against the oracle (runs on an MI355X).

Bars: routing ids and every pager decision bit-exact; fp32 outputs within
1e-5 and bf16 outputs within 1e-2 of the float64 oracle, measured as
max|gpu - oracle| / max|oracle| per call; paged output byte-identical to
resident output."""
import numpy as np
import pytest
import torch

from oracle.moe import moe_forward, route
from oracle.pager import PagerOracle
from tests._util import oracle_trace_matches
from wisp_amd import _lib
from wisp_amd.record import parse_record

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def rel_err(a: torch.Tensor, b: torch.Tensor) -> float:
    a, b = a.double().cpu(), b.double().cpu()
    return float((a - b).abs().max() / b.abs().max().clamp_min(1e-30))


def gpu_route(logits: torch.Tensor, K: int, renorm: bool = True):
    T, E = logits.shape
    lg = logits.to(DEV).contiguous()
    w = torch.empty((T, K), dtype=torch.float32, device=DEV)
    ids = torch.empty((T, K), dtype=torch.int32, device=DEV)
    dt = _lib.WISP_F32 if lg.dtype == torch.float32 else _lib.WISP_BF16
    _lib.check(_lib.lib().wisp_route_topk_softmax(lg.data_ptr(), dt, T, E, K, int(renorm),
                                                  w.data_ptr(), ids.data_ptr(), None,
                                                  _lib.stream_handle()), "route")
    torch.cuda.synchronize()
    return w.cpu(), ids.cpu()


@pytest.mark.parametrize("E,K", [(8, 2), (16, 2), (128, 8), (256, 8), (512, 16), (60, 4)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_route_matches_oracle(E, K, dtype):
    g = torch.Generator().manual_seed(E * 31 + K)
    logits = (torch.randn(97, E, generator=g) * 1.5).to(dtype)
    w, ids = gpu_route(logits, K)
    w_ref, ids_ref = route(logits.float(), K)
    assert ids.numpy().tolist() == ids_ref.tolist()
    assert np.allclose(w.numpy(), w_ref, rtol=2e-6, atol=1e-7)
    w2, _ = gpu_route(logits, K, renorm=False)
    w2_ref, _ = route(logits.float(), K, renormalize=False)
    assert np.allclose(w2.numpy(), w2_ref, rtol=2e-6, atol=1e-7)


def tie_logits(rng, T, E, K):
    """Router logits full of exact ties: values from a small set that holds
    both zeros (-0.0 ranks as +0.0), with some -inf entries, at least K finite
    per row (exact in float32 and bfloat16)."""
    vals = np.array([-2.0, -1.0, -0.0, 0.0, 1.0, 2.0, 3.0], dtype=np.float32)
    lg = rng.choice(vals, size=(T, E)).astype(np.float32)
    for t in range(T):
        n_inf = int(rng.integers(0, max(1, E - K)))
        lg[t, rng.choice(E, n_inf, replace=False)] = -np.inf
    return torch.from_numpy(lg)


@pytest.mark.parametrize("E,K", [(8, 2), (60, 4), (128, 8), (256, 8), (512, 16)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_route_ties_match_oracle(E, K, dtype):
    """Equal logits in several lanes (the router's second maximum over the
    ids' complements) and in one lane (its best of two), -0.0 against +0.0
    and -inf entries: ids exact (value descending, lower id first), weights
    within float32 rounding of the float64 oracle."""
    rng = np.random.default_rng(E * 13 + K)
    logits = tie_logits(rng, 64, E, K).to(dtype)
    w, ids = gpu_route(logits, K)
    w_ref, ids_ref = route(logits.float(), K)
    assert ids.numpy().tolist() == ids_ref.tolist()
    assert np.allclose(w.numpy(), w_ref, rtol=2e-6, atol=1e-7)


class DevPager:
    def __init__(self, E, cap):
        self.E, self.cap = E, cap
        self.map = torch.full((E,), -1, dtype=torch.int32, device=DEV)
        self.s2e = torch.full((cap,), -1, dtype=torch.int32, device=DEV)
        self.tick = torch.zeros(cap, dtype=torch.int64, device=DEV)
        self.ctr = torch.zeros(8, dtype=torch.int64, device=DEV)

    def call(self, ids, K, single_group=False):
        t = torch.as_tensor(np.asarray(ids, dtype=np.int32).reshape(-1, K)).to(DEV)
        T = t.shape[0]
        words = _lib.lib().wisp_record_words(T, K)
        rec = torch.zeros(words, dtype=torch.int32, pin_memory=True)
        slots = torch.full((max(1, T * K),), -7, dtype=torch.int32, device=DEV)
        rc = _lib.lib().wisp_pager_decide(t.data_ptr() if T else None, T, K, self.E, self.cap,
                                          int(single_group), self.map.data_ptr(),
                                          self.s2e.data_ptr(), self.tick.data_ptr(),
                                          self.ctr.data_ptr(), slots.data_ptr(),
                                          rec.data_ptr(), words, _lib.stream_handle())
        assert rc == 0
        torch.cuda.synchronize()
        out = parse_record(rec.numpy(), T, K)
        out["slots"] = slots[: T * K].view(T, K).cpu().tolist() if T * K else []
        return out


@pytest.mark.parametrize("E,K,cap,tmax", [(8, 2, 4, 3), (16, 2, 4, 4), (128, 8, 8, 1),
                                           (128, 8, 24, 6), (128, 8, 32, 64), (8, 2, 2, 16),
                                           (512, 8, 64, 8), (100, 3, 7, 5), (256, 8, 100, 20),
                                           (512, 16, 300, 40),
                                           # the register path's edges: every lane a slot,
                                           # E <= 64 (one mask word pair), odd E and cap
                                           (128, 8, 64, 24), (64, 4, 64, 40), (100, 7, 63, 30),
                                           (128, 8, 65, 24),
                                           # the LDS path with top-k not a multiple of 4 (the
                                           # ids' 16-byte reads and stores fall back to words)
                                           (200, 3, 70, 30), (130, 5, 66, 40), (256, 6, 90, 50)])
def test_gpu_pager_matches_oracle(E, K, cap, tmax):
    rng = np.random.default_rng(E * 7 + cap)
    ora, dp = PagerOracle(E, cap), DevPager(E, cap)
    for step in range(80):
        T = int(rng.integers(0, tmax + 1))
        ids = [rng.choice(E, K, replace=False).tolist() for _ in range(T)]
        res = ora.forward(ids)
        rec = dp.call(ids, K)
        assert rec["status"] == 0, (step, rec)
        oracle_trace_matches(res, rec)
        assert rec["slots"] == res["slots"]
        assert dp.s2e.tolist() == ora.slot_to_expert
        assert dp.tick.tolist() == ora.lru_tick
        assert dp.map.tolist() == ora.expert_map()
        assert dp.ctr[:5].tolist() == [ora.lru_clock, ora.stats_forward, ora.stats_miss,
                                       ora.stats_evict, ora.stats_hits]


@pytest.mark.parametrize("E,K,cap,T", [(128, 8, 32, 520), (128, 8, 128, 1100),
                                        (128, 8, 64, 700), (512, 8, 64, 600),
                                        (200, 8, 100, 520), (256, 16, 300, 300),
                                        (300, 6, 150, 700)])
def test_gpu_pager_above_the_staged_id_limit(E, K, cap, T):
    """Calls of more than 4096 (token, k) pairs: the pager reads the routed
    ids from global memory and mirrors its device record to the host record
    at its end.  Register path (E <= 128, cap <= 64) and LDS path; greedy
    token groups (cap < E) and one group (cap = E).  Each call is followed by
    a small staged call on the same state; every decision, slot, tick and
    counter is checked against the oracle."""
    assert T * K > 4096
    rng = np.random.default_rng(E * 13 + cap + T)
    ora, dp = PagerOracle(E, cap), DevPager(E, cap)
    for step in range(6):
        n = T if step % 2 == 0 else int(rng.integers(1, 9))
        # skewed routing, so groups see hits as well as misses
        p = rng.dirichlet(np.full(E, 0.5))
        ids = [rng.choice(E, K, replace=False, p=p).tolist() for _ in range(n)]
        res = ora.forward(ids)
        rec = dp.call(ids, K)
        assert rec["status"] == 0, (step, rec["status"])
        oracle_trace_matches(res, rec)
        assert rec["slots"] == res["slots"], step
        assert dp.s2e.tolist() == ora.slot_to_expert, step
        assert dp.tick.tolist() == ora.lru_tick, step
        assert dp.map.tolist() == ora.expert_map(), step
        assert dp.ctr[:5].tolist() == [ora.lru_clock, ora.stats_forward, ora.stats_miss,
                                       ora.stats_evict, ora.stats_hits], step


def test_gpu_pager_overflow():
    dp = DevPager(8, 2)
    rec = dp.call([[0, 1, 1], [2, 3, 4]], 3)
    assert rec["status"] == _lib.WISP_ERR_SUBBATCH and rec["fail_group"] == 1
    ora = PagerOracle(8, 2)
    with pytest.raises(RuntimeError, match="sub-batch"):
        ora.forward([[0, 1, 1], [2, 3, 4]])
    assert dp.s2e.tolist() == ora.slot_to_expert and int(dp.ctr[4]) == ora.stats_hits
    # the completed group's pairs hold their slots; the failed group's are
    # written "not computed" (-1), not left at the buffer's initial -7
    m = dp.map.tolist()
    assert rec["slots"][0] == [m[0], m[1], m[1]] and min(rec["slots"][0]) >= 0
    assert rec["slots"][1] == [-1, -1, -1]


def test_gpu_pager_overflow_lds_path():
    """The same on the LDS path (E > 128): a group of one token that needs more
    experts than cap fails after the first group completed."""
    dp, ora = DevPager(200, 4), PagerOracle(200, 4)
    ids = [[0, 1, 2, 3, 0, 1, 2, 3], [10, 11, 12, 13, 14, 15, 16, 17]]
    rec = dp.call(ids, 8)
    assert rec["status"] == _lib.WISP_ERR_SUBBATCH and rec["fail_group"] == 1
    with pytest.raises(RuntimeError, match="sub-batch"):
        ora.forward(ids)
    assert dp.s2e.tolist() == ora.slot_to_expert and dp.map.tolist() == ora.expert_map()
    m = dp.map.tolist()
    assert rec["slots"][0] == [m[e] for e in ids[0]] and min(rec["slots"][0]) >= 0
    assert rec["slots"][1] == [-1] * 8


def run_experts(x, w, slots, w13, w2, algo=_lib.WISP_ALGO_GEMV):
    T, H = x.shape
    K = w.shape[1]
    I = w2.shape[2]
    E = w13.shape[0]
    act = torch.empty(max(1, T * K) * I, dtype=x.dtype, device=DEV)
    out = torch.empty_like(x)
    nbytes = _lib.lib().wisp_moe_work_bytes(max(1, T), K, H, E)
    work = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
    dt = _lib.WISP_F32 if x.dtype == torch.float32 else _lib.WISP_BF16
    _lib.check(_lib.lib().wisp_moe_experts(
        x.data_ptr(), dt, T, H, I, K, w.data_ptr(), slots.data_ptr(), E, w13.data_ptr(),
        w13.stride(0), w2.data_ptr(), w2.stride(0), act.data_ptr(), out.data_ptr(),
        work.data_ptr(), nbytes, algo, _lib.stream_handle()), "experts")
    torch.cuda.synchronize()
    return out


def _expert_case(seed, T, H, I, E, K, dtype):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, H, generator=g).to(dtype)
    w13 = (torch.randn(E, 2 * I, H, generator=g) * 0.02).to(dtype)
    w2 = (torch.randn(E, H, I, generator=g) * 0.02).to(dtype)
    logits = torch.randn(T, E, generator=g)
    w, ids = route(logits, K)
    return x, w, ids, w13, w2


# the last case's w2 rows (256 chunks of 16 bytes) take the looping w2 kernel
@pytest.mark.parametrize("T,H,I,E,K", [(1, 512, 256, 16, 2), (3, 512, 256, 16, 2),
                                        (1, 256, 64, 8, 2), (2, 1024, 384, 12, 4),
                                        (2, 256, 1024, 4, 2)])
def test_experts_gemv_fp32(T, H, I, E, K):
    x, w, ids, w13, w2 = _expert_case(T * 100 + H, T, H, I, E, K, torch.float32)
    ref = moe_forward(x, w, ids, w13, w2)
    out = run_experts(x.to(DEV), torch.tensor(w, dtype=torch.float32, device=DEV),
                      torch.tensor(ids, dtype=torch.int32, device=DEV), w13.to(DEV), w2.to(DEV))
    assert rel_err(out, ref) < 1e-5


# w2 rows past 128 chunks of 16 bytes take the looping w2 kernel (I 3072,
# 4608, 8192 and Mixtral's 14336, top-2 and top-8)
@pytest.mark.parametrize("T,H,I,E,K", [(1, 2048, 768, 16, 8), (2, 2048, 768, 12, 8),
                                        (1, 4096, 1024, 4, 2), (1, 1024, 512, 8, 2),
                                        (1, 1024, 3072, 4, 2), (2, 512, 4608, 4, 2),
                                        (1, 256, 14336, 3, 2), (1, 256, 8192, 8, 8),
                                        (2, 256, 14336, 8, 8)])
def test_experts_gemv_bf16(T, H, I, E, K):
    x, w, ids, w13, w2 = _expert_case(T * 7 + H, T, H, I, E, K, torch.bfloat16)
    out = run_experts(x.to(DEV), torch.tensor(w, dtype=torch.float32, device=DEV),
                      torch.tensor(ids, dtype=torch.int32, device=DEV), w13.to(DEV), w2.to(DEV))
    assert rel_err(out, moe_forward(x, w, ids, w13, w2)) < 1e-2
    # with act rounded to bf16 as the kernel stores it, agreement is much tighter
    assert rel_err(out, moe_forward(x, w, ids, w13, w2, act_round="bf16")) < 4e-3


def test_experts_absent_slot_contributes_zero():
    x, w, ids, w13, w2 = _expert_case(5, 1, 512, 256, 8, 2, torch.float32)
    slots = torch.tensor(ids, dtype=torch.int32)
    slots[0, 1] = -1
    wt = torch.tensor(w, dtype=torch.float32)
    out = run_experts(x.to(DEV), wt.to(DEV), slots.to(DEV), w13.to(DEV), w2.to(DEV))
    wz = wt.clone()
    wz[0, 1] = 0
    ref = moe_forward(x, wz.numpy(), ids, w13, w2)
    assert rel_err(out, ref) < 1e-5


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_output_bytes_independent_of_slot_placement(dtype):
    x, w, ids, w13, w2 = _expert_case(11, 2, 2048, 768, 16, 8, dtype)
    wt = torch.tensor(w, dtype=torch.float32, device=DEV)
    a = run_experts(x.to(DEV), wt, torch.tensor(ids, dtype=torch.int32, device=DEV),
                    w13.to(DEV), w2.to(DEV))
    perm = torch.randperm(16, generator=torch.Generator().manual_seed(1))
    inv = torch.argsort(perm)
    b = run_experts(x.to(DEV), wt, inv[torch.as_tensor(ids)].to(torch.int32).to(DEV),
                    w13[perm].to(DEV), w2[perm].to(DEV))
    assert torch.equal(a.view(torch.int16 if dtype == torch.bfloat16 else torch.int32),
                       b.view(torch.int16 if dtype == torch.bfloat16 else torch.int32))


MFMA = _lib.WISP_ALGO_MFMA


def _dev_case(x, w, ids, w13, w2):
    return (x.to(DEV), torch.tensor(w, dtype=torch.float32, device=DEV),
            torch.tensor(ids, dtype=torch.int32, device=DEV), w13.to(DEV), w2.to(DEV))


# (T, H, I, E, K): one 16-token tile, several tiles, a multi-pass slot
# (more than 128 tokens on one expert), a tiny call
@pytest.mark.parametrize("T,H,I,E,K", [(16, 2048, 768, 16, 8), (64, 2048, 768, 32, 8),
                                        (300, 512, 256, 4, 2), (5, 512, 256, 8, 2),
                                        (40, 1024, 512, 128, 8)])
def test_experts_mfma_bf16(T, H, I, E, K):
    x, w, ids, w13, w2 = _expert_case(T * 13 + E, T, H, I, E, K, torch.bfloat16)
    out = run_experts(*_dev_case(x, w, ids, w13, w2), algo=MFMA)
    assert rel_err(out, moe_forward(x, w, ids, w13, w2)) < 1e-2
    assert rel_err(out, moe_forward(x, w, ids, w13, w2, act_round="bf16")) < 4e-3


def _counted_case(seed, counts, H, I):
    """K = 2 routing where expert e receives exactly counts[e] tokens: the
    sorted expert labels are dealt to (token t, k = 0) for the first T labels
    and (t, k = 1) for the rest, so no token meets an expert twice while every
    count is at most T."""
    labels = np.repeat(np.arange(len(counts)), counts)
    T = len(labels) // 2
    assert len(labels) == 2 * T and max(counts) <= T
    ids = np.stack([labels[:T], labels[T:]], axis=1).astype(np.int64)
    g = torch.Generator().manual_seed(seed)
    E = len(counts)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    w13 = (torch.randn(E, 2 * I, H, generator=g) * 0.02).to(torch.bfloat16)
    w2 = (torch.randn(E, H, I, generator=g) * 0.02).to(torch.bfloat16)
    w = torch.rand(T, 2, generator=g).numpy().astype(np.float32) + 0.1
    return x, w, ids, w13, w2


# Slot sizes at every edge of the 16-token tiles and 64-token passes of the
# prefill kernels (more than 128 tokens per call): empty, 1, 15/16/17,
# 33, 48/49, 64/65 and a three-pass slot.
@pytest.mark.parametrize("H,I", [(512, 256), (2048, 768)])
def test_experts_mfma_prefill_slot_sizes(H, I):
    counts = [0, 1, 15, 16, 17, 33, 48, 49, 64, 65, 130, 2]
    x, w, ids, w13, w2 = _counted_case(H + I, counts, H, I)
    assert x.shape[0] > 128
    out = run_experts(*_dev_case(x, w, ids, w13, w2), algo=MFMA)
    assert rel_err(out, moe_forward(x, w, ids, w13, w2)) < 1e-2
    assert rel_err(out, moe_forward(x, w, ids, w13, w2, act_round="bf16")) < 4e-3


def test_mfma_prefill_bytes_independent_of_grouping():
    # a token's bytes are the same whether the call holds 300 tokens (several
    # 64-token passes per slot), 150 or 40
    x, w, ids, w13, w2 = _expert_case(31, 300, 1024, 512, 16, 8, torch.bfloat16)
    xd, wd, idd, w13d, w2d = _dev_case(x, w, ids, w13, w2)
    whole = run_experts(xd, wd, idd, w13d, w2d, algo=MFMA)
    assert rel_err(whole, moe_forward(x, w, ids, w13, w2, act_round="bf16")) < 4e-3
    for a, b in [(0, 150), (150, 300), (100, 140)]:
        part = run_experts(xd[a:b].contiguous(), wd[a:b].contiguous(), idd[a:b].contiguous(),
                           w13d, w2d, algo=MFMA)
        assert torch.equal(part.view(torch.int16), whole[a:b].view(torch.int16)), (a, b)


def test_experts_mfma_absent_slot_contributes_zero():
    x, w, ids, w13, w2 = _expert_case(6, 20, 512, 256, 8, 2, torch.bfloat16)
    slots = torch.tensor(ids, dtype=torch.int32)
    slots[3, 1] = -1
    slots[7, 0] = -1
    wt = torch.tensor(w, dtype=torch.float32)
    out = run_experts(x.to(DEV), wt.to(DEV), slots.to(DEV), w13.to(DEV), w2.to(DEV), algo=MFMA)
    wz = wt.clone()
    wz[3, 1] = 0
    wz[7, 0] = 0
    assert rel_err(out, moe_forward(x, wz.numpy(), ids, w13, w2, act_round="bf16")) < 4e-3


# Slot ids outside [0, nslots) - at nslots, past it, far past it, below -1 -
# read no expert and contribute zero on every expert path, as a slot of -1
# does (the GEMV shapes take both w2 kernels: rows in registers and the
# looping one).
@pytest.mark.parametrize("algo,dtype,T,H,I,E,K", [
    (_lib.WISP_ALGO_GEMV, torch.float32, 3, 512, 256, 8, 2),
    (_lib.WISP_ALGO_GEMV, torch.bfloat16, 2, 1024, 384, 12, 4),
    (_lib.WISP_ALGO_GEMV, torch.bfloat16, 2, 256, 8192, 4, 2),
    (_lib.WISP_ALGO_MFMA, torch.bfloat16, 20, 512, 256, 8, 2)])
def test_experts_out_of_range_slot_contributes_zero(algo, dtype, T, H, I, E, K):
    x, w, ids, w13, w2 = _expert_case(T * 17 + I, T, H, I, E, K, dtype)
    slots = torch.tensor(ids, dtype=torch.int32)
    bad = [(0, 0, E), (0, K - 1, E + 5), (1, 1, 1 << 30), (T - 1, 0, -7)]
    wt = torch.tensor(w, dtype=torch.float32)
    wz = wt.clone()
    for t, k, s in bad:
        slots[t, k] = s
        wz[t, k] = 0
    out = run_experts(x.to(DEV), wt.to(DEV), slots.to(DEV), w13.to(DEV), w2.to(DEV), algo=algo)
    if dtype == torch.float32:
        assert rel_err(out, moe_forward(x, wz.numpy(), ids, w13, w2)) < 1e-5
    else:
        assert rel_err(out, moe_forward(x, wz.numpy(), ids, w13, w2, act_round="bf16")) < 4e-3


def test_mfma_bytes_independent_of_slots_and_grouping():
    # A token's output must not depend on its slot numbers nor on which other
    # tokens share the call: this is what makes paged == resident bytes.
    x, w, ids, w13, w2 = _expert_case(12, 48, 2048, 768, 16, 8, torch.bfloat16)
    xd, wd, idd, w13d, w2d = _dev_case(x, w, ids, w13, w2)
    whole = run_experts(xd, wd, idd, w13d, w2d, algo=MFMA)
    perm = torch.randperm(16, generator=torch.Generator().manual_seed(2))
    inv = torch.argsort(perm)
    moved = run_experts(xd, wd, inv[torch.as_tensor(ids)].to(torch.int32).to(DEV),
                        w13[perm].to(DEV), w2[perm].to(DEV), algo=MFMA)
    assert torch.equal(whole.view(torch.int16), moved.view(torch.int16))
    for a, b in [(0, 5), (5, 21), (21, 48)]:
        part = run_experts(xd[a:b].contiguous(), wd[a:b].contiguous(), idd[a:b].contiguous(),
                           w13d, w2d, algo=MFMA)
        assert torch.equal(part.view(torch.int16), whole[a:b].view(torch.int16)), (a, b)
