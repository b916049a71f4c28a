"""Page-in from packed bf16 masters on the GPU: every slot a call fills holds
its expert's master bytes exactly, and outputs equal those of a state that
pages the plain masters (WISP_PACKED_MASTERS=0), on both copy-kernel paths
(the fused one-token launch and the page-in kernel of larger calls), the
opt-in fused decode launch, resident priming and a resize."""
import numpy as np
import pytest
import torch

from wisp.integrations.vllm.fused_moe import WispMoEState

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _masters(E, H, I, seed):
    g = torch.Generator().manual_seed(seed)
    w13 = (torch.randn(E, 2 * I, H, generator=g) * 0.02).to(torch.bfloat16)
    w2 = (torch.randn(E, H, I, generator=g) * 0.02).to(torch.bfloat16)
    # blocks whose exponents span more than 15 values (the exception area),
    # zeros of both signs and an all-zero block, in w13 and w2 rows
    for e in range(0, E, 3):
        w13[e, e % (2 * I), 3] = 40.0
        w13[e, e % (2 * I), 9] = 1e-6
        w2[e, (5 * e) % H, 70 % I] = -24.0
        w2[e, (5 * e) % H, 71 % I] = 3e-7
    w13[1, 7, :64] = 0.0
    w13[2, 9, 64:128] = -0.0
    return w13.pin_memory(), w2.pin_memory()


def _slots_hold_masters(st, w13, w2):
    n = 0
    for s, e in enumerate(st.slot_to_expert):
        if e < 0:
            continue
        assert torch.equal(st.scratch_w13[s].cpu().view(torch.int16), w13[e].view(torch.int16)), (s, e)
        assert torch.equal(st.scratch_w2[s].cpu().view(torch.int16), w2[e].view(torch.int16)), (s, e)
        n += 1
    return n


def _pair(monkeypatch, w13, w2, cap, mode="paged"):
    """A state paging packed masters and one paging the plain masters."""
    monkeypatch.setenv("WISP_PAGEIN_ENGINE", "kernel")
    monkeypatch.setenv("WISP_PACKED_MASTERS", "1")
    packed = WispMoEState(w13, w2, cap, mode, DEV, 0)
    monkeypatch.setenv("WISP_PACKED_MASTERS", "0")
    plain = WispMoEState(w13, w2, cap, mode, DEV, 1)
    assert packed._packed is not None and plain._packed is None
    assert packed.pagein_engine == "kernel"
    assert packed.packed_bytes_per_expert < 0.9 * plain.packed_bytes_per_expert
    return packed, plain


@pytest.mark.parametrize("fused", ["0", "1"])
def test_packed_pagein_fills_slots_with_master_bytes(monkeypatch, fused):
    monkeypatch.setenv("WISP_DECODE_FUSED", fused)
    E, H, I, K, cap = 16, 256, 128, 4, 4 if fused == "1" else 8
    w13, w2 = _masters(E, H, I, 11)
    packed, plain = _pair(monkeypatch, w13, w2, cap)
    g = torch.Generator().manual_seed(12)
    sizes = [1, 1, 3, 1, 1, 9, 1, 2, 1, 1, 5, 1] if fused == "0" else [1] * 16
    filled = 0
    for i, T in enumerate(sizes):
        x = torch.randn(T, H, generator=g).to(torch.bfloat16).to(DEV)
        lg = torch.randn(T, E, generator=g).to(DEV)
        a = packed.forward(x, lg, K, True)
        b = plain.forward(x, lg, K, True)
        torch.cuda.synchronize()
        assert torch.equal(a.view(torch.int16), b.view(torch.int16)), (i, T)
        assert packed.slot_to_expert == plain.slot_to_expert, i
        filled += _slots_hold_masters(packed, w13, w2)
    assert filled > 0


def test_packed_resident_priming_and_resize(monkeypatch):
    E, H, I = 12, 192, 64
    w13, w2 = _masters(E, H, I, 21)
    packed, plain = _pair(monkeypatch, w13, w2, E, mode="resident")
    packed.prime_identity()
    plain.prime_identity()
    torch.cuda.synchronize()
    assert _slots_hold_masters(packed, w13, w2) == E
    monkeypatch.setenv("WISP_PACKED_MASTERS", "1")
    paged = WispMoEState(w13, w2, 4, "paged", DEV, 2)
    g = torch.Generator().manual_seed(22)
    for cap in (4, 7, 3):
        paged.resize_cap(cap)
        for _ in range(3):
            x = torch.randn(2, H, generator=g).to(torch.bfloat16).to(DEV)
            lg = torch.randn(2, E, generator=g).to(DEV)
            out = paged.forward(x, lg, 2, True)
            ref = packed.forward(x, lg, 2, True)
            torch.cuda.synchronize()
            assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
            _slots_hold_masters(paged, w13, w2)


def test_packed_copy_shared_and_rebuilt_after_a_master_write(monkeypatch):
    """States over the same masters share one packed copy; an in-place write
    to the masters (torch's version counter) makes the next state pack anew,
    and it pages the new values."""
    monkeypatch.setenv("WISP_PAGEIN_ENGINE", "kernel")
    monkeypatch.setenv("WISP_PACKED_MASTERS", "1")
    E, H, I = 8, 128, 64
    w13, w2 = _masters(E, H, I, 31)
    a = WispMoEState(w13, w2, 4, "paged", DEV, 0)
    b = WispMoEState(w13, w2, 4, "paged", DEV, 1)
    assert a._packed is not None and a._packed is b._packed
    w13[3].mul_(2.0)
    w2[3].mul_(-1.0)
    c = WispMoEState(w13, w2, 4, "paged", DEV, 2)
    assert c._packed is not None and c._packed is not a._packed
    lg = torch.zeros(1, E)
    lg[0, 3], lg[0, 5] = 8.0, 4.0
    x = torch.randn(1, H, generator=torch.Generator().manual_seed(32)).to(torch.bfloat16)
    c.forward(x.to(DEV), lg.to(DEV), 2, True)
    torch.cuda.synchronize()
    assert sorted(e for e in c.slot_to_expert if e >= 0) == [3, 5]
    assert _slots_hold_masters(c, w13, w2) == 2
