"""Pins the fused-MoE oracle (oracle/moe.py) without reusing its formulas:
routing against its defining invariants, the expert MLP against an
independent per-element evaluation, a library SwiGLU and special cases."""
import numpy as np
import pytest
import torch

from oracle.moe import moe_forward, moe_forward_loops, route


def test_route_invariants():
    g = torch.Generator().manual_seed(3)
    logits = torch.randn(64, 128, generator=g) * 2
    w, ids = route(logits, 8)
    assert np.allclose(w.sum(1), 1.0, atol=1e-12)
    assert (np.diff(w, axis=1) <= 0).all()                     # descending
    assert all(len(set(r)) == 8 for r in ids.tolist())         # distinct
    # the chosen ids are exactly the 8 largest logits
    lg = logits.numpy()
    for t in range(64):
        assert set(ids[t]) == set(np.argsort(-lg[t])[:8])
    # renormalised weights equal a softmax over the top-k logits alone
    for t in range(64):
        sel = lg[t, ids[t]].astype(np.float64)
        ref = np.exp(sel - sel.max()); ref /= ref.sum()
        assert np.allclose(w[t], ref, rtol=1e-12)


def test_route_full_k_and_no_renorm():
    logits = torch.tensor([[0.5, -1.0, 2.0, 0.0]])
    w, ids = route(logits, 4)
    assert ids.tolist() == [[2, 0, 3, 1]]
    w2, _ = route(logits, 2, renormalize=False)
    p = torch.softmax(logits.double(), -1)[0].numpy()
    assert np.allclose(w2[0], p[[2, 0]], rtol=1e-12)


def test_route_ties_go_to_lower_index():
    logits = torch.tensor([[1.0, 3.0, 3.0, 0.0, 3.0]])
    _, ids = route(logits, 3)
    assert ids.tolist() == [[1, 2, 4]]


def _tiny(seed=0, T=3, H=8, I=4, E=5, K=2):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, H, generator=g)
    w13 = torch.randn(E, 2 * I, H, generator=g) * 0.5
    w2 = torch.randn(E, H, I, generator=g) * 0.5
    logits = torch.randn(T, E, generator=g)
    w, ids = route(logits, K)
    return x, w, ids, w13, w2


def test_moe_matches_per_element_loops():
    for seed in range(4):
        x, w, ids, w13, w2 = _tiny(seed)
        a = moe_forward(x, w, ids, w13, w2)
        b = moe_forward_loops(x, w.tolist(), ids.tolist(), w13, w2)
        assert torch.allclose(a, b, rtol=1e-12, atol=1e-12)


def test_moe_k1_is_dense_swiglu():
    # k = 1 with weight 1: out = W2 (silu(W1 x) * (W3 x)), via torch's SiLU
    x, _, _, w13, w2 = _tiny(1, K=1)
    ids = np.full((x.shape[0], 1), 3)
    w = np.ones((x.shape[0], 1))
    out = moe_forward(x, w, ids, w13, w2)
    I = w2.shape[2]
    W1, W3 = w13[3, :I].double(), w13[3, I:].double()
    ref = torch.nn.functional.linear(
        torch.nn.functional.silu(x.double() @ W1.T) * (x.double() @ W3.T), w2[3].double())
    assert torch.allclose(out, ref, rtol=1e-12, atol=1e-12)


def test_moe_zero_cases_and_linearity():
    x, w, ids, w13, w2 = _tiny(2)
    assert moe_forward(x, w, ids, w13, torch.zeros_like(w2)).abs().max() == 0
    assert moe_forward(torch.zeros_like(x), w, ids, w13, w2).abs().max() == 0
    a = moe_forward(x, w, ids, w13, w2)
    b = moe_forward(x, w, ids, w13, 2.0 * w2)       # exact scaling in float32
    assert torch.allclose(b, 2.0 * a, rtol=1e-12, atol=1e-12)
    extra = 0.25 * w13[:, :w2.shape[1], :w2.shape[2]].double()
    c = moe_forward(x, w, ids, w13, w2.double() + extra)  # additivity in W2 (exact in f64)
    d = moe_forward(x, w, ids, w13, extra)
    assert torch.allclose(c, a + d, rtol=1e-9, atol=1e-9)


def test_moe_expert_table_permutation_invariant():
    # Relabelling experts (slot placement) cannot change the output.
    x, w, ids, w13, w2 = _tiny(4)
    perm = torch.randperm(w13.shape[0], generator=torch.Generator().manual_seed(9))
    inv = torch.argsort(perm)
    a = moe_forward(x, w, ids, w13, w2)
    b = moe_forward(x, w, inv.numpy()[ids], w13[perm], w2[perm])
    assert torch.equal(a, b)


def test_moe_absent_expert_contributes_zero():
    x, w, ids, w13, w2 = _tiny(5)
    emap = np.arange(w13.shape[0])
    emap[ids[0, 1]] = -1
    a = moe_forward(x, w, ids, w13, w2, expert_map=emap)
    keep = np.ones_like(w)
    keep[ids == ids[0, 1]] = 0
    b = moe_forward(x, w * keep, ids, w13, w2)
    assert torch.allclose(a, b, rtol=1e-12, atol=1e-12)
