"""Oracle: routing and the fused-MoE expert MLP on the CPU — TEST INFRASTRUCTURE ONLY.

The reference hands these steps to vLLM 0.11.2 (not vendored, absent here):

* ``route``      <- ``layer.select_experts(..., renormalize, scoring_func="softmax")``
                    (reference ``fused_moe.py:1054-1076``): float32 softmax over the
                    E router logits, top-k in descending order, then ``w /= w.sum()``.
* ``moe_forward`` <- ``fused_experts(x, w13, w2, topk_weights, topk_ids,
                    activation="silu", expert_map=...)`` (``fused_moe.py:1106-1118``,
                    ``1155-1167``): per routed (token, k) pair
                    ``h = W13[e] x``, ``act = silu(h[:I]) * h[I:]`` (gate rows first,
                    then up rows), ``y = W2[e] act``, and
                    ``out[t] = sum_k w[t, k] * y[t, k]`` in routing order k = 0..K-1.
                    An expert the map marks absent (-1) contributes zero.

Top-k order.  Experts are ranked by logit (descending, ties to the lower
index).  Softmax is monotone, so this is the probability order vLLM uses
except where two distinct logits round to one float32 probability; the
workload generators keep a gap at every top-k boundary so that case never
arises.

Numerics.  Everything accumulates in float64 from the exact float32/bf16
inputs.  ``act_round="bf16"`` rounds ``act`` to bfloat16 (round to nearest
even) before the down projection, as a bf16 kernel that stores its
intermediate in bf16 does.

Pinning (checks in ``tests/test_oracle_moe.py``): routing by the closed form
and its invariants (weights sum to 1, descending, ids distinct, k = E returns
every expert, renormalised weights equal the top-k-only softmax); the MLP by
an independent per-element pure-Python evaluation on tiny shapes, by
reduction to ``torch.nn.functional.silu`` dense SwiGLU for k = 1, by W2 = 0
and x = 0 giving 0, by linearity in W2 and by invariance of the combine under
permutation of the expert table.
"""
from __future__ import annotations

import numpy as np
import torch


def route(logits, k: int, renormalize: bool = True):
    """``logits [T, E]`` -> ``(weights float64 [T, k], ids int64 [T, k])``."""
    lg = torch.as_tensor(logits).to(torch.float32).to(torch.float64).numpy()
    T, E = lg.shape
    if not 1 <= k <= E:
        raise ValueError(f"top_k={k} outside [1, {E}]")
    ids = np.empty((T, k), dtype=np.int64)
    w = np.empty((T, k), dtype=np.float64)
    cols = np.arange(E)
    for t in range(T):
        order = np.lexsort((cols, -lg[t]))[:k]      # value desc, index asc
        ids[t] = order
        m = lg[t].max()
        p = np.exp(lg[t] - m)
        p /= p.sum()
        w[t] = p[order]
        if renormalize:
            w[t] /= w[t].sum()
    return w, ids


def _bf16(a: torch.Tensor) -> torch.Tensor:
    return a.to(torch.float32).to(torch.bfloat16).to(torch.float64)


def moe_forward(x, topk_w, topk_ids, w13, w2, expert_map=None, act_round: str | None = None,
                dtype=torch.float64) -> torch.Tensor:
    """Routed SwiGLU experts with the routing-order combine.

    ``x [T, H]``, ``topk_w [T, K]``, ``topk_ids [T, K]`` (global ids),
    ``w13 [E, 2I, H]``, ``w2 [E, H, I]``; ``expert_map`` (optional) maps a
    global id to -1 when the expert is absent.  Returns ``out [T, H]`` in
    ``dtype`` (float64 by default).
    """
    x = torch.as_tensor(x).to(dtype)
    tw = torch.as_tensor(np.asarray(topk_w, dtype=np.float64)).to(dtype)
    ids = np.asarray(topk_ids, dtype=np.int64)
    T, K = ids.shape
    H = x.shape[1]
    I = w2.shape[2]
    out = torch.zeros((T, H), dtype=dtype)
    # Evaluate expert by expert (only the experts that are routed to), then
    # combine per token strictly in routing order.
    y = torch.zeros((T, K, H), dtype=dtype)
    for e in np.unique(ids):
        e = int(e)
        if expert_map is not None and int(expert_map[e]) < 0:
            continue
        rows = np.argwhere(ids == e)                 # (t, k) pairs routed to e
        xt = x[torch.as_tensor(rows[:, 0])]          # [n, H]
        W13 = w13[e].to(dtype)
        W2 = w2[e].to(dtype)
        h = xt @ W13.T                               # [n, 2I]
        gate, up = h[:, :I], h[:, I:]
        act = torch.nn.functional.silu(gate) * up
        if act_round == "bf16":
            act = _bf16(act)
        elif act_round is not None:
            raise ValueError(act_round)
        y[torch.as_tensor(rows[:, 0]), torch.as_tensor(rows[:, 1])] = act @ W2.T
    for k in range(K):
        out += tw[:, k:k + 1] * y[:, k]
    return out


def moe_forward_loops(x, topk_w, topk_ids, w13, w2):
    """Independent per-element evaluation in pure Python float arithmetic
    (tiny shapes only): the checker for ``moe_forward``."""
    import math
    x = torch.as_tensor(x).to(torch.float64).tolist()
    w13 = torch.as_tensor(w13).to(torch.float64).tolist()
    w2 = torch.as_tensor(w2).to(torch.float64).tolist()
    T, K = len(topk_ids), len(topk_ids[0])
    H = len(x[0])
    I = len(w2[0][0])
    out = [[0.0] * H for _ in range(T)]
    for t in range(T):
        for k in range(K):
            e = int(topk_ids[t][k])
            wt = float(topk_w[t][k])
            act = []
            for i in range(I):
                g = sum(w13[e][i][j] * x[t][j] for j in range(H))
                u = sum(w13[e][I + i][j] * x[t][j] for j in range(H))
                act.append(g / (1.0 + math.exp(-g)) * u)
            for h in range(H):
                out[t][h] += wt * sum(w2[e][h][i] * act[i] for i in range(I))
    return torch.tensor(out, dtype=torch.float64)


def moe_forward_fast(x, topk_w, topk_ids, w13, w2) -> torch.Tensor:
    """The torch CPU fused-MoE timed as the CPU baseline: expert GEMMs in
    the weights' dtype with float32 accumulation (``torch.nn.functional.linear``),
    SiLU*mul in float32 rounded back to the weights' dtype, then the
    routing-order combine in float32."""
    x = torch.as_tensor(x)
    ids = np.asarray(topk_ids, dtype=np.int64)
    tw = torch.as_tensor(np.asarray(topk_w, dtype=np.float32))
    T, K = ids.shape
    I = w2.shape[2]
    y = torch.zeros((T, K, x.shape[1]), dtype=torch.float32)
    for e in np.unique(ids):
        rows = np.argwhere(ids == int(e))
        xt = x[torch.as_tensor(rows[:, 0])]
        h = torch.nn.functional.linear(xt, w13[int(e)]).float()
        act = (torch.nn.functional.silu(h[:, :I]) * h[:, I:]).to(x.dtype)
        y[torch.as_tensor(rows[:, 0]), torch.as_tensor(rows[:, 1])] = \
            torch.nn.functional.linear(act, w2[int(e)]).float()
    out = torch.zeros((T, x.shape[1]), dtype=torch.float32)
    for k in range(K):
        out += tw[:, k:k + 1] * y[:, k]
    return out.to(x.dtype)
