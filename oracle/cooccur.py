"""Oracle: restatement of the reference's cross-layer expert predictor and the
post-forward prefetch step — TEST INFRASTRUCTURE ONLY.

Follows the reference:

* ``CooccurOracle.observe_step``  <- ``CooccurTable.observe_step``
                                     (src/wisp/oracle/cooccur.py:79-104)
* ``CooccurOracle.to_dict/from_dict`` <- the JSON schema 1 (cooccur.py:146-195)
* ``predict_layer``               <- ``predict_layer`` (cooccur.py:233-287)
* ``prefetch_glue``               <- the post-forward block of the paged
                                     forward (src/wisp/integrations/vllm/
                                     fused_moe.py:1173-1233) with
                                     ``_cooccur_predict_top_k`` (634-650)

Scores are accumulated in CPython float (IEEE double) in the reference's
order: layers in step insertion order, each layer's experts in the iteration
order of the ``set`` the forward built, one add per (source layer, source
expert) to each destination expert's score; ties in the ranking go to the
lower expert id.  This module runs on CPython, so set orders are native.

Pinning.  The reference ships no tests for this code.  ``tests/
test_oracle_cooccur.py`` pins it with hand-derived known answers (pair counts
and marginals of small steps, scores with normalisation and decay worked by
hand, tie order), the closed form of the pair count of a step, JSON round
trips, and an independent brute-force re-derivation of the scores.
"""
from __future__ import annotations

from collections import Counter, defaultdict
from typing import Iterable, Mapping


class CooccurOracle:
    """Sparse per-layer-pair co-activation counts (cooccur.py:43-77)."""

    SCHEMA_VERSION = 1

    def __init__(self) -> None:
        self.count: dict[tuple[int, int], dict[int, Counter]] = defaultdict(
            lambda: defaultdict(Counter))
        self.layer_total: dict[tuple[int, int], int] = defaultdict(int)
        self.num_steps_observed = 0

    def observe_step(self, expert_ids_by_layer: Mapping[int, Iterable[int]]) -> None:
        per_layer = {L: list(eids) for L, eids in expert_ids_by_layer.items() if eids}
        for L_src, src in per_layer.items():
            for e in src:
                self.layer_total[(L_src, e)] += 1
        for L_src, src in per_layer.items():
            for e_src in src:
                per_dst = self.count[(L_src, e_src)]
                for L_dst, dst in per_layer.items():
                    if L_dst <= L_src:
                        continue
                    row = per_dst[L_dst]
                    for e_dst in dst:
                        row[e_dst] += 1
        self.num_steps_observed += 1

    def to_dict(self) -> dict:
        pairs = [[int(Ls), int(es), int(Ld), int(ed), int(n)]
                 for (Ls, es), per in self.count.items()
                 for Ld, row in per.items() for ed, n in row.items() if n > 0]
        marg = [[int(L), int(e), int(n)] for (L, e), n in self.layer_total.items() if n > 0]
        return {"schema_version": self.SCHEMA_VERSION,
                "num_steps_observed": int(self.num_steps_observed),
                "pairs": pairs, "marginals": marg}

    @classmethod
    def from_dict(cls, data: Mapping) -> "CooccurOracle":
        if int(data.get("schema_version", 1)) != cls.SCHEMA_VERSION:
            raise ValueError("unsupported cooccur schema_version")
        t = cls()
        for Ls, es, Ld, ed, n in data.get("pairs") or []:
            t.count[(int(Ls), int(es))][int(Ld)][int(ed)] = int(n)
        for L, e, n in data.get("marginals") or []:
            t.layer_total[(int(L), int(e))] = int(n)
        t.num_steps_observed = int(data.get("num_steps_observed", 0))
        return t


def predict_layer(table: CooccurOracle, seen_so_far: Mapping[int, Iterable[int]],
                  target_layer: int, *, k: int = 8, normalize: bool = True,
                  decay: float = 1.0, only_prev_layer: bool = False) -> list[int]:
    scores: defaultdict[int, float] = defaultdict(float)
    for L_src, src in seen_so_far.items():
        if L_src >= target_layer:
            continue
        if only_prev_layer and L_src != target_layer - 1:
            continue
        w = decay ** (target_layer - L_src - 1)
        for e_src in src:
            per_dst = table.count.get((L_src, e_src))
            if not per_dst:
                continue
            row = per_dst.get(target_layer)
            if not row:
                continue
            total = table.layer_total.get((L_src, e_src), 0) if normalize else 1
            denom = total if (normalize and total > 0) else 1
            for e_dst, c in row.items():
                scores[e_dst] += w * c / denom
    if not scores:
        return []
    ranked = sorted(scores.items(), key=lambda x: (-x[1], x[0]))
    return [e for e, _ in ranked[:k]]


def prefetch_glue(states: list, layer_idx: int, table: CooccurOracle | None,
                  step_obs: dict, online: bool) -> list[int]:
    """The reference's post-forward block for layer ``layer_idx`` (after its
    ``forward`` set ``last_unique_experts``): record the layer's experts for
    the step, predict the next layer's ``max(8, cap // 2)`` experts from the
    step so far (normalised, decay 0.5), prefetch them into the next layer's
    state, and at the last layer optionally learn the step and clear it.
    Returns the prediction (rank order)."""
    st = states[layer_idx]
    last_set = st.last_unique_experts
    predicted: list[int] = []
    if table is not None and last_set:
        step_obs[layer_idx] = last_set
        nxt = layer_idx + 1
        if nxt < len(states):
            ns = states[nxt]
            k = max(8, ns.cap_experts // 2)
            if step_obs:
                predicted = predict_layer(table, step_obs, nxt, k=k, normalize=True,
                                          decay=0.5, only_prev_layer=False)
            if predicted:
                ns.prefetch_async(set(predicted))
                ns.stats_pred_total += len(predicted)
        if layer_idx == len(states) - 1:
            if online:
                table.observe_step(step_obs)
            step_obs.clear()
    return predicted
