"""Expert co-activation table and cross-layer predictor, held in HBM.

Mirrors the reference's ``wisp.oracle.cooccur`` (``CooccurTable``,
``predict_layer``; src/wisp/oracle/cooccur.py:43-287) with the same JSON
schema (version 1: ``pairs`` ``[L_src, e_src, L_dst, e_dst, n]`` and
``marginals`` ``[L, e, n]``), but the counts live in a dense device tensor
``count[L_src][e_src][L_dst][e_dst]`` (int32; 151 MB at 48 layers x 128
experts) so that the paged forward can observe, predict and prefetch with
GPU kernels and no host round trip (``wisp_cooccur_*`` in ``libwisp_hip.so``).

Scores are accumulated in IEEE doubles in the reference's order (layers in
the order the step saw them, each layer's experts in their set iteration
order) and ranked by (score desc, id asc), so predictions match the
reference's bit for bit.  Pairs counted zero are treated as absent.
"""
from __future__ import annotations

import ctypes as C
import gzip
import json
import logging
import os
from typing import Iterable, Mapping, Union

import numpy as np
import torch

from wisp_amd import _lib
from wisp_amd._lib import check, lib

logger = logging.getLogger("wisp.integrations.vllm.cooccur")


class CooccurTable:
    """Per-layer-pair expert co-activation counts on one GPU.

    ``count[L_src, e_src, L_dst, e_dst]`` = number of steps in which expert
    ``e_src`` fired at layer ``L_src`` and ``e_dst`` at ``L_dst > L_src``;
    ``layer_total[L, e]`` = steps in which ``e`` fired at ``L``.  The table
    also holds the current step's per-layer observations, which the paged
    forward fills layer by layer.
    """

    SCHEMA_VERSION = 1

    def __init__(self, layers: int, experts: int, device: torch.device | str = "cuda") -> None:
        if not (1 <= layers <= 256 and 1 <= experts <= 512):
            raise ValueError("CooccurTable covers 1..256 layers and 1..512 experts")
        self.layers, self.experts = int(layers), int(experts)
        self.device = torch.device(device)
        L, E = self.layers, self.experts
        dev = self.device
        self.count = torch.zeros((L, E, L, E), dtype=torch.int32, device=dev)
        self.layer_total = torch.zeros((L, E), dtype=torch.int32, device=dev)
        self._obs_keys = torch.zeros((L, E), dtype=torch.int32, device=dev)
        self._obs_n = torch.zeros(L, dtype=torch.int32, device=dev)
        self._obs_seq = torch.zeros(L, dtype=torch.int32, device=dev)
        self._meta = torch.zeros(4, dtype=torch.int32, device=dev)
        self._pred_ids = torch.zeros(E, dtype=torch.int32, device=dev)
        self._pred_n = torch.zeros(1, dtype=torch.int32, device=dev)
        self._weights: dict[float, torch.Tensor] = {}
        self._c = _lib.Cooccur()
        c = self._c
        c.layers, c.experts = L, E
        c.count, c.total = self.count.data_ptr(), self.layer_total.data_ptr()
        c.obs_keys, c.obs_n = self._obs_keys.data_ptr(), self._obs_n.data_ptr()
        c.obs_seq, c.meta = self._obs_seq.data_ptr(), self._meta.data_ptr()

    # -- step observations (device) ----------------------------------------
    def observe_layer(self, layer: int, ids: torch.Tensor, n: int | None = None,
                      ordered: bool = False) -> None:
        """Record ``layer``'s experts for the current step from the first
        ``n`` int32 device ids: as the set the forward builds from their
        ascending unique (``ordered=False``), or in the given order."""
        n = ids.numel() if n is None else int(n)
        check(lib().wisp_cooccur_observe_layer(C.byref(self._c), int(layer), ids.data_ptr(), n,
                                               int(bool(ordered)), _lib.stream_handle()),
              "cooccur observe")

    def _weights_for(self, decay: float) -> torch.Tensor:
        w = self._weights.get(decay)
        if w is None:
            # Python float powers, exactly as the reference computes them
            w = torch.tensor([decay ** d for d in range(self.layers)], dtype=torch.float64,
                             device=self.device)
            self._weights[decay] = w
        return w

    def predict_device(self, target_layer: int, k: int, *, normalize: bool = True,
                       decay: float = 1.0, only_prev_layer: bool = False):
        """Top-``k`` prediction for ``target_layer`` from the step so far, as
        device tensors ``(ids [E] int32, n [1] int32)`` (no host sync)."""
        k = max(0, min(int(k), self.experts))
        w = self._weights_for(float(decay))
        check(lib().wisp_cooccur_predict(C.byref(self._c), int(target_layer), k, w.data_ptr(),
                                         int(bool(normalize)), int(bool(only_prev_layer)),
                                         self._pred_ids.data_ptr(), self._pred_n.data_ptr(),
                                         _lib.stream_handle()), "cooccur predict")
        return self._pred_ids, self._pred_n

    def end_step(self, learn: bool) -> None:
        """Add the step's pairs to the counts when ``learn``; clear the step."""
        check(lib().wisp_cooccur_end_step(C.byref(self._c), int(bool(learn)),
                                          _lib.stream_handle()), "cooccur end_step")

    # -- reference API -----------------------------------------------------
    def observe_step(self, expert_ids_by_layer: Mapping[int, Iterable[int]]) -> None:
        """Update from one step's per-layer activations (reference
        cooccur.py:79-104).  Uses the table's step buffers: not for use in the
        middle of a decode step."""
        self.end_step(False)
        for L, eids in expert_ids_by_layer.items():
            ids = [int(e) for e in eids]
            if ids:
                self.observe_layer(int(L), torch.tensor(ids, dtype=torch.int32,
                                                        device=self.device), ordered=True)
        self.end_step(True)

    @property
    def num_steps_observed(self) -> int:
        return int(self._meta[1].item())

    @property
    def n_source_keys(self) -> int:
        return int((self.count.view(self.layers * self.experts, -1) > 0).any(dim=1).sum().item())

    @property
    def n_pairs(self) -> int:
        return int((self.count > 0).sum().item())

    def memory_estimate_bytes(self) -> int:
        return self.count.numel() * 4 + self.layer_total.numel() * 4

    # -- serialisation (schema 1, reference cooccur.py:146-218) -------------
    def to_dict(self) -> dict:
        cnt = self.count.cpu().numpy()
        nz = np.argwhere(cnt > 0)
        pairs = [[int(a), int(b), int(c), int(d), int(cnt[a, b, c, d])] for a, b, c, d in nz]
        tot = self.layer_total.cpu().numpy()
        marg = [[int(L), int(e), int(tot[L, e])] for L, e in np.argwhere(tot > 0)]
        return {"schema_version": self.SCHEMA_VERSION,
                "num_steps_observed": self.num_steps_observed,
                "pairs": pairs, "marginals": marg,
                "stats": {"n_source_keys": self.n_source_keys, "n_pairs": len(pairs),
                          "memory_estimate_bytes": self.memory_estimate_bytes()}}

    @classmethod
    def from_dict(cls, data: Mapping[str, object], layers: int | None = None,
                  experts: int | None = None, device: torch.device | str = "cuda"
                  ) -> "CooccurTable":
        version = int(data.get("schema_version", 1))
        if version != cls.SCHEMA_VERSION:
            raise ValueError(f"CooccurTable.from_dict: schema_version={version} unsupported "
                             f"(expected {cls.SCHEMA_VERSION})")
        pairs = np.asarray(data.get("pairs") or [], dtype=np.int64).reshape(-1, 5)
        marg = np.asarray(data.get("marginals") or [], dtype=np.int64).reshape(-1, 3)
        if layers is None:
            layers = int(max(pairs[:, [0, 2]].max(initial=-1), marg[:, 0].max(initial=-1))) + 1
        if experts is None:
            experts = int(max(pairs[:, [1, 3]].max(initial=-1), marg[:, 1].max(initial=-1))) + 1
        t = cls(max(1, layers), max(1, experts), device)
        L, E = t.layers, t.experts
        keep = ((pairs[:, 0] < L) & (pairs[:, 2] < L) & (pairs[:, 1] < E) & (pairs[:, 3] < E) &
                (pairs[:, 0] >= 0) & (pairs[:, 1] >= 0) & (pairs[:, 2] >= 0) & (pairs[:, 3] >= 0))
        if not keep.all():
            logger.warning("wisp.cooccur: %d pairs outside %d layers x %d experts dropped",
                           int((~keep).sum()), L, E)
        cnt = np.zeros((L, E, L, E), dtype=np.int32)
        p = pairs[keep]
        cnt[p[:, 0], p[:, 1], p[:, 2], p[:, 3]] = p[:, 4]
        tot = np.zeros((L, E), dtype=np.int32)
        mk = (marg[:, 0] >= 0) & (marg[:, 0] < L) & (marg[:, 1] >= 0) & (marg[:, 1] < E)
        m = marg[mk]
        tot[m[:, 0], m[:, 1]] = m[:, 2]
        t.count.copy_(torch.from_numpy(cnt))
        t.layer_total.copy_(torch.from_numpy(tot))
        t._meta[1] = int(data.get("num_steps_observed", 0))
        return t

    def save(self, path: Union[str, os.PathLike]) -> None:
        spath = os.fspath(path)
        os.makedirs(os.path.dirname(spath) or ".", exist_ok=True)
        text = json.dumps(self.to_dict(), separators=(",", ":"))
        if spath.endswith(".gz"):
            with gzip.open(spath, "wt", encoding="utf-8") as f:
                f.write(text)
        else:
            with open(spath, "w", encoding="utf-8") as f:
                f.write(text)

    @classmethod
    def load(cls, path: Union[str, os.PathLike], layers: int | None = None,
             experts: int | None = None, device: torch.device | str = "cuda") -> "CooccurTable":
        spath = os.fspath(path)
        opener = gzip.open if spath.endswith(".gz") else open
        with opener(spath, "rt", encoding="utf-8") as f:
            data = json.load(f)
        return cls.from_dict(data, layers, experts, device)


def predict_layer(table: CooccurTable, seen_so_far: Mapping[int, Iterable[int]],
                  target_layer: int, *, k: int = 8, normalize: bool = True,
                  decay: float = 1.0, only_prev_layer: bool = False) -> list[int]:
    """Top-``k`` expert ids at ``target_layer`` given the experts seen at
    earlier layers (reference cooccur.py:233-287), computed on the GPU.
    Uses the table's step buffers: not for use in the middle of a decode
    step."""
    table.end_step(False)
    for L, eids in seen_so_far.items():
        ids = [int(e) for e in eids]
        if ids and 0 <= int(L) < table.layers:
            table.observe_layer(int(L), torch.tensor(ids, dtype=torch.int32,
                                                     device=table.device), ordered=True)
    ids, n = table.predict_device(target_layer, k, normalize=normalize, decay=decay,
                                  only_prev_layer=only_prev_layer)
    out = ids[: int(n.item())].tolist()
    table.end_step(False)
    return out


__all__ = ["CooccurTable", "predict_layer"]
