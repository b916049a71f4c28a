"""Paged fused-MoE layer for MI355X: the reference's plug-in surface over HIP kernels.

Mirrors ``src/wisp/integrations/vllm/fused_moe.py`` of the reference:

* ``WISP_MODE`` (``paged`` default, ``resident``, ``copy``; legacy aliases
  ``day1``/``day2a``/``day2b``) and ``WISP_CAP_EXPERTS`` with the same
  resolution rules (reference 76-118);
* ``WispMoEState(cpu_w13, cpu_w2, cap_experts, mode, device, layer_idx)``
  with ``ensure_resident``, ``prime_identity``, ``resize_cap`` and the
  residency views ``slot_to_expert`` / ``expert_to_slot`` /
  ``expert_map_device`` / ``lru_tick`` / ``lru_clock`` / ``stats_*``
  (reference 126-490);
* ``install_wisp_moe(*, mode=None, cap_experts=None) -> bool`` and
  ``is_installed()``, patching ``create_weights``,
  ``process_weights_after_loading`` and ``forward_cuda`` of
  ``UnquantizedFusedMoEMethod`` (reference 660-1315).  When vLLM is not
  importable the patch targets the stand-in class of
  ``wisp.integrations.vllm.layer`` with the same methods.

Everything on the call path runs in ``libwisp_hip.so``: routing, the pager
(state lives on the GPU; the host views above are read back on demand), the
page-in copies and the expert kernels.  There is no PyTorch or CPU fallback.

Resident mode is the paged machinery with ``cap = E`` and the identity map
(slot ``e`` holds expert ``e``), so paged and resident outputs come from the
same kernels and are byte-identical.
"""
from __future__ import annotations

import ctypes as C
import logging
import os
import weakref
from typing import Any, Callable

import torch

from wisp_amd import _lib
from wisp_amd._lib import check, lib

logger = logging.getLogger("wisp.integrations.vllm.fused_moe")

_PATCHED_FLAG = "_wisp_patched"


# ---------------------------------------------------------------------------
# Mode handling (reference fused_moe.py:76-118)
# ---------------------------------------------------------------------------



def _require_device(t: torch.Tensor, dev: torch.device, name: str) -> None:
    """The kernels take raw device pointers: a tensor elsewhere (host memory,
    another GPU) would be read as device memory, so it is refused here."""
    if t.device.type != dev.type or (dev.index is not None and t.device.index != dev.index):
        raise ValueError(f"wisp: {name} is on {t.device}; the layer runs on {dev}")


def _check_out(out: torch.Tensor, like: torch.Tensor) -> None:
    """A caller's output buffer must be exactly what the kernels write: a
    contiguous [T, H] tensor of the activations' dtype on their device."""
    if out.shape != like.shape or out.dtype != like.dtype or not out.is_contiguous():
        raise ValueError(f"wisp: out must be a contiguous {tuple(like.shape)} {like.dtype} tensor")
    _require_device(out, like.device, "out")

class _Mode:
    COPY = "copy"          # full-tensor copy per forward (correctness only)
    RESIDENT = "resident"  # every expert resident, identity map
    PAGED = "paged"        # LRU paging of cap scratch slots (default)


_LEGACY_MODE_ALIASES = {"day1": _Mode.COPY, "day2a": _Mode.RESIDENT, "day2b": _Mode.PAGED}


def _resolve_mode() -> str:
    raw = os.environ.get("WISP_MODE", _Mode.PAGED).strip().lower()
    raw = _LEGACY_MODE_ALIASES.get(raw, raw)
    if raw not in (_Mode.COPY, _Mode.RESIDENT, _Mode.PAGED):
        logger.warning("WISP_MODE=%r unrecognised; defaulting to paged", raw)
        return _Mode.PAGED
    return raw


def _resolve_cap_experts(num_experts: int) -> int:
    """Paged-mode cap: ``WISP_CAP_EXPERTS`` unset -> ``min(E, 24)``; not an
    int -> ``E`` (with a warning); otherwise clamped to ``[2, E]``."""
    raw = os.environ.get("WISP_CAP_EXPERTS")
    if raw is None:
        return min(num_experts, 24)
    try:
        cap = int(raw)
    except ValueError:
        logger.warning("WISP_CAP_EXPERTS=%r is not an int; using num_experts=%d", raw, num_experts)
        return num_experts
    return max(2, min(cap, num_experts))


def _resolve_pagein_streams() -> int:
    """``WISP_PAGEIN_STREAMS``: 0 (default) issues page-in copies on the
    caller's stream; 1 or 2 uses that many side copy streams fenced with
    events (worth it only when independent work can overlap the copies)."""
    raw = os.environ.get("WISP_PAGEIN_STREAMS", "0")
    try:
        n = int(raw)
    except ValueError:
        logger.warning("WISP_PAGEIN_STREAMS=%r is not an int; using 0", raw)
        return 0
    return max(0, min(2, n))


def _resolve_pagein_engine() -> int:
    """``WISP_PAGEIN_ENGINE``: ``kernel`` (default) copies loaded experts with
    a GPU kernel that reads the pinned masters directly, so decode calls never
    wait for the host; ``memcpy`` uses hipMemcpyAsync issued by the host after
    it has read the pager's decision (the side-stream option applies to it)."""
    raw = os.environ.get("WISP_PAGEIN_ENGINE", "kernel").strip().lower()
    if raw not in ("kernel", "memcpy"):
        logger.warning("WISP_PAGEIN_ENGINE=%r is not 'kernel' or 'memcpy'; using kernel", raw)
        raw = "kernel"
    return _lib.WISP_PAGEIN_KERNEL if raw == "kernel" else _lib.WISP_PAGEIN_MEMCPY


def _resolve_packed_masters() -> bool:
    """``WISP_PACKED_MASTERS`` (default on): a bf16 state also keeps a
    packed copy of its masters (``wisp_pack_bf16``: the same values in ~0.77x
    the bytes for typical weights), which the copy-kernel engine pages in
    from and unpacks into the slot.  ``0`` pages the masters as they are."""
    return os.environ.get("WISP_PACKED_MASTERS", "1").strip().lower() not in (
        "0", "false", "no", "off")


class _PackedRef:
    """A weak reference to a (packed tensor, stride) pair."""

    def __init__(self, pair: tuple) -> None:
        self._t = weakref.ref(pair[0])
        self._stride = pair[1]

    def __call__(self):
        t = self._t()
        return None if t is None else (t, self._stride)


# packed master copies by (masters, their version counters): layers that
# share masters share the copy while any of them holds it
_PACKED_MASTERS: dict = {}


def _resolve_decode_fused() -> bool:
    """``WISP_DECODE_FUSED=1``: a one-token call whose top-k equals cap runs
    the pager, the page-in and w13 (per slot) as one launch instead of a
    pager launch and a page-in + w13 launch (``wisp_layer_set_decode_fused``).
    Off by default: the fused launch is ~2 us shorter per call that loads
    nothing, but its pager runs behind the w13 stream's loads."""
    return os.environ.get("WISP_DECODE_FUSED", "0").strip().lower() in ("1", "true", "yes", "on")


_DTYPES = {torch.float32: _lib.WISP_F32, torch.bfloat16: _lib.WISP_BF16}


def _check_master(t: torch.Tensor, name: str) -> None:
    if t.device.type != "cpu":
        raise ValueError(f"{name} must live in host memory")
    if t.dim() != 3 or t.stride(2) != 1 or t.stride(1) != t.shape[2]:
        raise ValueError(f"{name} must be [E, rows, cols] with each expert contiguous")


class _Workspace:
    """Per-layer device workspaces and the pinned decision record, grown on demand."""

    def __init__(self, device: torch.device, hidden: int, inter: int,
                 dtype: torch.dtype, fp8: bool = False) -> None:
        self.device, self.hidden, self.inter, self.dtype = device, hidden, inter, dtype
        self.fp8 = fp8
        self.pairs = 0
        self.record_words = 0
        self.work_bytes = 0
        self.work = None
        self.struct = _lib.Workspace()
        self.struct.struct_bytes = C.sizeof(_lib.Workspace)
        self.topk_w = self.topk_ids = self.slots = self.flags = self.loads = None
        self.act = self.record = self.record_dev = None

    def _retire(self) -> None:
        """Wait for every queued kernel before a buffer is replaced.  The
        pinned decision record is written by the pager kernel through its
        device mapping, which torch's host allocator cannot see, so dropping
        it while a queued pager still writes it could hand the block to the
        next pinned allocation mid-write; the device buffers may be in use on
        another stream than the one that allocated them.  Growth doubles, so
        this happens a handful of times per layer."""
        if self.record is not None or self.work is not None or self.pairs:
            torch.cuda.synchronize(self.device)

    def ensure(self, T: int, K: int, nslots: int) -> "_lib.Workspace":
        pairs = max(1, T * K)
        words = lib().wisp_record_words(T, K)
        need = 0
        if self.fp8 and self.hidden > 0:
            need = lib().wisp_moe_fp8_work_bytes(max(1, T), K, self.hidden, self.inter, nslots)
        elif self.dtype == torch.bfloat16 and self.hidden > 0:
            need = lib().wisp_moe_work_bytes(max(1, T), K, self.hidden, nslots)
        if pairs > self.pairs or words > self.record_words or need > self.work_bytes:
            self._retire()
        if pairs > self.pairs:
            self.pairs = max(pairs, 2 * self.pairs)
            dev = self.device
            self.topk_w = torch.empty(self.pairs, dtype=torch.float32, device=dev)
            self.topk_ids = torch.empty(self.pairs, dtype=torch.int32, device=dev)
            self.slots = torch.empty(self.pairs, dtype=torch.int32, device=dev)
            self.flags = torch.zeros(self.pairs + 1, dtype=torch.int32, device=dev)
            self.loads = torch.zeros(2 * self.pairs, dtype=torch.int32, device=dev)
            self.act = torch.empty(self.pairs * self.inter, dtype=self.dtype, device=dev)
        if words > self.record_words:
            self.record_words = max(words, 2 * self.record_words)
            self.record = torch.zeros(self.record_words, dtype=torch.int32, pin_memory=True)
            self.record_dev = torch.zeros(self.record_words, dtype=torch.int32,
                                          device=self.device)
        # the grouped (MFMA) paths' per-slot pair lists and per-pair outputs
        if need > self.work_bytes:
            self.work_bytes = max(need, 2 * self.work_bytes)
            self.work = torch.empty(self.work_bytes, dtype=torch.uint8, device=self.device)
        s = self.struct
        s.max_pairs = self.pairs
        s.topk_w, s.topk_ids = self.topk_w.data_ptr(), self.topk_ids.data_ptr()
        s.slots, s.act = self.slots.data_ptr(), self.act.data_ptr()
        s.flags, s.loads = self.flags.data_ptr(), self.loads.data_ptr()
        s.record, s.record_words = self.record.data_ptr(), self.record_words
        s.record_dev = self.record_dev.data_ptr()
        s.work = self.work.data_ptr() if self.work is not None else None
        s.work_bytes = self.work_bytes
        return s


class WispMoEState:
    """Per-layer paging state (reference ``WispMoEState``, fused_moe.py:126-236).

    Masters ``cpu_w13 [E, 2I, H]`` / ``cpu_w2 [E, H, I]`` stay in pinned host
    memory.  The HBM scratch is one slab per slot, ``[w13 | w2]``, so a miss
    is one copy when the masters are laid out the same way.  Pager state
    (``expert_map_device``, slot table, ticks, clock and counters) lives on
    the GPU and is updated by the pager kernel; the Python views below read
    it back when accessed.
    """

    def __init__(self, cpu_w13: torch.Tensor, cpu_w2: torch.Tensor, cap_experts: int,
                 mode: str, device: torch.device, layer_idx: int) -> None:
        if cpu_w13.dtype not in _DTYPES or cpu_w2.dtype != cpu_w13.dtype:
            raise NotImplementedError(f"wisp: expert dtype {cpu_w13.dtype} not supported "
                                      "(float32 and bfloat16 are)")
        _check_master(cpu_w13, "cpu_w13")
        _check_master(cpu_w2, "cpu_w2")
        E, two_i, H = cpu_w13.shape
        I = cpu_w2.shape[2]
        if cpu_w2.shape[0] != E:
            raise ValueError("cpu_w13 and cpu_w2 disagree on num_experts")
        # A pager-only state (shapes that are not a gated MLP) can page and
        # be inspected but not run forward.
        is_mlp = two_i == 2 * I and cpu_w2.shape[1] == H
        if not (1 <= cap_experts <= E):
            raise ValueError(f"cap_experts={cap_experts} outside [1, {E}]")
        self.layer_idx = int(layer_idx)
        self.num_experts = int(E)
        self.cap_experts = int(cap_experts)
        self.mode = mode
        self.hidden, self.inter = (int(H), int(I)) if is_mlp else (0, 0)
        self._w13_shape = tuple(cpu_w13.shape[1:])
        self._w2_shape = tuple(cpu_w2.shape[1:])
        self.dtype = cpu_w13.dtype
        self.cpu_w13 = cpu_w13 if cpu_w13.is_pinned() else cpu_w13.pin_memory()
        self.cpu_w2 = cpu_w2 if cpu_w2.is_pinned() else cpu_w2.pin_memory()
        self.device = torch.device(device)
        self._w13_elems = two_i * H
        self._w2_elems = cpu_w2.shape[1] * I
        # slab rounded up to 16 bytes so every slot stays 16-byte aligned
        per16 = 16 // cpu_w13.element_size()
        self._slab_elems = -(-(self._w13_elems + self._w2_elems) // per16) * per16
        self._alloc_scratch(self.cap_experts)
        dev = self.device
        self.expert_map_device = torch.full((E,), -1, dtype=torch.int32, device=dev)
        self._counters = torch.zeros(8, dtype=torch.int64, device=dev)
        self.stats_pred_hits = 0
        self._pf_record: torch.Tensor | None = None
        self._pf_words = 0
        self._pf_n = 0
        self._ws = _Workspace(dev, self.hidden, max(1, I), self.dtype)
        self._last_pairs = 0
        self._packed: torch.Tensor | None = None
        self._packed_stride = 0
        if (self.dtype == torch.bfloat16 and is_mlp and _resolve_packed_masters()
                and _resolve_pagein_engine() == _lib.WISP_PAGEIN_KERNEL):
            self._pack_masters()
        self._handle = C.c_void_p()
        self._desc = self._make_desc()
        check(lib().wisp_layer_create(C.byref(self._desc), C.byref(self._handle)),
              "wisp_layer_create")
        check(lib().wisp_layer_set_decode_fused(self._handle, int(_resolve_decode_fused())),
              "wisp_layer_set_decode_fused")

    # -- construction helpers ---------------------------------------------
    def _alloc_scratch(self, cap: int) -> None:
        (r13, c13), (r2, c2) = self._w13_shape, self._w2_shape
        self._scratch = torch.empty((cap, self._slab_elems), dtype=self.dtype, device=self.device)
        self.scratch_w13 = torch.as_strided(self._scratch, (cap, r13, c13),
                                            (self._slab_elems, c13, 1), 0)
        self.scratch_w2 = torch.as_strided(self._scratch, (cap, r2, c2),
                                           (self._slab_elems, c2, 1), self._w13_elems)
        self._slot_to_expert = torch.full((cap,), -1, dtype=torch.int32, device=self.device)
        self._lru_tick = torch.zeros(cap, dtype=torch.int64, device=self.device)

    def _pack_masters(self) -> None:
        """The masters' packed copy in pinned memory (no copy when the shape
        does not pack: H and I must be multiples of 64).  States over the
        same master tensors, unmodified since (torch's version counter),
        share one packed copy.  The copy is taken here: a state pages the
        masters as they were when it was built (the masters are written
        once, at weight loading, before the states exist)."""
        w13, w2 = self.cpu_w13, self.cpu_w2
        args = (self.num_experts, self.hidden, self.inter, w13.data_ptr(), w13.stride(0),
                w2.data_ptr(), w2.stride(0))
        key = args + (w13._version, w2._version)
        ref = _PACKED_MASTERS.get(key)
        hit = ref() if ref is not None else None
        if hit is not None:
            self._packed, self._packed_stride = hit
            return
        stride = lib().wisp_pack_bf16_stride(*args)
        if not stride:
            return
        packed = torch.empty(self.num_experts * stride, dtype=torch.uint8, pin_memory=True)
        check(lib().wisp_pack_bf16(*args, packed.data_ptr(), stride), "wisp_pack_bf16")
        self._packed, self._packed_stride = packed, int(stride)
        for k in [k for k, r in _PACKED_MASTERS.items() if r() is None]:
            del _PACKED_MASTERS[k]
        _PACKED_MASTERS[key] = _PackedRef((packed, int(stride)))

    @property
    def packed_bytes_per_expert(self) -> int:
        """Bytes one page-in moves over the host link per expert: the packed
        stride, or the expert's plain bytes without a packed copy."""
        if self._packed is not None:
            return self._packed_stride
        return (self._w13_elems + self._w2_elems) * self.cpu_w13.element_size()

    def _make_desc(self) -> "_lib.LayerDesc":
        d = _lib.LayerDesc()
        d.struct_bytes = C.sizeof(_lib.LayerDesc)
        d.num_experts, d.cap = self.num_experts, self.cap_experts
        d.hidden, d.inter = self.hidden, self.inter
        d.dtype = _DTYPES[self.dtype]
        d.pagein_streams = _resolve_pagein_streams()
        d.pagein_engine = _resolve_pagein_engine()
        d.w13_elems, d.w2_elems = self._w13_elems, self._w2_elems
        d.mode = _lib.WISP_MODE_RESIDENT if self.mode == _Mode.RESIDENT else _lib.WISP_MODE_PAGED
        d.scratch_w13, d.scratch_w13_stride = self.scratch_w13.data_ptr(), self._slab_elems
        d.scratch_w2, d.scratch_w2_stride = self.scratch_w2.data_ptr(), self._slab_elems
        d.master_w13, d.master_w13_stride = self.cpu_w13.data_ptr(), self.cpu_w13.stride(0)
        d.master_w2, d.master_w2_stride = self.cpu_w2.data_ptr(), self.cpu_w2.stride(0)
        d.expert_map = self.expert_map_device.data_ptr()
        d.slot_to_expert = self._slot_to_expert.data_ptr()
        d.lru_tick = self._lru_tick.data_ptr()
        d.counters = self._counters.data_ptr()
        if self._packed is not None:
            d.packed_master, d.packed_stride = self._packed.data_ptr(), self._packed_stride
        return d

    def __del__(self) -> None:
        h = getattr(self, "_handle", None)
        if h is not None and h.value:
            try:
                lib().wisp_layer_destroy(h)
            except Exception:  # pragma: no cover - interpreter shutdown
                pass
            self._handle = C.c_void_p()

    # -- host views of the device state (read back on access) -------------
    def _ctr(self, i: int) -> int:
        return int(self._counters[i].item())

    def _set_ctr(self, i: int, v: int) -> None:
        self._counters[i] = int(v)

    slot_to_expert = property(lambda self: self._slot_to_expert.tolist())
    lru_tick = property(lambda self: self._lru_tick.tolist())
    lru_clock = property(lambda self: self._ctr(0))
    stats_forward = property(lambda self: self._ctr(1), lambda self, v: self._set_ctr(1, v))
    stats_miss = property(lambda self: self._ctr(2), lambda self, v: self._set_ctr(2, v))
    stats_evict = property(lambda self: self._ctr(3), lambda self, v: self._set_ctr(3, v))
    stats_hits = property(lambda self: self._ctr(4), lambda self, v: self._set_ctr(4, v))
    stats_pred_total = property(lambda self: self._ctr(5), lambda self, v: self._set_ctr(5, v))

    @property
    def expert_to_slot(self) -> dict[int, int]:
        return {e: s for s, e in enumerate(self.slot_to_expert) if e != -1}

    @property
    def last_unique_experts(self) -> set[int]:
        """Experts routed to by the last layer call (reference 1173-1177)."""
        if self._last_pairs == 0:
            return set()
        return set(torch.unique(self._ws.topk_ids[: self._last_pairs]).tolist())

    @property
    def last_topk(self) -> tuple[torch.Tensor, torch.Tensor]:
        """(weights, ids) of the last layer call, as ``[T, K]`` device tensors."""
        T, K = self._last_shape
        return (self._ws.topk_w[: T * K].view(T, K), self._ws.topk_ids[: T * K].view(T, K))

    @property
    def last_slots(self) -> torch.Tensor:
        T, K = self._last_shape
        return self._ws.slots[: T * K].view(T, K)

    @property
    def last_record(self) -> torch.Tensor:
        """The pinned decision record of the last paged call (waits for the
        device to finish the calls already queued; decode calls on the
        copy-kernel engine keep their record in device memory until asked)."""
        check(lib().wisp_layer_sync_record(self._handle, C.byref(self._ws.struct)),
              "last_record")
        return self._ws.record

    @property
    def pagein_engine(self) -> str:
        """``"kernel"`` or ``"memcpy"``: the page-in engine in use (the kernel
        engine falls back to memcpy for masters that are not pinned)."""
        eng = lib().wisp_layer_pagein_engine(self._handle)
        return "kernel" if eng == _lib.WISP_PAGEIN_KERNEL else "memcpy"

    # -- reference API ------------------------------------------------------
    def prime_identity(self) -> None:
        """Copy expert ``i`` into slot ``i`` for every expert and set the
        identity map (reference 242-258); requires ``cap == E``."""
        if self.cap_experts != self.num_experts:
            raise AssertionError("prime_identity requires cap == num_experts")
        check(lib().wisp_layer_prime_identity(self._handle, _lib.stream_handle()),
              "prime_identity")

    def ensure_resident(self, needed_experts: torch.Tensor) -> None:
        """Make every expert in ``needed_experts`` resident (one LRU call,
        reference 264-358).  Raises ``RuntimeError`` mentioning "sub-batch"
        when more distinct experts are needed than ``cap_experts``."""
        ids = needed_experts.reshape(-1).to(device=self.device, dtype=torch.int32).contiguous()
        n = ids.numel()
        ws = self._ws.ensure(n, 1, self.cap_experts)
        rc = lib().wisp_layer_ensure_resident(self._handle, ids.data_ptr() if n else None, n,
                                              C.byref(ws), _lib.stream_handle())
        check(rc, "ensure_resident")

    def forward(self, x: torch.Tensor, router_logits: torch.Tensor, top_k: int,
                renormalize: bool = True, out: torch.Tensor | None = None,
                algo: int = _lib.WISP_ALGO_AUTO) -> torch.Tensor:
        """One layer call: ``x [T, H]``, ``router_logits [T, E]`` -> ``[T, H]``."""
        if self.hidden == 0:
            raise ValueError("wisp: expert tensors are not a gated MLP (w13 [E, 2I, H], "
                             "w2 [E, H, I]); this state can page but not run forward")
        if x.dtype != self.dtype or x.dim() != 2 or x.shape[1] != self.hidden:
            raise ValueError(f"x must be [T, {self.hidden}] {self.dtype}")
        if router_logits.shape != (x.shape[0], self.num_experts):
            raise ValueError(f"router_logits must be [T, {self.num_experts}]")
        _require_device(x, self.device, "x")
        _require_device(router_logits, self.device, "router_logits")
        if router_logits.dtype not in _DTYPES:
            router_logits = router_logits.float()
        x = x.contiguous()
        router_logits = router_logits.contiguous()
        T = x.shape[0]
        if out is None:
            out = torch.empty_like(x)
        else:
            _check_out(out, x)
        ws = self._ws.ensure(T, top_k, self.cap_experts)
        rc = lib().wisp_layer_forward(self._handle, x.data_ptr(), router_logits.data_ptr(),
                                      _DTYPES[router_logits.dtype], T, int(top_k),
                                      int(bool(renormalize)), out.data_ptr(), C.byref(ws),
                                      int(algo), _lib.stream_handle())
        self._last_pairs, self._last_shape = T * top_k, (T, top_k)
        check(rc, "wisp_layer_forward")
        return out

    def prefetch_async(self, predicted_experts) -> None:
        """Speculatively page ``predicted_experts`` into this layer (reference
        360-433): the decisions run on the current stream, the copies on the
        layer's side stream, and the layer's next call waits for them.  The
        iteration order of ``predicted_experts`` fixes which slot each expert
        takes; experts of the last call and the predicted ones are never
        evicted."""
        ids = [int(e) for e in predicted_experts]
        if not ids:
            self._pf_n = 0  # nothing predicted: no decisions (last_prefetch is empty)
            return
        t = torch.tensor(ids, dtype=torch.int32, device=self.device)
        self._prefetch(t, None, len(ids), ordered=True, count_pred=False)

    def _prefetch(self, ids: torch.Tensor, n_dev: torch.Tensor | None, n: int, ordered: bool,
                  count_pred: bool) -> None:
        words = lib().wisp_prefetch_record_words(n)
        if self._pf_record is None or self._pf_words < words:
            if self._pf_record is not None:
                # the last prefetch's copies on the side stream may still
                # read the old record
                torch.cuda.synchronize(self.device)
            self._pf_words = max(words, lib().wisp_prefetch_record_words(self.num_experts))
            self._pf_record = torch.zeros(self._pf_words, dtype=torch.int32, device=self.device)
        self._pf_n = n
        last = self._ws.topk_ids if self._last_pairs else None
        check(lib().wisp_layer_prefetch(
            self._handle, ids.data_ptr(), n_dev.data_ptr() if n_dev is not None else None, n,
            int(bool(ordered)), int(bool(count_pred)),
            last.data_ptr() if last is not None else None, self._last_pairs,
            self._pf_record.data_ptr(), self._pf_words, _lib.stream_handle()), "prefetch")

    @property
    def last_prefetch(self) -> dict:
        """Decisions of the last prefetch: ``{"evicted": [(e, s)], "loaded":
        [(e, s)], "clock": bool}`` (waits for the device)."""
        if self._pf_record is None or self._pf_n == 0:
            return {"evicted": [], "loaded": [], "clock": False}
        r = self._pf_record.cpu().tolist()
        n = self._pf_n
        ev, ld = r[4:4 + 2 * n], r[4 + 2 * n:4 + 4 * n]
        return {"evicted": [(ev[2 * i], ev[2 * i + 1]) for i in range(r[0])],
                "loaded": [(ld[2 * i], ld[2 * i + 1]) for i in range(r[1])],
                "clock": bool(r[2])}

    def pagein_stats(self) -> tuple[float, float]:
        """(milliseconds, bytes) of page-in copies since the last query,
        counting the calls made while timing is on (``profile(True)``)."""
        ms, nbytes = C.c_float(), C.c_double()
        check(lib().wisp_layer_last_pagein(self._handle, C.byref(ms), C.byref(nbytes)),
              "pagein_stats")
        return float(ms.value), float(nbytes.value)

    def profile(self, enable: bool = True) -> dict:
        """Read and reset the execution time (ms, dispatch timestamps) of the
        ``w13`` and ``w2`` expert kernels of all layer calls since the last
        read, the number of ``calls`` and of ``w13_calls`` (calls whose w13
        time is in ``w13``: a decode call that pages experts in runs its w13
        inside the page-in launch, which is timed as page-in); then switch
        timing on or off.  The switch covers ``pagein_stats`` too; timing is
        off by default, since its events lengthen the stream.
        ``w2_noload`` / ``w2_noload_calls``: the w2 time of the calls whose
        fused page-in + w13 launch copied nothing (the calls behind ``w13``
        on that path), so both stages can be averaged over one set of calls."""
        a, b, n, n13 = C.c_double(), C.c_double(), C.c_int64(), C.c_int64()
        b_nl, n_nl = C.c_double(), C.c_int64()
        check(lib().wisp_layer_profile_noload(self._handle, C.byref(b_nl), C.byref(n_nl)),
              "profile")
        check(lib().wisp_layer_profile(self._handle, int(enable), C.byref(a), C.byref(b),
                                       C.byref(n), C.byref(n13)), "profile")
        return {"w13": float(a.value), "w2": float(b.value), "calls": int(n.value),
                "w13_calls": int(n13.value), "w2_noload": float(b_nl.value),
                "w2_noload_calls": int(n_nl.value)}

    def resize_cap(self, new_cap: int) -> None:
        """Resize the scratch to ``new_cap`` slots at a drained barrier
        (reference 439-490): grow keeps every resident expert and adds free
        slots; shrink drops the experts of the tail slots (they re-page on
        demand)."""
        new_cap = max(2, min(int(new_cap), self.num_experts))
        old_cap = self.cap_experts
        if new_cap == old_cap:
            return
        torch.cuda.synchronize(self.device)
        old_scratch, old_s2e, old_tick = self._scratch, self._slot_to_expert, self._lru_tick
        self._alloc_scratch(new_cap)
        keep = min(old_cap, new_cap)
        self._scratch[:keep].copy_(old_scratch[:keep])
        self._slot_to_expert[:keep].copy_(old_s2e[:keep])
        self._lru_tick[:keep].copy_(old_tick[:keep])
        if new_cap < old_cap:
            tail = old_s2e[new_cap:]
            dropped = tail[tail >= 0].long()
            self.expert_map_device.index_fill_(0, dropped, -1)
        self.cap_experts = new_cap
        torch.cuda.synchronize(self.device)
        self._desc = self._make_desc()
        check(lib().wisp_layer_set_scratch(self._handle, self.scratch_w13.data_ptr(),
                                           self.scratch_w2.data_ptr(), new_cap,
                                           self._slot_to_expert.data_ptr(),
                                           self._lru_tick.data_ptr()), "resize_cap")


# ---------------------------------------------------------------------------
# Process-wide state (reference 497-593)
# ---------------------------------------------------------------------------

_WISP_RUNTIME_CONFIG: dict[str, Any] = {"mode": _Mode.RESIDENT, "cap_experts_override": None}
_LAYER_STATES: list[WispMoEState] = []
_LAYER_BY_ID: dict[int, WispMoEState] = {}


def resize_layer_caps(new_cap: int) -> int:
    """Resize every registered layer's scratch; returns the number resized."""
    for st in _LAYER_STATES:
        st.resize_cap(new_cap)
    if _LAYER_STATES:
        torch.cuda.empty_cache()
    return len(_LAYER_STATES)


def current_layer_cap() -> int | None:
    return _LAYER_STATES[0].cap_experts if _LAYER_STATES else None


def num_registered_layers() -> int:
    return len(_LAYER_STATES)


def num_experts_per_layer() -> int | None:
    return _LAYER_STATES[0].num_experts if _LAYER_STATES else None


def expert_bytes_per_cap() -> int:
    """HBM bytes one scratch slot holds (its w13 and w2), summed over the
    registered layers: what changing the per-layer cap by one slot frees or
    claims (reference 571-582)."""
    total = 0
    for st in _LAYER_STATES:
        total += st.scratch_w13[0].numel() * st.scratch_w13.element_size()
        total += st.scratch_w2[0].numel() * st.scratch_w2.element_size()
    return total


def snapshot_expert_stats(reset: bool = True) -> dict:
    miss = sum(s.stats_miss for s in _LAYER_STATES)
    hit = sum(s.stats_hits for s in _LAYER_STATES)
    fwd = sum(s.stats_forward for s in _LAYER_STATES)
    ws = max((len(s.last_unique_experts) for s in _LAYER_STATES), default=0)
    if reset:
        for s in _LAYER_STATES:
            s.stats_miss = 0
            s.stats_hits = 0
            s.stats_forward = 0
    return {"miss": miss, "hit": hit, "forward": fwd, "ws": ws}


# ---------------------------------------------------------------------------
# Patched methods (reference 660-1237)
# ---------------------------------------------------------------------------


def _slab_masters(num_experts: int, hidden: int, inter: int, dtype: torch.dtype,
                  pin: bool) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Host masters as one ``[w13 | w2]`` slab per expert (one copy per miss)."""
    slab = 3 * inter * hidden
    buf = torch.empty((num_experts, slab), dtype=dtype, pin_memory=pin)
    w13 = torch.as_strided(buf, (num_experts, 2 * inter, hidden), (slab, hidden, 1), 0)
    w2 = torch.as_strided(buf, (num_experts, hidden, inter), (slab, inter, 1), 2 * inter * hidden)
    return buf, w13, w2


def _patched_create_weights(self, layer: torch.nn.Module, num_experts: int, hidden_size: int,
                            intermediate_size_per_partition: int, params_dtype: torch.dtype,
                            **extra_weight_attrs) -> None:
    """Allocate the expert masters in host memory (reference 673-759); the
    loader's ``param.data.copy_`` then writes them without touching HBM."""
    if getattr(self.moe, "has_bias", False):
        raise NotImplementedError(
            "wisp: has_bias=True MoE checkpoints are not supported (expert biases are not paged)")
    if not getattr(self.moe, "is_act_and_mul", True):
        raise NotImplementedError("wisp: only gated (act-and-mul) experts are supported")
    buf, w13, w2 = _slab_masters(num_experts, hidden_size, intermediate_size_per_partition,
                                 params_dtype, pin=False)
    w13_p = torch.nn.Parameter(w13, requires_grad=False)
    w2_p = torch.nn.Parameter(w2, requires_grad=False)
    layer.register_parameter("w13_weight", w13_p)
    layer.register_parameter("w2_weight", w2_p)
    try:  # vLLM's weight attributes (loader hooks), when vLLM is present
        from vllm.model_executor.utils import set_weight_attrs
        set_weight_attrs(w13_p, extra_weight_attrs)
        set_weight_attrs(w2_p, extra_weight_attrs)
    except ImportError:
        for p in (w13_p, w2_p):
            for k, v in extra_weight_attrs.items():
                setattr(p, k, v)
    layer._wisp_cpu_slab = buf
    layer._wisp_cpu_pin_w13 = w13
    layer._wisp_cpu_pin_w2 = w2


def _patched_process_weights_after_loading(self, layer: torch.nn.Module) -> None:
    """Pin the masters and build the layer's paging state (reference 762-927)."""
    if getattr(layer, "_wisp_state", None) is not None or \
            getattr(layer, "_wisp_cpu_w13", None) is not None:
        return
    type(self)._wisp_original_process_weights_after_loading(self, layer)
    if getattr(layer, "w13_weight", None) is None or getattr(layer, "w2_weight", None) is None:
        return
    device = torch.device("cuda", torch.cuda.current_device())
    slab = getattr(layer, "_wisp_cpu_slab", None)
    if slab is not None:
        pinned = slab if slab.is_pinned() else slab.pin_memory()
        E, n = pinned.shape
        H = layer._wisp_cpu_pin_w13.shape[2]
        I = layer._wisp_cpu_pin_w2.shape[2]
        cpu_w13 = torch.as_strided(pinned, (E, 2 * I, H), (n, H, 1), 0)
        cpu_w2 = torch.as_strided(pinned, (E, H, I), (n, I, 1), 2 * I * H)
        layer._wisp_cpu_slab = pinned
    else:  # weights were created elsewhere: move them to pinned host memory
        cpu_w13 = layer.w13_weight.data.cpu().pin_memory()
        cpu_w2 = layer.w2_weight.data.cpu().pin_memory()
    layer._wisp_cpu_pin_w13, layer._wisp_cpu_pin_w2 = cpu_w13, cpu_w2

    mode: str = _WISP_RUNTIME_CONFIG["mode"]
    if mode == _Mode.COPY:
        layer._wisp_cpu_w13, layer._wisp_cpu_w2 = cpu_w13, cpu_w2
        layer._wisp_state = None
        _placeholders(layer, cpu_w13.dtype, device)
        return
    E = int(cpu_w13.shape[0])
    override = _WISP_RUNTIME_CONFIG["cap_experts_override"]
    if mode == _Mode.RESIDENT:
        cap = E
    else:
        cap = override if override is not None else _resolve_cap_experts(E)
    state = WispMoEState(cpu_w13, cpu_w2, cap, mode, device, len(_LAYER_STATES))
    _LAYER_STATES.append(state)
    _LAYER_BY_ID[id(layer)] = state
    if mode == _Mode.RESIDENT:
        state.prime_identity()
    layer._wisp_state = state
    _placeholders(layer, cpu_w13.dtype, device)
    logger.info("wisp[%s]: layer %d: num_experts=%d cap_experts=%d pinned=%.2f GiB "
                "scratch=%.2f GiB", mode, state.layer_idx, E, cap,
                E * state._slab_elems * cpu_w13.element_size() / 2**30,
                cap * state._slab_elems * cpu_w13.element_size() / 2**30)


def _placeholders(layer: torch.nn.Module, dtype: torch.dtype, device: torch.device) -> None:
    """0-element device placeholders on the layer's weight params (reference 896-898)."""
    layer.w13_weight.data = torch.empty(0, dtype=dtype, device=device)
    layer.w2_weight.data = torch.empty(0, dtype=dtype, device=device)


def _route_and_experts(x, router_logits, top_k, renormalize, w13, w2) -> torch.Tensor:
    """All experts resident in ``w13 [E, 2I, H]`` / ``w2 [E, H, I]`` device
    tensors: route, then run the expert kernels with slot = expert id."""
    T, H = x.shape
    E = w13.shape[0]
    I = w2.shape[2]
    dev = x.device
    for t, name in ((router_logits, "router_logits"), (w13, "w13"), (w2, "w2")):
        _require_device(t, dev, name)
    st = _lib.stream_handle()
    x = x.contiguous()
    logits = router_logits if router_logits.dtype in _DTYPES else router_logits.float()
    logits = logits.contiguous()
    topk_w = torch.empty((T, top_k), dtype=torch.float32, device=dev)
    topk_ids = torch.empty((T, top_k), dtype=torch.int32, device=dev)
    check(lib().wisp_route_topk_softmax(logits.data_ptr(), _DTYPES[logits.dtype], T, E, top_k,
                                        int(bool(renormalize)), topk_w.data_ptr(),
                                        topk_ids.data_ptr(), None, st), "route")
    act = torch.empty((max(1, T * top_k), I), dtype=x.dtype, device=dev)
    out = torch.empty_like(x)
    nbytes = lib().wisp_moe_work_bytes(max(1, T), top_k, H, E)
    work = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    check(lib().wisp_moe_experts(x.data_ptr(), _DTYPES[x.dtype], T, H, I, top_k,
                                 topk_w.data_ptr(), topk_ids.data_ptr(), E, w13.data_ptr(),
                                 w13.stride(0), w2.data_ptr(), w2.stride(0), act.data_ptr(),
                                 out.data_ptr(), work.data_ptr(), nbytes, _lib.WISP_ALGO_AUTO,
                                 st), "experts")
    return out


# Arguments of vLLM's forward_cuda this path supports only at these values
# (softmax routing, SiLU experts, no grouped top-k, no EPLB).  The EPLB
# bookkeeping tensors are ignored while enable_eplb is False.
_SUPPORTED_ONLY = {
    "use_grouped_topk": False, "topk_group": None, "num_expert_group": None,
    "custom_routing_function": None, "scoring_func": "softmax", "routed_scaling_factor": 1.0,
    "e_score_correction_bias": None, "apply_router_weight_on_input": False,
    "activation": "silu", "enable_eplb": False,
}


def _check_supported(kw: dict) -> None:
    for name, want in _SUPPORTED_ONLY.items():
        v = kw.get(name, want)
        if (v is not None) if want is None else (v != want):
            raise NotImplementedError(f"wisp: {name}={v!r} is not supported on the paged "
                                      "MoE path")


def _patched_forward_cuda(self, layer: torch.nn.Module, x: torch.Tensor, *args: Any,
                          **kwargs: Any):
    """Mode dispatch (reference 930-987)."""
    state: WispMoEState | None = getattr(layer, "_wisp_state", None)
    if state is None and getattr(layer, "_wisp_cpu_w13", None) is not None:
        # copy mode: stage every expert into a fresh device buffer per call
        return _copy_mode_forward(layer, x, *args, **kwargs)
    if state is None:
        return type(self)._wisp_original_forward_cuda(self, layer, x, *args, **kwargs)
    return _wisp_forward_cuda_paged(self, layer, x, state, *args, **kwargs)


def _bind_call_args(use_grouped_topk: bool, top_k: int, router_logits: torch.Tensor,
                    renormalize: bool, topk_group: int | None = None,
                    num_expert_group: int | None = None, global_num_experts: int = -1,
                    expert_map: torch.Tensor | None = None,
                    custom_routing_function: Callable | None = None,
                    scoring_func: str = "softmax", routed_scaling_factor: float = 1.0,
                    e_score_correction_bias: torch.Tensor | None = None,
                    apply_router_weight_on_input: bool = False, activation: str = "silu",
                    enable_eplb: bool = False, expert_load_view: torch.Tensor | None = None,
                    logical_to_physical_map: torch.Tensor | None = None,
                    logical_replica_count: torch.Tensor | None = None) -> dict:
    """vLLM's ``forward_cuda`` signature (reference 990-1013)."""
    return dict(locals())


def _copy_mode_forward(layer, x, *args, **kwargs):
    a = _bind_call_args(*args, **kwargs)
    if a["expert_map"] is not None:
        raise NotImplementedError("wisp: expert-parallel expert_map is not supported")
    _check_supported(a)
    w13 = layer._wisp_cpu_w13.to(x.device, non_blocking=True)
    w2 = layer._wisp_cpu_w2.to(x.device, non_blocking=True)
    return _route_and_experts(x, a["router_logits"], a["top_k"], a["renormalize"], w13, w2)


def _wisp_forward_cuda_paged(self, layer: torch.nn.Module, x: torch.Tensor,
                             state: WispMoEState, *args: Any, **kwargs: Any):
    """Paged (and resident) layer call: routing, pager, page-in and experts
    all in ``libwisp_hip.so`` (reference 990-1237)."""
    a = _bind_call_args(*args, **kwargs)
    if a["expert_map"] is not None:
        # The reference warns and falls back to the upstream kernel here
        # (1019-1045); expert parallelism is not part of this path.
        raise NotImplementedError("wisp: a caller-supplied expert_map (EP) is not supported "
                                  "on the paged MoE path")
    _check_supported(a)
    if getattr(layer, "zero_expert_num", 0):
        raise NotImplementedError("wisp: zero experts are not supported")
    out = state.forward(x, a["router_logits"], a["top_k"], a["renormalize"])
    if state.mode == _Mode.PAGED:
        _prefetch_after_forward(state)
    return out


# ---------------------------------------------------------------------------
# Cross-layer speculative prefetch (reference 596-650, 1173-1233)
# ---------------------------------------------------------------------------

_COOCCUR_TABLE: Any = None  # None: not loaded yet; False: disabled


def _flag(name: str) -> bool:
    return os.environ.get(name, "0").strip().lower() in ("1", "true", "yes")


def _maybe_load_cooccur(state: WispMoEState) -> Any:
    """The process-wide co-occurrence table, sized for the registered
    layers: warm from ``WISP_COOCCUR_PATH`` or cold when
    ``WISP_COOCCUR_ONLINE`` is set; None when neither (prefetch then does
    nothing, as in the reference)."""
    global _COOCCUR_TABLE
    if _COOCCUR_TABLE is not None:
        return _COOCCUR_TABLE or None
    from .cooccur import CooccurTable
    path = os.environ.get("WISP_COOCCUR_PATH", "").strip()
    online = _flag("WISP_COOCCUR_ONLINE")
    if not path and not online:
        return None
    layers = max(len(_LAYER_STATES), state.layer_idx + 1)
    try:
        if path and os.path.isfile(path):
            _COOCCUR_TABLE = CooccurTable.load(path, layers, state.num_experts, state.device)
            logger.info("wisp.vllm: loaded warm cooccur table from %s (%d observed steps)",
                        path, _COOCCUR_TABLE.num_steps_observed)
        else:
            _COOCCUR_TABLE = CooccurTable(layers, state.num_experts, state.device)
            logger.info("wisp.vllm: cooccur table starts cold (online=%s)", online)
    except Exception as e:  # pragma: no cover - bad file
        logger.warning("wisp.vllm: cooccur init failed: %s - disabling", e)
        _COOCCUR_TABLE = False
        return None
    return _COOCCUR_TABLE


def _reset_cooccur() -> None:
    """Forget the process-wide table (the next paged call reloads it)."""
    global _COOCCUR_TABLE
    _COOCCUR_TABLE = None


def _prefetch_after_forward(state: WispMoEState) -> None:
    """Post-forward step of a paged layer with ``WISP_PREFETCH`` set
    (reference 1173-1233): record this layer's experts for the step, predict
    the next layer's ``max(8, cap // 2)`` experts (normalised, decay 0.5) and
    prefetch them into it; at the last layer learn the step when
    ``WISP_COOCCUR_ONLINE`` is set, then clear it.  All of it is queued on
    the current stream; nothing waits for the device."""
    if not _flag("WISP_PREFETCH") or state._last_pairs == 0:
        return
    table = _maybe_load_cooccur(state)
    if table is None or state.layer_idx >= table.layers:
        return
    table.observe_layer(state.layer_idx, state._ws.topk_ids, state._last_pairs)
    nxt = state.layer_idx + 1
    if nxt < len(_LAYER_STATES) and nxt < table.layers:
        ns = _LAYER_STATES[nxt]
        k = max(8, ns.cap_experts // 2)
        ids, n_dev = table.predict_device(nxt, k, normalize=True, decay=0.5)
        ns._prefetch(ids, n_dev, min(k, table.experts), ordered=False, count_pred=True)
    if state.layer_idx == len(_LAYER_STATES) - 1:
        table.end_step(_flag("WISP_COOCCUR_ONLINE"))


# ---------------------------------------------------------------------------
# Install (reference 1245-1315)
# ---------------------------------------------------------------------------


def _method_class():
    """vLLM's ``UnquantizedFusedMoEMethod`` if importable, else the local stand-in."""
    try:
        from vllm.model_executor.layers.fused_moe.unquantized_fused_moe_method import (  # noqa
            UnquantizedFusedMoEMethod,
        )
    except ImportError:
        from .layer import UnquantizedFusedMoEMethod
    return UnquantizedFusedMoEMethod


def install_wisp_moe(*, mode: str | None = None, cap_experts: int | None = None) -> bool:
    """Idempotent install: records the runtime config (``WISP_MODE`` when
    ``mode`` is None; ``cap_experts`` overrides ``WISP_CAP_EXPERTS``) and
    patches the MoE method class once.  True iff this call patched."""
    lib()  # fail loudly now if the HIP library is missing
    cls = _method_class()
    _WISP_RUNTIME_CONFIG["mode"] = mode if mode is not None else _resolve_mode()
    _WISP_RUNTIME_CONFIG["cap_experts_override"] = cap_experts
    if getattr(cls, _PATCHED_FLAG, False):
        logger.debug("wisp: already patched; runtime config refreshed to mode=%s cap=%s",
                     _WISP_RUNTIME_CONFIG["mode"], cap_experts)
        return False
    cls._wisp_original_create_weights = cls.create_weights
    cls._wisp_original_process_weights_after_loading = cls.process_weights_after_loading
    cls._wisp_original_forward_cuda = cls.forward_cuda
    cls.create_weights = _patched_create_weights
    cls.process_weights_after_loading = _patched_process_weights_after_loading
    cls.forward_cuda = _patched_forward_cuda
    setattr(cls, _PATCHED_FLAG, True)
    logger.info("wisp: patched %s.%s (mode=%s cap_experts=%s)", cls.__module__, cls.__name__,
                _WISP_RUNTIME_CONFIG["mode"], cap_experts)
    # Also page the block-FP8 MoE method, best effort, as the reference does
    # (1297-1303): a failure there must not break the unquantised path.
    try:
        from .fused_moe_fp8 import install_wisp_fp8
        install_wisp_fp8()
    except Exception as e:  # pragma: no cover - depends on the host's vLLM
        logger.warning("wisp: FP8 MoE patch not applied (%s)", e)
    return True


def is_installed() -> bool:
    return bool(getattr(_method_class(), _PATCHED_FLAG, False))


__all__ = ["install_wisp_moe", "is_installed", "WispMoEState"]
