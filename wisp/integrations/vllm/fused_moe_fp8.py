"""Block-FP8 paged MoE for MI355X: the reference's FP8 plug-in surface over HIP kernels.

Mirrors ``src/wisp/integrations/vllm/fused_moe_fp8.py`` of the reference:

* ``_resolve_cap_experts`` (48-58): ``WISP_CAP_EXPERTS`` unset or not an int
  -> ``min(E, 24)``; otherwise clamped to ``[8, E]`` (the lower bound wins
  when ``E < 8``);
* ``WispMoEStateFP8(cpu_w13, cpu_w2, cpu_s13, cpu_s2, cap_experts, device,
  layer_idx)`` (61-145): pages the (weight, scale) pairs of w13 and w2 per
  expert with the same LRU rules as the unquantised state, and exposes
  ``scratch_w13/w2/s13/s2``, ``slot_to_expert``, ``expert_to_slot``,
  ``expert_map_device``, ``lru_tick``, ``lru_clock``, ``stats_*`` and
  ``quant_config``;
* ``install_wisp_fp8()`` / ``is_fp8_installed()`` (362-390), patching
  ``create_weights``, ``process_weights_after_loading`` and ``apply`` of
  ``Fp8MoEMethod`` (vLLM's when importable, else the stand-in of
  ``wisp.integrations.vllm.layer``).

Weights are float8_e4m3fn with float32 block scales
``s13 [E, 2*ceil(I/bn), ceil(H/bk)]`` / ``s2 [E, ceil(H/bn), ceil(I/bk)]``;
activations are bfloat16.  The expert math is vLLM's fp8_w8a8 block path
(per-token-group activation quantisation, block-scaled GEMMs), computed by
``wisp_moe_experts_fp8`` in ``libwisp_hip.so`` on the MI355X's fp8 MFMA.

Host layout.  The patched ``create_weights`` allocates one pinned host slab
per expert, ``[w13 | w2 | s13 | s2]``, and registers views of it as the four
parameters, so the checkpoint loader writes the slab in place.  The masters
are then pinned without a second copy (the reason the reference keeps its
FP8 weight masters pageable, 215-223) and a miss moves one contiguous range;
the HBM scratch uses the same slab per slot.  Masters handed over as four
separate tensors are used where they lie: pinned ones feed the copy kernel,
pageable ones the memcpy engine (whose hipMemcpyAsync stages them).
"""
from __future__ import annotations

import ctypes as C
import logging
import math
import os
from types import SimpleNamespace
from typing import Any

import torch

from wisp_amd import _lib
from wisp_amd._lib import check, lib
from .fused_moe import (WispMoEState, _Mode, _require_device, _resolve_pagein_engine,
                        _resolve_pagein_streams, _Workspace)

logger = logging.getLogger("wisp.integrations.vllm.fused_moe_fp8")

_PATCHED_FLAG = "_wisp_fp8_patched"
FP8 = torch.float8_e4m3fn

# Registry of FP8 layer states (separate from the unquantised registry).
_FP8_LAYER_STATES: list["WispMoEStateFP8"] = []


def _resolve_cap_experts(num_experts: int) -> int:
    """FP8 cap: unset or not an int -> ``min(E, 24)``; else ``max(8, min(cap, E))``."""
    raw = os.environ.get("WISP_CAP_EXPERTS")
    if raw is None:
        return min(num_experts, 24)
    try:
        cap = int(raw)
    except ValueError:
        return min(num_experts, 24)
    return max(8, min(cap, num_experts))


class Fp8SlabLayout:
    """Byte layout of one expert's ``[w13 | w2 | s13 | s2]`` slab."""

    def __init__(self, hidden: int, inter: int, block: tuple[int, int]) -> None:
        bn, bk = int(block[0]), int(block[1])
        H, I = int(hidden), int(inter)
        self.hidden, self.inter, self.block = H, I, (bn, bk)
        self.s13_shape = (2 * math.ceil(I / bn), math.ceil(H / bk))
        self.s2_shape = (math.ceil(H / bn), math.ceil(I / bk))
        self.w13_bytes = 2 * I * H
        self.w2_bytes = H * I
        self.s13_elems = self.s13_shape[0] * self.s13_shape[1]
        self.s2_elems = self.s2_shape[0] * self.s2_shape[1]
        self.o_w2 = self.w13_bytes
        # scales start 16-byte aligned (no padding for H, I multiples of 16)
        self.o_s13 = -(-(self.w13_bytes + self.w2_bytes) // 16) * 16
        self.o_s2 = self.o_s13 + 4 * self.s13_elems
        self.used = self.o_s2 + 4 * self.s2_elems
        self.slab = -(-self.used // 256) * 256

    def views(self, buf: torch.Tensor):
        """``buf [N, slab] uint8`` -> ``(w13 [N, 2I, H], w2 [N, H, I]`` e4m3fn,
        ``s13, s2`` float32) views."""
        N, H, I, sl = buf.shape[0], self.hidden, self.inter, self.slab
        base = buf.storage_offset()
        w13 = torch.as_strided(buf, (N, 2 * I, H), (sl, H, 1), base).view(FP8)
        w2 = torch.as_strided(buf, (N, H, I), (sl, I, 1), base + self.o_w2).view(FP8)
        f = buf.view(torch.float32)
        fb = f.storage_offset()
        s13 = torch.as_strided(f, (N, *self.s13_shape), (sl // 4, self.s13_shape[1], 1),
                               fb + self.o_s13 // 4)
        s2 = torch.as_strided(f, (N, *self.s2_shape), (sl // 4, self.s2_shape[1], 1),
                              fb + self.o_s2 // 4)
        return w13, w2, s13, s2


def fp8_slab_masters(num_experts: int, hidden: int, inter: int, block: tuple[int, int],
                     pin: bool = True):
    """Host masters as one ``[w13 | w2 | s13 | s2]`` slab per expert:
    ``(buf, w13, w2, s13, s2)``; the scales start at 1.0 like vLLM's."""
    lay = Fp8SlabLayout(hidden, inter, block)
    buf = torch.zeros((num_experts, lay.slab), dtype=torch.uint8, pin_memory=pin)
    w13, w2, s13, s2 = lay.views(buf)
    s13.fill_(1.0)
    s2.fill_(1.0)
    return buf, w13, w2, s13, s2


def _check_fp8_master(t: torch.Tensor, name: str, dtype: torch.dtype) -> None:
    if t.device.type != "cpu":
        raise ValueError(f"{name} must live in host memory")
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}")
    if t.dim() != 3 or t.stride(2) != 1 or t.stride(1) != t.shape[2]:
        raise ValueError(f"{name} must be [E, rows, cols] with each expert contiguous")


class WispMoEStateFP8(WispMoEState):
    """Per-layer FP8 paging state (reference ``WispMoEStateFP8``,
    fused_moe_fp8.py:61-145): pages (weight, scale) pairs for w13 and w2.

    The pager, page-in and layer call are the unquantised state's (same
    C++ layer, same kernels for routing and paging); the expert stage runs
    the block-FP8 kernels.  Activations and outputs are bfloat16.
    """

    def __init__(self, cpu_w13: torch.Tensor, cpu_w2: torch.Tensor, cpu_s13: torch.Tensor,
                 cpu_s2: torch.Tensor, cap_experts: int, device, layer_idx: int,
                 block: tuple[int, int] | None = None) -> None:
        _check_fp8_master(cpu_w13, "cpu_w13", FP8)
        _check_fp8_master(cpu_w2, "cpu_w2", FP8)
        _check_fp8_master(cpu_s13, "cpu_s13", torch.float32)
        _check_fp8_master(cpu_s2, "cpu_s2", torch.float32)
        E, two_i, H = cpu_w13.shape
        I = cpu_w2.shape[2]
        if cpu_w2.shape[:2] != (E, H) or two_i != 2 * I:
            raise ValueError("cpu_w13 [E, 2I, H] and cpu_w2 [E, H, I] disagree")
        if block is None:  # the block shape follows from the scale shapes
            block = (-(-I // (cpu_s13.shape[1] // 2)), -(-H // cpu_s13.shape[2]))
        lay = Fp8SlabLayout(H, I, block)
        if tuple(cpu_s13.shape) != (E, *lay.s13_shape) or \
                tuple(cpu_s2.shape) != (E, *lay.s2_shape):
            raise ValueError(f"scale shapes {tuple(cpu_s13.shape)}, {tuple(cpu_s2.shape)} do "
                             f"not match block {block} for H={H}, I={I}")
        if cap_experts < 1:
            raise ValueError(f"cap_experts={cap_experts} < 1")
        self._layout = lay
        self.block_shape = list(lay.block)
        self.layer_idx = int(layer_idx)
        self.num_experts = int(E)
        # the reference's clamp max(8, min(cap, E)) can exceed E: the extra
        # slots exist (and take the first misses, as free slots are taken
        # from the top) exactly as in the reference
        self.cap_experts = int(cap_experts)
        self.mode = _Mode.PAGED
        self.hidden, self.inter = int(H), int(I)
        self.dtype = torch.bfloat16  # activations
        self.weight_dtype = FP8
        self.cpu_w13, self.cpu_w2, self.cpu_s13, self.cpu_s2 = cpu_w13, cpu_w2, cpu_s13, cpu_s2
        self.device = torch.device(device)
        self._w13_elems = two_i * H
        self._w2_elems = H * I
        self._alloc_scratch(self.cap_experts)
        dev = self.device
        self.expert_map_device = torch.full((E,), -1, dtype=torch.int32, device=dev)
        self._counters = torch.zeros(8, dtype=torch.int64, device=dev)
        self.stats_pred_hits = 0
        self._pf_record = None
        self._pf_words = 0
        self._pf_n = 0
        self._ws = _Workspace(dev, self.hidden, I, torch.bfloat16, fp8=True)
        self._last_pairs = 0
        self._handle = C.c_void_p()
        self._desc = self._make_desc()
        check(lib().wisp_layer_create(C.byref(self._desc), C.byref(self._handle)),
              "wisp_layer_create")
        self.quant_config = _make_quant_config(self)

    def _alloc_scratch(self, cap: int) -> None:
        lay = self._layout
        self._scratch = torch.empty((cap, lay.slab), dtype=torch.uint8, device=self.device)
        self.scratch_w13, self.scratch_w2, self.scratch_s13, self.scratch_s2 = \
            lay.views(self._scratch)
        self._slot_to_expert = torch.full((cap,), -1, dtype=torch.int32, device=self.device)
        self._lru_tick = torch.zeros(cap, dtype=torch.int64, device=self.device)

    def _make_desc(self) -> "_lib.LayerDesc":
        lay = self._layout
        d = _lib.LayerDesc()
        d.struct_bytes = C.sizeof(_lib.LayerDesc)
        d.num_experts, d.cap = self.num_experts, self.cap_experts
        d.hidden, d.inter = self.hidden, self.inter
        d.dtype = _lib.WISP_FP8_E4M3
        d.mode = _lib.WISP_MODE_PAGED
        d.pagein_streams = _resolve_pagein_streams()
        d.pagein_engine = _resolve_pagein_engine()
        d.w13_elems, d.w2_elems = self._w13_elems, self._w2_elems
        d.scratch_w13, d.scratch_w13_stride = self.scratch_w13.data_ptr(), lay.slab
        d.scratch_w2, d.scratch_w2_stride = self.scratch_w2.data_ptr(), lay.slab
        d.master_w13, d.master_w13_stride = self.cpu_w13.data_ptr(), self.cpu_w13.stride(0)
        d.master_w2, d.master_w2_stride = self.cpu_w2.data_ptr(), self.cpu_w2.stride(0)
        d.expert_map = self.expert_map_device.data_ptr()
        d.slot_to_expert = self._slot_to_expert.data_ptr()
        d.lru_tick = self._lru_tick.data_ptr()
        d.counters = self._counters.data_ptr()
        d.block_n, d.block_k = lay.block
        d.s13_elems, d.s2_elems = lay.s13_elems, lay.s2_elems
        d.scratch_s13, d.scratch_s13_stride = self.scratch_s13.data_ptr(), lay.slab // 4
        d.scratch_s2, d.scratch_s2_stride = self.scratch_s2.data_ptr(), lay.slab // 4
        d.master_s13, d.master_s13_stride = self.cpu_s13.data_ptr(), self.cpu_s13.stride(0)
        d.master_s2, d.master_s2_stride = self.cpu_s2.data_ptr(), self.cpu_s2.stride(0)
        return d

    def resize_cap(self, new_cap: int) -> None:
        raise NotImplementedError("wisp.fp8: the FP8 state has no live resize (the reference's "
                                  "WispMoEStateFP8 has none either)")


def _make_quant_config(st: WispMoEStateFP8) -> Any:
    """vLLM's FusedMoEQuantConfig over the scratch scales when vLLM is
    present (reference 244-249), else a plain record of the same fields."""
    try:
        from vllm.model_executor.layers.fused_moe.config import fp8_w8a8_moe_quant_config
    except ImportError:
        return SimpleNamespace(w1_scale=st.scratch_s13, w2_scale=st.scratch_s2, a1_scale=None,
                               a2_scale=None, block_shape=list(st.block_shape))
    return fp8_w8a8_moe_quant_config(w1_scale=st.scratch_s13, w2_scale=st.scratch_s2,
                                     a1_scale=None, a2_scale=None,
                                     block_shape=list(st.block_shape))


# ---------------------------------------------------------------------------
# Patched Fp8MoEMethod (reference 147-359)
# ---------------------------------------------------------------------------


def _set_attrs(p: torch.nn.Parameter, attrs: dict) -> None:
    try:
        from vllm.model_executor.utils import set_weight_attrs
        set_weight_attrs(p, attrs)
    except ImportError:
        for k, v in attrs.items():
            setattr(p, k, v)


def _patched_create_weights(self, layer, num_experts, hidden_size,
                            intermediate_size_per_partition, params_dtype, **extra_weight_attrs):
    """Allocate the FP8 masters as one pinned host slab per expert (reference
    150-203 allocates four CPU tensors); non-block-quant methods keep the
    original."""
    if not getattr(self, "block_quant", False):
        return type(self)._wisp_original_create_weights(
            self, layer, num_experts, hidden_size, intermediate_size_per_partition,
            params_dtype, **extra_weight_attrs)
    I = intermediate_size_per_partition
    block_n, block_k = self.weight_block_size[0], self.weight_block_size[1]
    if I % block_n != 0:
        raise ValueError(f"wisp.fp8: intermediate size {I} is not divisible by the weight "
                         f"quantisation block_n = {block_n}")
    layer.intermediate_size_per_partition = I
    layer.hidden_size = hidden_size
    layer.num_experts = num_experts
    layer.orig_dtype = params_dtype
    layer.weight_block_size = self.weight_block_size
    buf, w13, w2, s13, s2 = fp8_slab_masters(num_experts, hidden_size, I, (block_n, block_k),
                                             pin=True)
    params = {}
    for name, t in (("w13_weight", w13), ("w2_weight", w2), ("w13_weight_scale_inv", s13),
                    ("w2_weight_scale_inv", s2)):
        p = torch.nn.Parameter(t, requires_grad=False)
        layer.register_parameter(name, p)
        params[name] = p
    _set_attrs(params["w13_weight"], extra_weight_attrs)
    _set_attrs(params["w2_weight"], extra_weight_attrs)
    scale_attrs = dict(extra_weight_attrs)
    try:
        from vllm.model_executor.layers.fused_moe.layer import FusedMoeWeightScaleSupported
        scale_attrs["quant_method"] = FusedMoeWeightScaleSupported.BLOCK.value
    except ImportError:
        scale_attrs["quant_method"] = "block"
    _set_attrs(params["w13_weight_scale_inv"], scale_attrs)
    _set_attrs(params["w2_weight_scale_inv"], scale_attrs)
    layer._wisp_fp8_slab = buf
    layer.w13_input_scale = None
    layer.w2_input_scale = None
    self.rocm_aiter_moe_enabled = False


def _slab_masters_of(layer, block: tuple[int, int]):
    """The layer's four block-FP8 tensors as views of one pinned ``[E, slab]``
    host buffer, so that a miss moves an expert's weights and scales in one
    copy.  After the patched create_weights the buffer already exists (the
    layer's parameters are its views and the checkpoint loader filled them in
    place); otherwise one is made and the loaded tensors are copied into it
    from wherever they live."""
    buf = getattr(layer, "_wisp_fp8_slab", None)
    w13 = layer.w13_weight.data
    E, two_i, H = w13.shape
    if buf is not None:
        return Fp8SlabLayout(H, two_i // 2, block).views(buf)
    buf, *views = fp8_slab_masters(E, H, two_i // 2, block, pin=True)
    loaded = (w13, layer.w2_weight.data, layer.w13_weight_scale_inv.data,
              layer.w2_weight_scale_inv.data)
    for dst, src in zip(views, loaded):
        dst.copy_(src)
    layer._wisp_fp8_slab = buf
    return tuple(views)


def _patched_process_weights_after_loading(self, layer) -> None:
    """Create the layer's block-FP8 paging state (the hook of reference
    206-269): non-block FP8 keeps vLLM's own processing, a second call
    changes nothing, and the layer's device parameters become 0-element
    placeholders, since the expert kernels read the state's scratch."""
    if getattr(layer, "_wisp_fp8_state", None) is not None:
        return
    if not getattr(self, "block_quant", False):
        return type(self)._wisp_original_process_weights_after_loading(self, layer)
    block = tuple(int(b) for b in self.weight_block_size)
    masters = _slab_masters_of(layer, block)
    gpu = torch.device("cuda", torch.cuda.current_device())
    E = int(masters[0].shape[0])
    st = WispMoEStateFP8(*masters, _resolve_cap_experts(E), gpu, len(_FP8_LAYER_STATES),
                         block=block)
    _FP8_LAYER_STATES.append(st)
    layer._wisp_fp8_state = st
    for name, dtype in (("w13_weight", FP8), ("w2_weight", FP8),
                        ("w13_weight_scale_inv", torch.float32),
                        ("w2_weight_scale_inv", torch.float32)):
        getattr(layer, name).data = torch.empty(0, dtype=dtype, device=gpu)
    self.moe_quant_config = st.quant_config
    logger.info("wisp.fp8: layer %d init num_experts=%d cap=%d gpu_scratch=%.2f GiB engine=%s",
                st.layer_idx, E, st.cap_experts, st._scratch.numel() / 2 ** 30,
                st.pagein_engine)


# Arguments of vLLM's apply this path supports only at these values (the
# kernels implement softmax routing with SiLU experts).
_SUPPORTED_ONLY = {
    "use_grouped_topk": False, "topk_group": None, "num_expert_group": None,
    "custom_routing_function": None, "scoring_func": "softmax", "routed_scaling_factor": 1.0,
    "e_score_correction_bias": None, "apply_router_weight_on_input": False,
    "activation": "silu", "enable_eplb": False,
}


def _patched_apply(self, layer, x, router_logits, top_k, renormalize, use_grouped_topk=False,
                   topk_group=None, num_expert_group=None, global_num_experts=-1,
                   expert_map=None, custom_routing_function=None, scoring_func="softmax",
                   routed_scaling_factor=1.0, e_score_correction_bias=None,
                   apply_router_weight_on_input=False, activation="silu", enable_eplb=False,
                   expert_load_view=None, logical_to_physical_map=None,
                   logical_replica_count=None):
    """FP8 layer call (reference 272-359): route, page, block-FP8 experts."""
    st: WispMoEStateFP8 | None = getattr(layer, "_wisp_fp8_state", None)
    if st is None:
        return type(self)._wisp_original_apply(
            self, layer, x, router_logits, top_k, renormalize, use_grouped_topk=use_grouped_topk,
            topk_group=topk_group, num_expert_group=num_expert_group,
            global_num_experts=global_num_experts, expert_map=expert_map,
            custom_routing_function=custom_routing_function, scoring_func=scoring_func,
            routed_scaling_factor=routed_scaling_factor,
            e_score_correction_bias=e_score_correction_bias,
            apply_router_weight_on_input=apply_router_weight_on_input, activation=activation,
            enable_eplb=enable_eplb, expert_load_view=expert_load_view,
            logical_to_physical_map=logical_to_physical_map,
            logical_replica_count=logical_replica_count)
    if expert_map is not None:
        raise NotImplementedError("wisp.fp8: EP expert_map + paging not composed yet")
    got = dict(use_grouped_topk=use_grouped_topk, topk_group=topk_group,
               num_expert_group=num_expert_group, custom_routing_function=custom_routing_function,
               scoring_func=scoring_func, routed_scaling_factor=routed_scaling_factor,
               e_score_correction_bias=e_score_correction_bias,
               apply_router_weight_on_input=apply_router_weight_on_input, activation=activation,
               enable_eplb=enable_eplb)
    for name, want in _SUPPORTED_ONLY.items():
        v = got[name]
        if (v is not None) if want is None else (v != want):
            raise NotImplementedError(f"wisp.fp8: {name}={v!r} is not supported on the paged "
                                      "FP8 path")
    if global_num_experts not in (-1, st.num_experts):
        raise NotImplementedError("wisp.fp8: global_num_experts differs from the layer's")
    if getattr(layer, "zero_expert_num", 0):
        raise NotImplementedError("wisp.fp8: zero experts are not supported")
    return st.forward(x, router_logits, top_k, renormalize)


def route_and_experts_fp8(x, router_logits, top_k, renormalize, w13, w2, s13, s2,
                          block) -> torch.Tensor:
    """All FP8 experts resident in device tensors ``w13 [E, 2I, H]``,
    ``w2 [E, H, I]`` (e4m3fn) with scales ``s13`` / ``s2`` (float32): route,
    then the block-FP8 expert kernels with slot = expert id."""
    T, H = x.shape
    E = w13.shape[0]
    I = w2.shape[2]
    dev = x.device
    for t, name in ((router_logits, "router_logits"), (w13, "w13"), (w2, "w2"), (s13, "s13"),
                    (s2, "s2")):
        _require_device(t, dev, name)
    st = _lib.stream_handle()
    if x.dtype != torch.bfloat16:
        raise NotImplementedError("wisp.fp8: activations must be bfloat16")
    x = x.contiguous()
    logits = router_logits if router_logits.dtype in (torch.float32, torch.bfloat16) \
        else router_logits.float()
    logits = logits.contiguous()
    ldt = _lib.WISP_F32 if logits.dtype == torch.float32 else _lib.WISP_BF16
    topk_w = torch.empty((T, top_k), dtype=torch.float32, device=dev)
    topk_ids = torch.empty((T, top_k), dtype=torch.int32, device=dev)
    check(lib().wisp_route_topk_softmax(logits.data_ptr(), ldt, T, E, top_k,
                                        int(bool(renormalize)), topk_w.data_ptr(),
                                        topk_ids.data_ptr(), None, st), "route")
    act = torch.empty((max(1, T * top_k), I), dtype=torch.bfloat16, device=dev)
    out = torch.empty_like(x)
    nbytes = lib().wisp_moe_fp8_work_bytes(max(1, T), top_k, H, I, E)
    work = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    check(lib().wisp_moe_experts_fp8(
        x.data_ptr(), T, H, I, top_k, topk_w.data_ptr(), topk_ids.data_ptr(), E,
        w13.data_ptr(), w13.stride(0), s13.data_ptr(), s13.stride(0), w2.data_ptr(),
        w2.stride(0), s2.data_ptr(), s2.stride(0), int(block[0]), int(block[1]),
        act.data_ptr(), out.data_ptr(), work.data_ptr(), nbytes, _lib.WISP_ALGO_AUTO, st),
        "experts_fp8")
    return out


def _method_class():
    """vLLM's ``Fp8MoEMethod`` if importable, else the local stand-in."""
    try:
        from vllm.model_executor.layers.quantization.fp8 import Fp8MoEMethod  # noqa
    except ImportError:
        from .layer import Fp8MoEMethod
    return Fp8MoEMethod


def install_wisp_fp8() -> bool:
    """Patch ``Fp8MoEMethod`` (block-quant path) for working-set paging.
    Idempotent; True iff this call patched."""
    lib()  # fail loudly now if the HIP library is missing
    cls = _method_class()
    if getattr(cls, _PATCHED_FLAG, False):
        return False
    cls._wisp_original_create_weights = cls.create_weights
    cls._wisp_original_process_weights_after_loading = cls.process_weights_after_loading
    cls._wisp_original_apply = cls.apply
    cls.create_weights = _patched_create_weights
    cls.process_weights_after_loading = _patched_process_weights_after_loading
    cls.apply = _patched_apply
    setattr(cls, _PATCHED_FLAG, True)
    logger.info("wisp.fp8: patched %s.%s (block-quant working-set paging)", cls.__module__,
                cls.__name__)
    return True


def is_fp8_installed() -> bool:
    return bool(getattr(_method_class(), _PATCHED_FLAG, False))


__all__ = ["install_wisp_fp8", "is_fp8_installed", "WispMoEStateFP8", "fp8_slab_masters",
           "Fp8SlabLayout", "route_and_experts_fp8"]
