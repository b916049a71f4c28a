"""ctypes binding of ``libwisp_hip.so`` (the C ABI in ``include/wisp_hip.h``).

The library is built in-tree by ``wisp_amd.build``.  There is no fallback:
if the shared library is missing, ``lib()`` raises.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libwisp_hip.so"

WISP_OK = 0
WISP_ERR_INVALID = 1
WISP_ERR_SUBBATCH = 2
WISP_ERR_HIP = 3
WISP_ERR_UNSUPPORTED = 4

WISP_F32 = 0
WISP_BF16 = 1
WISP_FP8_E4M3 = 2

WISP_MODE_PAGED = 0
WISP_MODE_RESIDENT = 1

WISP_ALGO_AUTO = 0
WISP_ALGO_GEMV = 1
WISP_ALGO_MFMA = 2
WISP_PAGEIN_MEMCPY = 0
WISP_PAGEIN_KERNEL = 1
WISP_NOALLOC_SCRATCH_BYTES = 64 << 20  # a default build's; the library's: noalloc_scratch_bytes()

# Decision-record header words (wisp_amd/csrc/pager_core.h).
REC_STATUS, REC_GROUPS_DONE, REC_GROUPS_PLANNED, REC_FAIL_GROUP, REC_FAIL_UNIQUE, \
    REC_EVICTED, REC_LOADED = range(7)

_vp, _i32, _i64, _sz, _f32p = C.c_void_p, C.c_int, C.c_int64, C.c_size_t, C.POINTER(C.c_float)


class LayerDesc(C.Structure):
    _fields_ = [
        ("num_experts", C.c_int), ("cap", C.c_int), ("hidden", C.c_int), ("inter", C.c_int),
        ("dtype", C.c_int), ("mode", C.c_int), ("pagein_streams", C.c_int),
        ("pagein_engine", C.c_int),
        ("w13_elems", _sz), ("w2_elems", _sz),
        ("scratch_w13", _vp), ("scratch_w13_stride", _sz),
        ("scratch_w2", _vp), ("scratch_w2_stride", _sz),
        ("master_w13", _vp), ("master_w13_stride", _sz),
        ("master_w2", _vp), ("master_w2_stride", _sz),
        ("expert_map", _vp), ("slot_to_expert", _vp), ("lru_tick", _vp), ("counters", _vp),
        ("block_n", C.c_int), ("block_k", C.c_int), ("s13_elems", _sz), ("s2_elems", _sz),
        ("scratch_s13", _vp), ("scratch_s13_stride", _sz),
        ("scratch_s2", _vp), ("scratch_s2_stride", _sz),
        ("master_s13", _vp), ("master_s13_stride", _sz),
        ("master_s2", _vp), ("master_s2_stride", _sz),
        ("packed_master", _vp), ("packed_stride", _sz),
        ("struct_bytes", _sz),
    ]


class Cooccur(C.Structure):
    _fields_ = [
        ("layers", C.c_int), ("experts", C.c_int), ("count", _vp), ("total", _vp),
        ("obs_keys", _vp), ("obs_n", _vp), ("obs_seq", _vp), ("meta", _vp),
    ]


class Workspace(C.Structure):
    _fields_ = [
        ("max_pairs", C.c_int), ("topk_w", _vp), ("topk_ids", _vp), ("slots", _vp),
        ("flags", _vp), ("loads", _vp), ("act", _vp), ("record", _vp),
        ("record_words", C.c_int), ("record_dev", _vp), ("work", _vp), ("work_bytes", _sz),
        ("struct_bytes", _sz),
    ]


# name -> (restype, argtypes); every function declared in include/wisp_hip.h.
SIGNATURES = {
    "wisp_last_error": (C.c_char_p, []),
    "wisp_abi_version": (_i32, []),
    "wisp_pack_bf16_stride": (_sz, [_i32, _i32, _i32, _vp, _sz, _vp, _sz]),
    "wisp_pack_bf16": (_i32, [_i32, _i32, _i32, _vp, _sz, _vp, _sz, _vp, _sz]),
    "wisp_record_words": (_i32, [_i32, _i32]),
    "wisp_route_topk_softmax": (_i32, [_vp, _i32, _i32, _i32, _i32, _i32, _vp, _vp, _vp, _vp]),
    "wisp_pager_decide": (_i32, [_vp, _i32, _i32, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _vp,
                                 _vp, _i32, _vp]),
    "wisp_pager_decide_host": (_i32, [_vp, _i32, _i32, _i32, _i32, _i32, _vp, _vp, _vp, _vp,
                                      _vp, _vp, _i32]),
    "wisp_cpython_set_order": (_i32, [_vp, _i32, _vp]),
    "wisp_subbatch_plan": (_i32, [_vp, _i32, _i32, _i32, _vp]),
    "wisp_pagein_issue": (_i32, [_vp, _i32, _i32, _i32, _i32, _vp, _sz, _vp, _sz, _vp, _sz, _vp,
                                 _sz, _sz, _sz, _i32, _vp]),
    "wisp_moe_experts": (_i32, [_vp, _i32, _i32, _i32, _i32, _i32, _vp, _vp, _i32, _vp, _sz,
                                _vp, _sz, _vp, _vp, _vp, _sz, _i32, _vp]),
    "wisp_moe_work_bytes": (_sz, [_i32, _i32, _i32, _i32]),
    "wisp_noalloc_scratch_bytes": (_sz, []),
    "wisp_moe_experts_noalloc": (_i32, [_vp, _i32, _i32, _i32, _i32, _i32, _vp, _vp, _i32, _vp,
                                        _sz, _vp, _sz, _vp, _i32, _vp]),
    "wisp_moe_experts_fp8": (_i32, [_vp, _i32, _i32, _i32, _i32, _vp, _vp, _i32, _vp, _sz, _vp,
                                    _sz, _vp, _sz, _vp, _sz, _i32, _i32, _vp, _vp, _vp, _sz, _i32,
                                    _vp]),
    "wisp_quant_fp8_groups": (_i32, [_vp, _i32, _i32, _i32, _i32, _vp, _vp, _vp]),
    "wisp_moe_fp8_work_bytes": (_sz, [_i32, _i32, _i32, _i32, _i32]),
    "wisp_layer_create": (_i32, [C.POINTER(LayerDesc), C.POINTER(_vp)]),
    "wisp_layer_destroy": (_i32, [_vp]),
    "wisp_layer_set_scratch": (_i32, [_vp, _vp, _vp, _i32, _vp, _vp]),
    "wisp_layer_forward": (_i32, [_vp, _vp, _vp, _i32, _i32, _i32, _i32, _vp,
                                  C.POINTER(Workspace), _i32, _vp]),
    "wisp_layer_ensure_resident": (_i32, [_vp, _vp, _i32, C.POINTER(Workspace), _vp]),
    "wisp_layer_prime_identity": (_i32, [_vp, _vp]),
    "wisp_layer_last_pagein": (_i32, [_vp, _f32p, C.POINTER(C.c_double)]),
    "wisp_layer_pagein_engine": (_i32, [_vp]),
    "wisp_layer_set_decode_fused": (_i32, [_vp, _i32]),
    "wisp_layer_sync_record": (_i32, [_vp, C.POINTER(Workspace)]),
    "wisp_layer_profile": (_i32, [_vp, _i32, C.POINTER(C.c_double), C.POINTER(C.c_double),
                                  C.POINTER(C.c_int64), C.POINTER(C.c_int64)]),
    "wisp_layer_profile_noload": (_i32, [_vp, C.POINTER(C.c_double), C.POINTER(C.c_int64)]),
    "wisp_cooccur_observe_layer": (_i32, [C.POINTER(Cooccur), _i32, _vp, _i32, _i32, _vp]),
    "wisp_cooccur_predict": (_i32, [C.POINTER(Cooccur), _i32, _i32, _vp, _i32, _i32, _vp, _vp,
                                    _vp]),
    "wisp_cooccur_end_step": (_i32, [C.POINTER(Cooccur), _i32, _vp]),
    "wisp_prefetch_record_words": (_i32, [_i32]),
    "wisp_layer_prefetch": (_i32, [_vp, _vp, _vp, _i32, _i32, _i32, _vp, _i32, _vp, _i32, _vp]),
    "wisp_probe_h2d": (_i32, [_vp, _vp, _sz, _i32, _i32, _f32p]),
    "wisp_probe_hbm_copy": (_i32, [_vp, _vp, _sz, _vp]),
}

_LIB: C.CDLL | None = None


def lib() -> C.CDLL:
    """Load the in-tree library (once).  Raises if it was not built."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"wisp_amd: {LIB_PATH} is missing - build it with `python -m wisp_amd.build` "
                "(there is no non-HIP fallback)")
        h = C.CDLL(os.fspath(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(h, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = h
    return _LIB


class SubBatchError(RuntimeError):
    """Working set of one call exceeds the scratch (reference: the
    "sub-batch" RuntimeError of fused_moe.py:315-327)."""


def last_error() -> str:
    return lib().wisp_last_error().decode(errors="replace")


def check(rc: int, what: str) -> None:
    if rc == WISP_OK:
        return
    msg = last_error()
    if rc == WISP_ERR_SUBBATCH:
        raise SubBatchError(
            f"wisp: per-kernel-call working set exceeds cap_experts; the forward path "
            f"must sub-batch ({what}: {msg})")
    if rc == WISP_ERR_UNSUPPORTED:
        raise NotImplementedError(f"{what}: {msg}")
    if rc == WISP_ERR_INVALID:
        raise ValueError(f"{what}: invalid argument ({msg})")
    raise RuntimeError(f"{what}: HIP error ({msg})")


def ptr(t) -> int | None:
    """Raw address of a tensor (None for None)."""
    return None if t is None else t.data_ptr()


def stream_handle(stream=None) -> int:
    import torch
    s = torch.cuda.current_stream() if stream is None else stream
    return s.cuda_stream
