#!/usr/bin/env python3
"""Paged MoE decode benchmark on one MI355X.

Workload (default): the Qwen3-30B-A3B-shaped MoE layer at batch 1 with a
cap=8 HBM scratch and all 128 expert masters in pinned host memory (hidden
2048, expert intermediate 768, top-8 softmax with renormalisation, bf16
random-init weights).  Router logits carry a Zipf(1.1) per-expert bias and a
0.6 probability of re-using the previous step's expert set.

A step is one bs=1 token through the layer: routing, the GPU pager, page-in
of the missed experts over the host link, the expert GEMMs and the combine.
Eight independent instances of the layer (own scratch, own pager, own
256-step routing sequence; shared host masters) are driven round-robin, so
consecutive steps read different 72 MiB scratches and the expert kernels
stream from HBM rather than from the 256 MB last-level cache.

Printed: one JSON line with tok/s (layer calls per second), the live
HIP-event roofline of the dominant expert kernel, page-in bandwidth against
the measured host link, and the CPU baseline (oracle pager + torch CPU
fused-MoE on a time-bounded sample, timed on this host's cores).  tok/s is
timed with the library's kernel timing off, as it ships; the kernel and
page-in durations come from a second pass of the same steps with
dispatch-timestamp events on those launches (each timed launch lengthens the
stream by a few microseconds).

``--workload`` selects other layer configurations for measurement runs (the
default line above is the one the benchmark is quoted on):
  prefill   one 512-token prefill chunk, Qwen3 layer, cap=32 paged and resident
  batch32   bs=32 decode, Qwen3 layer, cap=32 paged and resident
  mixtral   Mixtral-8x7B layer, cap=4, bs=1 and bs=16 decode
  stack     48 Qwen3 layers, cap=24 each, bs=1 decode through the stack
  fp8       the default decode line on the Qwen3-30B-A3B-FP8 layer (e4m3fn
            weights with [128, 128] float32 block scales, w8a8)
  fp8-prefill, fp8-batch32   the prefill and batch32 lines on that FP8 layer
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

HBM_PEAK_GBPS = 8000.0          # MI355X HBM3E, GB/s
BF16_PEAK_TFLOPS = 2500.0       # dense bf16 MFMA
FP8_PEAK_TFLOPS = 5000.0        # dense fp8 MFMA
METRIC = "MoE decode tok/s, Qwen3-30B-A3B shape bs=1 cap=8; expert GEMM % HBM peak"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_name() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(routes, w13, w2, seconds: float, warm: int = 8) -> dict:
    """Oracle routing + LRU pager + torch CPU SwiGLU experts over the decode
    routing sequences (one pager per sequence, round-robin, as on the GPU):
    ``warm`` untimed steps, then steps timed one by one with
    ``time.perf_counter`` until ``seconds`` of timed work; throughput = 1 /
    the median step time."""
    import torch

    from oracle.moe import moe_forward_fast, route
    from oracle.pager import PagerOracle
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    K = routes[0].shape.top_k
    pagers = [PagerOracle(wl.shape.experts, wl.shape.cap) for wl in routes]
    R, per = len(routes), routes[0].steps
    n = 0
    spent = 0.0
    times = []
    while spent < seconds and n < 64 * R * per:
        r, pos = n % R, (n // R) % per
        t0 = time.perf_counter()
        w, ids = route(routes[r].logits[pos], K)
        pagers[r].forward(ids.tolist())
        moe_forward_fast(routes[r].x[pos], w, ids, w13, w2)
        dt = time.perf_counter() - t0
        if n >= warm:
            spent += dt
            times.append(dt)
        n += 1
    med = statistics.median(times)
    return {"value": round(1.0 / med, 2), "unit": "tok/s", "cores": cores, "kind": "port",
            "sample": f"median of {len(times)} bs=1 decode steps of the qwen3 layer "
                      f"({med * 1e3:.3f} ms; mean {spent / len(times) * 1e3:.3f} ms) after {warm} "
                      f"warm-up steps, round-robin over {R} routing sequences with one pager "
                      f"each, time-bounded to {seconds:.0f} s (oracle routing + LRU pager + torch "
                      f"CPU SwiGLU experts on bf16 weights in host memory, so no page-in); "
                      f"{cpu_name()}"}


def pmc_traffic(path: str, kernel: str):
    """HBM bytes per launch of ``kernel`` from a committed profiler summary
    (FETCH_SIZE + WRITE_SIZE per dispatch, calibrated against a copy kernel
    of known size), or None."""
    try:
        with open(path) as f:
            d = json.load(f)
        k = d["kernels"][kernel]
        return int(round(k["fetch_bytes"] + k["write_bytes"]))
    except (OSError, KeyError, ValueError, TypeError):
        return None


def timing_off(path: str, kernel: str, nbytes: int):
    """The same kernel's duration in the bench's first pass (the library's
    timing off, no dispatch events) from a committed kernel-trace summary,
    as a roofline entry beside the event-timed one, or None."""
    try:
        with open(path) as f:
            t = json.load(f)["timing_off"][kernel]
        us = float(t["avg_us"])
        gbps = nbytes / (us * 1e-6) / 1e9
        return {"avg_us_per_call": us, "achieved": round(gbps, 1),
                "frac": round(gbps / HBM_PEAK_GBPS, 4), "launches": t["launches"],
                "source": os.path.basename(path)}
    except (OSError, KeyError, ValueError, TypeError):
        return None


def h2d_link(nbytes: int, iters: int = 20, streams: int = 1) -> float:
    """p50 pinned-host -> HBM hipMemcpyAsync bandwidth in GB/s."""
    import ctypes as C

    import torch

    from wisp_amd import _lib
    src = torch.empty(nbytes, dtype=torch.uint8, pin_memory=True)
    dst = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    ms = (C.c_float * iters)()
    _lib.check(_lib.lib().wisp_probe_h2d(dst.data_ptr(), src.data_ptr(), nbytes, iters, streams,
                                         ms), "probe_h2d")
    return nbytes / (statistics.median(list(ms)[2:]) * 1e-3) / 1e9


# ---------------------------------------------------------------------------
# Measurement runs of the other layer configurations (--workload).
# ---------------------------------------------------------------------------

def _collect(states) -> dict:
    """Kernel time (ms), calls and page-in ms/bytes summed over the states
    since timing was switched on; switches it off."""
    agg = {"w13_ms": 0.0, "w2_ms": 0.0, "calls": 0, "w13_calls": 0, "pin_ms": 0.0,
           "pin_bytes": 0.0, "w2_noload_ms": 0.0, "w2_noload_calls": 0}
    for st in states:
        p = st.profile(False)
        agg["w13_ms"] += p["w13"]
        agg["w2_ms"] += p["w2"]
        agg["calls"] += p["calls"]
        agg["w13_calls"] += p["w13_calls"]
        agg["w2_noload_ms"] += p["w2_noload"]
        agg["w2_noload_calls"] += p["w2_noload_calls"]
        ms, nb = st.pagein_stats()
        agg["pin_ms"] += ms
        agg["pin_bytes"] += nb
    return agg


def _timed(fn, n_warm: int, n: int, states, n_events: int | None = None) -> tuple[float, dict]:
    """Wall time of calls fn(n_warm) .. fn(n_warm + n - 1) after n_warm
    untimed ones, run as the library runs by default (timing off), with the
    pager's misses and hits over them; then the first ``n_events`` (default
    n) of the same calls again with dispatch-timestamp events on the expert
    kernels and the page-in, whose durations and bytes it collects."""
    import torch
    for i in range(n_warm):
        fn(i)
    torch.cuda.synchronize()
    m0, h0 = sum(st.stats_miss for st in states), sum(st.stats_hits for st in states)
    t0 = time.perf_counter()
    for i in range(n_warm, n_warm + n):
        fn(i)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    miss = sum(st.stats_miss for st in states) - m0
    hits = sum(st.stats_hits for st in states) - h0
    for st in states:
        st.profile(True)
        st.pagein_stats()
    for i in range(n_warm, n_warm + (n if n_events is None else n_events)):
        fn(i)
    torch.cuda.synchronize()
    agg = _collect(states)
    agg["miss"], agg["hits"] = miss, hits
    return elapsed, agg


def _gemm_report(agg: dict, shape, tokens_per_call: int, distinct_per_call: float,
                 kernels: str) -> dict:
    calls = max(1, agg["calls"])
    t13 = agg["w13_ms"] / max(1, agg["w13_calls"]) * 1e-3
    t = t13 + agg["w2_ms"] / calls * 1e-3
    flops = 2.0 * tokens_per_call * shape.top_k * 3 * shape.hidden * shape.inter
    byts = distinct_per_call * shape.expert_bytes
    return {"kernels": kernels, "avg_us_per_call": round(t * 1e6, 2),
            "w13_us": round(t13 * 1e6, 2),
            "w2_us": round(agg["w2_ms"] / calls * 1e3, 2),
            "achieved_TFLOPs": round(flops / t / 1e12, 2) if t else None,
            "frac_bf16_mfma_peak": round(flops / t / 1e12 / BF16_PEAK_TFLOPS, 4) if t else None,
            "achieved_GBps": round(byts / t / 1e9, 1) if t else None,
            "frac_hbm_peak": round(byts / t / 1e9 / HBM_PEAK_GBPS, 4) if t else None,
            "bytes_per_call": int(byts), "flops_per_call": int(flops)}


def _pagein_report(agg: dict) -> dict:
    gbps = agg["pin_bytes"] / (agg["pin_ms"] * 1e-3) / 1e9 if agg["pin_ms"] else 0.0
    return {"bytes": agg["pin_bytes"], "achieved_GBps": round(gbps, 2), "misses": agg["miss"],
            "hits": agg["hits"],
            "timing": "bytes and GB/s from the event pass, misses and hits from the timed pass"}


def _distinct(logits, K: int) -> int:
    """Distinct experts routed to by the tokens of one call (``logits [T, E]``):
    the expert weights one call of the grouped GEMM streams."""
    import torch
    return int(torch.unique(torch.topk(logits.float(), K, dim=-1).indices).numel())


def _line(metric, value, unit, args, steps, elapsed, config, **extra) -> dict:
    line = {"metric": metric, "value": round(value, 2), "unit": unit, "n_gpus": 1,
            "steps": steps, "warmup": args.warmup,
            "ms_per_step": round(elapsed / max(1, steps) * 1e3, 4), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
            "config": config}
    line.update(extra)
    return line


def _cpu_layer(wl, cap: int, calls: int) -> dict:
    """Oracle routing + pager (with greedy sub-batching) + torch CPU experts
    over ``calls`` layer calls of the workload."""
    import torch

    from oracle.moe import moe_forward_fast, route
    from oracle.pager import PagerOracle
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    w13, w2 = wl.views()
    K = wl.shape.top_k
    pager = PagerOracle(wl.shape.experts, cap)
    t0 = time.perf_counter()
    for c in range(calls):
        w, ids = route(wl.logits[c % wl.steps], K)
        pager.forward(ids.tolist())
        moe_forward_fast(wl.x[c % wl.steps], w, ids, w13, w2)
    dt = time.perf_counter() - t0
    return {"value": round(calls * wl.tokens / dt, 2), "unit": "tok/s", "cores": cores,
            "kind": "port", "sample": f"{calls} layer calls of {wl.tokens} tokens (oracle routing "
            f"+ LRU pager with sub-batching + torch CPU SwiGLU experts, weights in host memory); "
            f"{cpu_name()}"}


def _state_run(wl, cap: int, mode: str, n_warm: int, n: int):
    """Times ``n`` layer calls (call i uses step i % steps, after ``n_warm``
    untimed calls) of ``wl`` on a fresh state: paged with ``cap`` slots, or
    resident with every expert primed."""
    import torch

    from wisp.integrations.vllm.fused_moe import WispMoEState
    dev = torch.device("cuda", 0)
    w13, w2 = wl.views()
    K = wl.shape.top_k
    xs, lgs = wl.x.to(dev), wl.logits.to(dev)
    out = torch.empty_like(xs[0])
    st = WispMoEState(w13, w2, wl.shape.experts if mode == "resident" else cap, mode, dev, 0)
    if mode == "resident":
        st.prime_identity()
    r = _timed(lambda i: st.forward(xs[i % wl.steps], lgs[i % wl.steps], K, True, out=out),
               n_warm, n, [st])
    del st
    torch.cuda.empty_cache()
    return r


def bench_prefill(args) -> dict:
    from wisp_amd import workloads as W
    wl = W.gaussian_logits("batch", seed=0, steps=3, tokens=512, pin=True)
    sh = wl.shape
    pe, pa = _state_run(wl, sh.cap, "paged", 1, 2)
    re_, ra = _state_run(wl, sh.cap, "resident", 2, 20)
    dist = sum(_distinct(wl.logits[i], 8) for i in range(wl.steps)) / wl.steps
    cpu = None if args.no_cpu_baseline else _cpu_layer(wl, sh.cap, 1)
    return _line("MoE prefill tok/s, Qwen3-30B-A3B shape, 512-token chunk, cap=32 paged",
                 2 * 512 / pe, "tok/s", args, 2, pe,
                 {"workload": "qwen3 moe layer, 512-token prefill chunk, router logits N(0,1)",
                  "hidden": sh.hidden, "expert_intermediate": sh.inter, "experts": sh.experts,
                  "top_k": sh.top_k, "cap": sh.cap, "tokens": 512},
                 pagein=_pagein_report(pa),
                 resident={"tok_per_s": round(20 * 512 / re_, 1),
                           "expert_gemm": _gemm_report(ra, sh, 512, dist,
                                                       "mfma_w13_dma_kernel + mfma_w2_dma_kernel")},
                 cpu_baseline=cpu)


def bench_batch32(args) -> dict:
    from wisp_amd import workloads as W
    wl = W.batch_decode(steps=24, tokens=32, pin=True)
    sh = wl.shape
    pe, pa = _state_run(wl, sh.cap, "paged", 2, 16)
    re_, ra = _state_run(wl, sh.cap, "resident", 2, 128)
    cpu = None if args.no_cpu_baseline else _cpu_layer(wl, sh.cap, 4)
    dist = sum(_distinct(wl.logits[i], 8) for i in range(wl.steps)) / wl.steps
    return _line("MoE batched decode tok/s, Qwen3-30B-A3B shape, bs=32, cap=32 paged",
                 16 * 32 / pe, "tok/s", args, 16, pe,
                 {"workload": "qwen3 moe layer, bs=32 decode, router logits N(0,1)",
                  "hidden": sh.hidden, "expert_intermediate": sh.inter, "experts": sh.experts,
                  "top_k": sh.top_k, "cap": sh.cap, "batch": 32},
                 pagein=_pagein_report(pa),
                 resident={"tok_per_s": round(128 * 32 / re_, 1),
                           "expert_gemm": _gemm_report(ra, sh, 32, dist,
                                                       "mfma_w13_dma_kernel + mfma_w2_dma_kernel")},
                 cpu_baseline=cpu)


def bench_mixtral(args) -> dict:
    from wisp_amd import workloads as W
    wl = W.mixtral(steps=40, tokens=1, pin=True)
    sh = wl.shape
    pe, pa = _state_run(wl, sh.cap, "paged", 4, 32)
    re_, ra = _state_run(wl, sh.cap, "resident", 4, 32)
    wl16 = W.mixtral(steps=10, tokens=16, pin=False, weights=False)
    wl16.slabs = wl.slabs
    pe16, pa16 = _state_run(wl16, sh.cap, "paged", 2, 8)
    re16, ra16 = _state_run(wl16, sh.cap, "resident", 2, 8)
    cpu = None if args.no_cpu_baseline else _cpu_layer(wl, sh.cap, 8)
    return _line("MoE decode tok/s, Mixtral-8x7B shape bs=1 cap=4 paged", 32 / pe, "tok/s",
                 args, 32, pe,
                 {"workload": "mixtral-8x7b moe layer decode, router N(0,1) + bias N(0,0.5)",
                  "hidden": sh.hidden, "expert_intermediate": sh.inter, "experts": sh.experts,
                  "top_k": sh.top_k, "cap": sh.cap, "batch": 1},
                 pagein=_pagein_report(pa),
                 resident={"tok_per_s": round(32 / re_, 1),
                           "expert_gemm": _gemm_report(ra, sh, 1, 2.0,
                                                       "w13_silu_kernel + w2_combine_kernel")},
                 bs16={"paged_tok_per_s": round(8 * 16 / pe16, 2), "pagein": _pagein_report(pa16),
                       "resident_tok_per_s": round(8 * 16 / re16, 1),
                       "resident_expert_gemm": _gemm_report(
                           ra16, sh, 16, sum(_distinct(wl16.logits[i], 2) for i in range(10)) / 10,
                           "mfma_w13_dma_kernel + mfma_w2_dma_kernel")},
                 cpu_baseline=cpu)


def bench_stack(args) -> dict:
    """48 MoE layers (own scratch of 24 slots and own pager each, one shared
    set of pinned masters): each token runs through the 48 layers in order,
    the output of layer L being the input of layer L+1."""
    import torch

    from wisp_amd import workloads as W
    from wisp.integrations.vllm.fused_moe import WispMoEState
    sh = W.SHAPES["stack"]
    layers, tokens = 48, 512
    t_setup = time.perf_counter()
    base = W.qwen3_decode(steps=1, pin=True)
    w13, w2 = base.views()
    dev = torch.device("cuda", 0)
    lg = torch.from_numpy(W.stack_routing(seed=0, layers=layers, tokens=tokens)).to(dev)
    x0 = torch.randn((tokens, 1, sh.hidden), generator=torch.Generator().manual_seed(1)) \
        .to(sh.dtype).to(dev)
    states = [WispMoEState(w13, w2, sh.cap, "paged", dev, L) for L in range(layers)]
    log(f"stack setup {time.perf_counter() - t_setup:.1f}s")
    n_warm = 8
    after = None
    if args.prefetch:
        from wisp.integrations.vllm import fused_moe as fm
        os.environ["WISP_PREFETCH"] = "1"
        os.environ["WISP_COOCCUR_ONLINE"] = "1"
        os.environ.pop("WISP_COOCCUR_PATH", None)
        fm._reset_cooccur()
        fm._LAYER_STATES = states
        after = fm._prefetch_after_forward

    def token(i: int) -> None:
        h = x0[i]
        for L in range(layers):
            h = states[L].forward(h, lg[L, i:i + 1], sh.top_k, True)
            if after is not None:
                after(states[L])

    # the event pass covers the first 64 tokens (the whole stack runs ~30 s)
    elapsed, agg = _timed(token, n_warm, tokens - n_warm, states, min(64, tokens - n_warm))
    n = tokens - n_warm
    calls = max(1, agg["calls"])
    return _line("MoE-only 48-layer stack decode tok/s, Qwen3-30B-A3B shape bs=1 cap=24",
                 n / elapsed, "tok/s", args, n, elapsed,
                 {"workload": "48 qwen3 moe layers, bs=1 decode, Dirichlet(0.3) layer-conditioned "
                              "routing, one shared set of pinned masters",
                  "hidden": sh.hidden, "expert_intermediate": sh.inter, "experts": sh.experts,
                  "top_k": sh.top_k, "cap": sh.cap, "layers": layers, "tokens": n},
                 layer_calls_per_s=round(n * layers / elapsed, 1),
                 prefetch={"enabled": bool(args.prefetch),
                           "predicted": sum(st.stats_pred_total for st in states),
                           "evicted": sum(st.stats_evict for st in states)},
                 pagein=_pagein_report(agg),
                 expert_gemm_us_per_layer_call=round(
                     (agg["w13_ms"] / max(1, agg["w13_calls"]) + agg["w2_ms"] / calls) * 1e3, 2))


def _calibration_copy(dev) -> None:
    """A plain 256 MiB device copy: the calibration dispatch for the
    profiler's HBM byte counters (FETCH_SIZE / WRITE_SIZE of a copy of known
    size)."""
    import torch

    from wisp_amd import _lib
    cal = torch.empty(2, 256 << 20, dtype=torch.uint8, device=dev)
    _lib.check(_lib.lib().wisp_probe_hbm_copy(cal[1].data_ptr(), cal[0].data_ptr(), 256 << 20,
                                              _lib.stream_handle()), "hbm copy")
    torch.cuda.synchronize()
    del cal


def cpu_baseline_fp8(routes, views, seconds: float, warm: int = 8) -> dict:
    """Oracle routing + LRU pager + a torch CPU block-FP8 fused-MoE
    (``oracle.fp8.moe_forward_fp8_fast``: weight blocks dequantised per call,
    activations quantised per 128-group, float32 GEMMs) over the decode
    routing sequences, as ``cpu_baseline`` does for the bf16 layer:
    ``warm`` untimed steps, then steps timed one by one until ``seconds`` of
    timed work; throughput = 1 / the median step time."""
    import numpy as np
    import torch

    from oracle.fp8 import moe_forward_fp8_fast
    from oracle.moe import route
    from oracle.pager import PagerOracle
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    w13, w2, s13, s2 = views
    K = routes[0].shape.top_k
    pagers = [PagerOracle(wl.shape.experts, wl.shape.cap) for wl in routes]
    R, per = len(routes), routes[0].steps
    n = 0
    spent = 0.0
    times = []
    while spent < seconds and n < 64 * R * per:
        r, pos = n % R, (n // R) % per
        t0 = time.perf_counter()
        w, ids = route(routes[r].logits[pos], K)
        pagers[r].forward(ids.tolist())
        moe_forward_fp8_fast(routes[r].x[pos], w.astype(np.float32), ids, w13, w2, s13, s2)
        dt = time.perf_counter() - t0
        if n >= warm:
            spent += dt
            times.append(dt)
        n += 1
    med = statistics.median(times)
    return {"value": round(1.0 / med, 2), "unit": "tok/s", "cores": cores, "kind": "port",
            "sample": f"median of {len(times)} bs=1 decode steps of the qwen3-fp8 layer "
                      f"({med * 1e3:.3f} ms; mean {spent / len(times) * 1e3:.3f} ms) after "
                      f"{warm} warm-up steps, round-robin over {R} routing sequences with one "
                      f"pager each, time-bounded to {seconds:.0f} s (oracle routing + LRU pager "
                      f"+ torch CPU block-FP8 experts: weight blocks dequantised per call, "
                      f"activations quantised per 128-group, float32 GEMMs; weights in host "
                      f"memory, so no page-in); {cpu_name()}"}


def _fp8_state_run(wl, cap: int, n_warm: int, n: int):
    """``_state_run`` for a block-FP8 workload: ``n`` timed layer calls on a
    fresh FP8 state with ``cap`` slots (cap = E: every expert stays resident
    after its first call)."""
    import torch

    from wisp.integrations.vllm.fused_moe_fp8 import WispMoEStateFP8
    dev = torch.device("cuda", 0)
    K = wl.shape.top_k
    xs, lgs = wl.x.to(dev), wl.logits.to(dev)
    out = torch.empty_like(xs[0])
    st = WispMoEStateFP8(*wl.views(), cap, dev, 0)
    r = _timed(lambda i: st.forward(xs[i % wl.steps], lgs[i % wl.steps], K, True, out=out),
               n_warm, n, [st])
    del st
    torch.cuda.empty_cache()
    return r


def _fp8_gemm_report(agg: dict, wl, tokens_per_call: int, distinct_per_call: float) -> dict:
    sh = wl.shape
    calls = max(1, agg["calls"])
    t = (agg["w13_ms"] / max(1, agg["w13_calls"]) + agg["w2_ms"] / calls) * 1e-3
    flops = 2.0 * tokens_per_call * sh.top_k * 3 * sh.hidden * sh.inter
    byts = distinct_per_call * wl.expert_bytes
    kernels = ("fp8_w13_dma_kernel + fp8_w2_dma_kernel" if tokens_per_call > 16
               else "fp8_grouped_w13_kernel + fp8_grouped_w2_kernel")
    return {"kernels": kernels,
            "avg_us_per_call": round(t * 1e6, 2),
            "w13_us": round(agg["w13_ms"] / max(1, agg["w13_calls"]) * 1e3, 2),
            "w2_us": round(agg["w2_ms"] / calls * 1e3, 2),
            "achieved_TFLOPs": round(flops / t / 1e12, 2) if t else None,
            "frac_fp8_mfma_peak": round(flops / t / 1e12 / FP8_PEAK_TFLOPS, 4) if t else None,
            "achieved_GBps": round(byts / t / 1e9, 1) if t else None,
            "frac_hbm_peak": round(byts / t / 1e9 / HBM_PEAK_GBPS, 4) if t else None,
            "bytes_per_call": int(byts), "flops_per_call": int(flops)}


def bench_fp8_prefill(args) -> dict:
    from wisp_amd import workloads as W
    wl = W.fp8_layer(W.gaussian_logits("batch", seed=0, steps=3, tokens=512, weights=False),
                     pin=True)
    sh = wl.shape
    pe, pa = _fp8_state_run(wl, sh.cap, 1, 2)
    re_, ra = _fp8_state_run(wl, sh.experts, 3, 20)
    dist = sum(_distinct(wl.logits[i], 8) for i in range(wl.steps)) / wl.steps
    line = _line("MoE prefill tok/s, Qwen3-30B-A3B-FP8 shape, 512-token chunk, cap=32 paged",
                 2 * 512 / pe, "tok/s", args, 2, pe,
                 {"workload": "qwen3-fp8 moe layer, 512-token prefill chunk, router logits N(0,1)",
                  "hidden": sh.hidden, "expert_intermediate": sh.inter, "experts": sh.experts,
                  "top_k": sh.top_k, "cap": sh.cap, "tokens": 512, "weight_block": list(wl.block)},
                 pagein=_pagein_report(pa),
                 resident={"tok_per_s": round(20 * 512 / re_, 1),
                           "expert_gemm": _fp8_gemm_report(ra, wl, 512, dist)})
    line["dtype"] = "fp8_e4m3 (bf16 activations, f32 accumulate)"
    return line


def bench_fp8_batch32(args) -> dict:
    from wisp_amd import workloads as W
    wl = W.fp8_layer(W.batch_decode(steps=24, tokens=32, weights=False), pin=True)
    sh = wl.shape
    pe, pa = _fp8_state_run(wl, sh.cap, 2, 16)
    re_, ra = _fp8_state_run(wl, sh.experts, 24, 128)
    dist = sum(_distinct(wl.logits[i], 8) for i in range(wl.steps)) / wl.steps
    line = _line("MoE batched decode tok/s, Qwen3-30B-A3B-FP8 shape, bs=32, cap=32 paged",
                 16 * 32 / pe, "tok/s", args, 16, pe,
                 {"workload": "qwen3-fp8 moe layer, bs=32 decode, router logits N(0,1)",
                  "hidden": sh.hidden, "expert_intermediate": sh.inter, "experts": sh.experts,
                  "top_k": sh.top_k, "cap": sh.cap, "batch": 32, "weight_block": list(wl.block)},
                 pagein=_pagein_report(pa),
                 resident={"tok_per_s": round(128 * 32 / re_, 1),
                           "expert_gemm": _fp8_gemm_report(ra, wl, 32, dist)})
    line["dtype"] = "fp8_e4m3 (bf16 activations, f32 accumulate)"
    return line


def bench_fp8(args) -> dict:
    """The default decode measurement on the block-FP8 twin of the Qwen3
    layer: same routing sequences, eight layer instances sharing one set of
    pinned FP8 masters."""
    import torch

    from wisp_amd import workloads as W
    from wisp.integrations.vllm.fused_moe_fp8 import WispMoEStateFP8
    R = args.replicas
    n_warm = R + args.warmup  # one priming call per instance, then `warmup` in total
    per = -(-(n_warm + args.steps) // R)
    t_setup = time.perf_counter()
    routes = [W.qwen3_decode(seed=r, steps=per, weights=False) for r in range(R)]
    wl = W.fp8_layer(routes[0], pin=True)
    sh = wl.shape
    views = wl.views()
    dev = torch.device("cuda", 0)
    xs = torch.stack([r.x for r in routes]).to(dev)
    lgs = torch.stack([r.logits for r in routes]).to(dev)
    states = [WispMoEStateFP8(*views, sh.cap, dev, r) for r in range(R)]
    outs = [torch.empty((1, sh.hidden), dtype=torch.bfloat16, device=dev) for _ in range(R)]
    log(f"fp8 setup {time.perf_counter() - t_setup:.1f}s: engine {states[0].pagein_engine}")

    def call(i: int) -> None:
        r, pos = i % R, i // R
        states[r].forward(xs[r, pos], lgs[r, pos], sh.top_k, True, out=outs[r])

    elapsed, agg = _timed(call, n_warm, args.steps, states)
    _calibration_copy(dev)
    lay = wl.layout
    K = sh.top_k
    t13 = agg["w13_ms"] / max(1, agg["w13_calls"]) * 1e-3
    # w2 of the same calls whose w13 is timed (fused launches that copied nothing)
    t2 = agg["w2_noload_ms"] / max(1, agg["w2_noload_calls"]) * 1e-3
    w13_bytes = K * (lay.w13_bytes + 4 * lay.s13_elems)
    w2_bytes = K * (lay.w2_bytes + 4 * lay.s2_elems)
    a13 = w13_bytes / t13 / 1e9 if t13 > 0 else 0.0
    agemm = (w13_bytes + w2_bytes) / (t13 + t2) / 1e9 if t13 + t2 > 0 else 0.0
    link = h2d_link(wl.expert_bytes)
    cpu = None
    if not args.no_cpu_baseline:
        t_cpu = time.perf_counter()
        croutes = [W.Workload(r.name, sh, r.x, r.logits, wl.slabs) for r in routes]
        cpu = cpu_baseline_fp8(croutes, views, args.cpu_seconds)
        log(f"cpu baseline {time.perf_counter() - t_cpu:.1f}s")
    line = _line("MoE decode tok/s, Qwen3-30B-A3B-FP8 shape bs=1 cap=8 (block-FP8 w8a8)",
                 args.steps / elapsed, "tok/s", args, args.steps, elapsed,
                 {"workload": "qwen3-30b-a3b-fp8 moe layer decode, bs=1, cap=8, paged from "
                              "pinned host",
                  "hidden": sh.hidden, "expert_intermediate": sh.inter, "experts": sh.experts,
                  "top_k": K, "cap": sh.cap, "batch": 1, "layer_instances": R,
                  "weight_block": list(wl.block), "untimed_calls": n_warm,
                  "priming_calls_per_instance": 1,
                  "routing": "zipf(1.1) bias + 0.6 reuse of previous top-8"},
                 roofline={"kernel": "pagein_fp8_w13_kernel (gate/up block-FP8 MFMA + SiLU*mul, "
                                     "one token; page-in blocks idle)",
                           "bound": "hbm", "achieved": round(a13, 1), "peak": HBM_PEAK_GBPS,
                           "unit": "GB/s", "frac": round(a13 / HBM_PEAK_GBPS, 4),
                           "traffic": pmc_traffic(os.path.join(
                               os.path.dirname(os.path.abspath(__file__)), "profiles",
                               "qwen3_fp8_decode_pmc.json"), "pagein_fp8_w13_kernel"),
                           "bytes_per_call": w13_bytes,
                           "avg_us_per_call": round(t13 * 1e6, 3),
                           "timing": "dispatch-timestamp events over a second pass of the timed "
                                     "calls; the fused page-in + w13 launch of the calls that "
                                     "paged nothing in (on the others it is page-in time)"},
                 expert_gemm={"kernels": "pagein_fp8_w13_kernel + fp8_w2_one_kernel",
                              "bytes_per_token": w13_bytes + w2_bytes,
                              "avg_us": round((t13 + t2) * 1e6, 3),
                              "achieved_GBps": round(agemm, 1),
                              "frac_hbm_peak": round(agemm / HBM_PEAK_GBPS, 4),
                              "w2_avg_us": round(t2 * 1e6, 3), "w13_calls": agg["w13_calls"],
                              "w2_calls": agg["w2_noload_calls"],
                              "timed_calls": agg["calls"],
                              "timing": "both stages averaged over the calls whose fused "
                                        "page-in + w13 launch copied nothing"},
                 pagein=dict(_pagein_report(agg), link_GBps_p50=round(link, 2),
                             expert_bytes=wl.expert_bytes),
                 cpu_baseline=cpu)
    line["dtype"] = "fp8_e4m3 (bf16 activations, f32 accumulate)"
    return line


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2048,
                    help="timed layer calls (default: 8 instances x 256 decode steps)")
    ap.add_argument("--warmup", type=int, default=8,
                    help="untimed calls in total before the timed window (the decode "
                         "workloads first give each layer instance one priming call)")
    ap.add_argument("--replicas", type=int, default=8)
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="time bound of the CPU baseline sample")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--workload", default="qwen3",
                    choices=["qwen3", "prefill", "batch32", "mixtral", "stack", "fp8",
                             "fp8-prefill", "fp8-batch32"])
    ap.add_argument("--prefetch", action="store_true",
                    help="stack workload: cross-layer speculative prefetch with a co-occurrence "
                         "table learned online (WISP_PREFETCH=1, WISP_COOCCUR_ONLINE=1)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported by this build "
              "(the paged MoE path has no multi-GPU mode)", file=sys.stderr)
        return 2

    if args.workload != "qwen3":
        line = {"prefill": bench_prefill, "batch32": bench_batch32, "mixtral": bench_mixtral,
                "stack": bench_stack, "fp8": bench_fp8, "fp8-prefill": bench_fp8_prefill,
                "fp8-batch32": bench_fp8_batch32}[args.workload](args)
        print(json.dumps(line), flush=True)
        return 0

    import torch

    from wisp_amd import workloads as W
    from wisp.integrations.vllm.fused_moe import WispMoEState

    R = args.replicas
    # Each instance first takes one priming call: its cold fill, which loads
    # the first token's experts into its empty scratch.  With cap == top_k
    # the scratch holds exactly the last call's experts after every call, so
    # one call puts an instance in the pager's steady state (the analogue of
    # the model load that fills a serving layer's scratch).  Then `warmup`
    # untimed calls in total, round-robin, then the K timed calls.
    n_prime = R
    n_warm = n_prime + args.warmup
    per = -(-(n_warm + args.steps) // R)
    t_setup = time.perf_counter()
    base = W.qwen3_decode(seed=0, steps=per, pin=True)
    sh = base.shape
    w13, w2 = base.views()
    dev = torch.device("cuda", 0)
    routes = [base] + [W.qwen3_decode(seed=r, steps=per, weights=False) for r in range(1, R)]
    xs = torch.stack([wl.x for wl in routes]).to(dev)          # [R, per, 1, H]
    lgs = torch.stack([wl.logits for wl in routes]).to(dev)    # [R, per, 1, E]
    states = [WispMoEState(w13, w2, sh.cap, "paged", dev, r) for r in range(R)]
    outs = [torch.empty((1, sh.hidden), dtype=sh.dtype, device=dev) for _ in range(R)]
    log(f"setup {time.perf_counter() - t_setup:.1f}s: {R} x qwen3 layer, cap={sh.cap}, "
        f"{per} routing steps each")

    def call(i: int) -> None:
        r, pos = i % R, i // R
        states[r].forward(xs[r, pos], lgs[r, pos], sh.top_k, True, out=outs[r])

    def counts() -> tuple[int, int]:
        return sum(st.stats_miss for st in states), sum(st.stats_hits for st in states)

    def run_steps() -> float:
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(n_warm, n_warm + args.steps):
            call(i)
        torch.cuda.synchronize()
        return time.perf_counter() - t0

    for i in range(n_warm):
        call(i)
    torch.cuda.synchronize()

    # `value`: the K steps as the library runs them, with timing off (each
    # event-timed launch lengthens the stream by a few microseconds)
    m0, h0 = counts()
    elapsed = run_steps()
    m1, h1 = counts()
    miss, hits = m1 - m0, h1 - h0
    log(f"timed {args.steps} layer calls in {elapsed:.3f}s")

    # kernel and page-in durations: the same K steps again with
    # dispatch-timestamp events on the w13, w2 and page-in launches
    for st in states:
        st.profile(True)
        st.pagein_stats()
    elapsed_ev = run_steps()
    log(f"timed {args.steps} layer calls with kernel events in {elapsed_ev:.3f}s")
    prof = {"w13": 0.0, "w2": 0.0, "calls": 0, "w13_calls": 0, "w2_noload": 0.0,
            "w2_noload_calls": 0}
    pin_ms = pin_bytes = 0.0
    for st in states:
        for k, v in st.profile(False).items():
            prof[k] += v
        ms, nb = st.pagein_stats()
        pin_ms, pin_bytes = pin_ms + ms, pin_bytes + nb
    K = sh.top_k
    w13_bytes = K * 2 * sh.inter * sh.hidden * sh.elem_bytes
    w2_bytes = K * sh.hidden * sh.inter * sh.elem_bytes
    calls = max(1, prof["calls"])
    t13 = prof["w13"] / max(1, prof["w13_calls"]) * 1e-3
    # the pair over one set of calls: w2 of the same calls whose w13 is timed
    # (those whose fused page-in + w13 launch copied nothing)
    t2 = prof["w2_noload"] / max(1, prof["w2_noload_calls"]) * 1e-3
    t2_all = prof["w2"] / calls * 1e-3
    a13 = w13_bytes / t13 / 1e9 if t13 > 0 else 0.0
    agemm = (w13_bytes + w2_bytes) / (t13 + t2) / 1e9 if t13 + t2 > 0 else 0.0

    _calibration_copy(dev)

    link = h2d_link(sh.expert_bytes)
    link_big = h2d_link(256 << 20, iters=8)
    pin_gbps = pin_bytes / (pin_ms * 1e-3) / 1e9 if pin_ms > 0 else 0.0

    cpu = None
    if not args.no_cpu_baseline:
        t_cpu = time.perf_counter()
        cpu = cpu_baseline(routes, w13, w2, args.cpu_seconds)
        log(f"cpu baseline {time.perf_counter() - t_cpu:.1f}s")
    pmc_path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                            "qwen3_decode_pmc.json")
    # bf16 masters page in from their packed copy unless WISP_PACKED_MASTERS=0
    packed = states[0]._packed is not None
    w13_kernel = "pagein_w13_packed_kernel" if packed else "pagein_w13_kernel"
    traffic = pmc_traffic(pmc_path, w13_kernel)
    link_best = max(link, link_big)  # the host link's best measured hipMemcpyAsync rate
    # bytes the host link carried: the packed copy's stride per loaded expert
    link_bytes = pin_bytes * states[0].packed_bytes_per_expert / sh.expert_bytes
    link_gbps = link_bytes / (pin_ms * 1e-3) / 1e9 if pin_ms > 0 else 0.0

    value = args.steps / elapsed
    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(elapsed / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "qwen3-30b-a3b moe layer decode, bs=1, cap=8, paged from pinned host",
            "hidden": sh.hidden, "expert_intermediate": sh.inter, "experts": sh.experts,
            "top_k": K, "cap": sh.cap, "batch": 1, "layer_instances": R,
            "untimed_calls": n_warm,
            "priming_calls_per_instance": 1,
            "routing": "zipf(1.1) bias + 0.6 reuse of previous top-8",
        },
        "roofline": {
            "kernel": f"{w13_kernel} (gate/up GEMV + SiLU*mul; page-in blocks idle)",
            "bound": "hbm",
            "achieved": round(a13, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(a13 / HBM_PEAK_GBPS, 4),
            "traffic": traffic,
            "bytes_per_call": w13_bytes,
            "avg_us_per_call": round(t13 * 1e6, 3),
            "timing": f"dispatch-timestamp events over a second pass of the {args.steps} steps "
                      f"({elapsed_ev / args.steps * 1e3:.4f} ms per step with the events); "
                      f"the fused page-in + w13 launch of the {prof['w13_calls']} calls that "
                      f"paged nothing in (on the others it is page-in time)",
            "timing_off": timing_off(pmc_path, w13_kernel, w13_bytes),
        },
        "expert_gemm": {
            "kernels": f"{w13_kernel} + w2_combine_kernel",
            "bytes_per_token": w13_bytes + w2_bytes,
            "avg_us": round((t13 + t2) * 1e6, 3),
            "achieved_GBps": round(agemm, 1),
            "frac_hbm_peak": round(agemm / HBM_PEAK_GBPS, 4),
            "w2_avg_us": round(t2 * 1e6, 3),
            "w13_calls": prof["w13_calls"],
            "w2_calls": prof["w2_noload_calls"],
            "w2_avg_us_all_calls": round(t2_all * 1e6, 3),
            "timed_calls": prof["calls"],
            "timing": "both stages averaged over the calls whose fused page-in + w13 launch "
                      "copied nothing",
        },
        "pagein": {
            "bytes": pin_bytes,
            "achieved_GBps": round(pin_gbps, 2),
            "packed_masters": packed,
            "link_bytes_per_expert": states[0].packed_bytes_per_expert,
            "expert_bytes": sh.expert_bytes,
            "link_bytes": link_bytes,
            "link_achieved_GBps": round(link_gbps, 2),
            "link_GBps_9MiB_p50": round(link, 2),
            "link_GBps_256MiB_p50": round(link_big, 2),
            "frac_of_link": round(link_gbps / link_best, 4) if link_best else None,
            "misses": miss, "hits": hits,
            "misses_per_call": round(miss / max(1, args.steps), 3),
            "timing": "copy-kernel events over the second pass; misses and hits of the first; "
                      "bytes and achieved_GBps count each loaded expert's bf16 bytes, link_* "
                      "the bytes read over the host link",
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
