"""wisp_moe_experts_noalloc through the C ABI against wisp_moe_experts.

The entry point that allocates nothing keeps act and the MFMA work buffer in
the library's static device array; its outputs must be bit-identical to the
entry point that takes them as arguments, on two calls in a row (the second
smaller, so it runs on what the first left in the array), for the GEMV and the
MFMA path and the fp32 GEMV path.  A call larger than the array is refused
before any launch.
"""
import ctypes as C

import numpy as np
import pytest
import torch

from wisp_amd import _lib

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _case(T, H, I, E, K, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn((T, H), generator=g)).to(dtype).to(DEV)
    w13 = (torch.randn((E, 2 * I, H), generator=g) * 0.02).to(dtype).to(DEV)
    w2 = (torch.randn((E, H, I), generator=g) * 0.02).to(dtype).to(DEV)
    ids = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)]).to(torch.int32)
    if T > 1:
        ids[1, 0] = -1  # an absent slot contributes zero
    w = torch.softmax(torch.randn((T, K), generator=g), dim=-1)
    return x, w13, w2, ids.to(DEV), w.to(DEV)


def _with_buffers(x, w13, w2, slots, w, algo, dtype):
    T, H = x.shape
    E, _, I = w2.shape
    K = slots.shape[1]
    act = torch.empty((max(1, T * K), I), dtype=dtype, device=DEV)
    nbytes = _lib.lib().wisp_moe_work_bytes(max(1, T), K, H, E)
    work = torch.empty(max(256, nbytes), dtype=torch.uint8, device=DEV)
    out = torch.empty_like(x)
    _lib.check(_lib.lib().wisp_moe_experts(
        x.data_ptr(), _lib.WISP_BF16 if dtype == torch.bfloat16 else _lib.WISP_F32, T, H, I, K,
        w.data_ptr(), slots.data_ptr(), E, w13.data_ptr(), w13.stride(0), w2.data_ptr(),
        w2.stride(0), act.data_ptr(), out.data_ptr(), work.data_ptr(), work.numel(), algo,
        _lib.stream_handle()), "experts")
    return out


def _noalloc(x, w13, w2, slots, w, algo, dtype):
    T, H = x.shape
    E, _, I = w2.shape
    K = slots.shape[1]
    out = torch.empty_like(x)
    _lib.check(_lib.lib().wisp_moe_experts_noalloc(
        x.data_ptr(), _lib.WISP_BF16 if dtype == torch.bfloat16 else _lib.WISP_F32, T, H, I, K,
        w.data_ptr(), slots.data_ptr(), E, w13.data_ptr(), w13.stride(0), w2.data_ptr(),
        w2.stride(0), out.data_ptr(), algo, _lib.stream_handle()), "experts_noalloc")
    return out


def _bits(t):
    return t.view(torch.int16) if t.dtype == torch.bfloat16 else t.view(torch.int32)


@pytest.mark.parametrize("dtype,algo,shape", [
    (torch.bfloat16, _lib.WISP_ALGO_GEMV, (2048, 768, 32, 8)),
    (torch.bfloat16, _lib.WISP_ALGO_MFMA, (2048, 768, 32, 8)),
    (torch.bfloat16, _lib.WISP_ALGO_AUTO, (512, 256, 16, 4)),
    (torch.float32, _lib.WISP_ALGO_GEMV, (512, 256, 16, 2)),
], ids=["bf16-gemv", "bf16-mfma", "bf16-auto", "f32-gemv"])
def test_noalloc_equals_workspace_entry_point(dtype, algo, shape):
    H, I, E, K = shape
    for T, seed in ((24, 1), (5, 2)):  # the second call is smaller
        print(f"noalloc {dtype} algo={algo} H={H} I={I} E={E} K={K} T={T}", flush=True)
        x, w13, w2, slots, w = _case(T, H, I, E, K, dtype, seed)
        ref = _with_buffers(x, w13, w2, slots, w, algo, dtype)
        got = _noalloc(x, w13, w2, slots, w, algo, dtype)
        torch.cuda.synchronize()
        assert torch.equal(_bits(got), _bits(ref)), T
        assert bool(torch.isfinite(got.float()).all())


def test_noalloc_refuses_calls_beyond_its_array():
    H, I, E, K = 2048, 768, 16, 8
    T = 4096  # act alone is 48 MiB, plus 268 MiB of MFMA work
    assert _lib.lib().wisp_noalloc_scratch_bytes() < (48 + 268) << 20
    x = torch.zeros((T, H), dtype=torch.bfloat16, device=DEV)
    w13 = torch.zeros((E, 2 * I, H), dtype=torch.bfloat16, device=DEV)
    w2 = torch.zeros((E, H, I), dtype=torch.bfloat16, device=DEV)
    slots = torch.zeros((T, K), dtype=torch.int32, device=DEV)
    w = torch.zeros((T, K), dtype=torch.float32, device=DEV)
    out = torch.full((T, H), 7, dtype=torch.bfloat16, device=DEV)
    rc = _lib.lib().wisp_moe_experts_noalloc(
        x.data_ptr(), _lib.WISP_BF16, T, H, I, K, w.data_ptr(), slots.data_ptr(), E,
        w13.data_ptr(), w13.stride(0), w2.data_ptr(), w2.stride(0), out.data_ptr(),
        _lib.WISP_ALGO_MFMA, _lib.stream_handle())
    torch.cuda.synchronize()
    assert rc == _lib.WISP_ERR_INVALID
    assert "WISP_NOALLOC_SCRATCH_BYTES" in _lib.last_error()
    assert bool((out == 7).all())  # nothing ran
