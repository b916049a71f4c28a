"""Oracle: block-FP8 (w8a8) fused-MoE experts on the CPU — TEST INFRASTRUCTURE ONLY.

The reference's FP8 path (``src/wisp/integrations/vllm/fused_moe_fp8.py``)
pages four tensors per expert (``w13``/``w2`` in float8_e4m3fn and their
float32 block scales, 61-145) and hands the math to vLLM 0.11.2 (not
vendored, absent here): ``fused_experts(..., quant_config=
fp8_w8a8_moe_quant_config(w1_scale=scratch_s13, w2_scale=scratch_s2,
a1_scale=None, a2_scale=None, block_shape=[bn, bk]))`` on the Triton backend
(245-249, 316-326).  The published algorithm of that call, restated here:

1. ``quant_groups`` (vLLM ``per_token_group_quant_fp8``): per row and group
   of ``bk`` columns, ``s = max(max|x|, 1e-10) / 448`` and
   ``q = e4m3fn(clamp(x / s, -448, 448))``, float32, round to nearest even.
2. ``block_gemm`` (vLLM ``fused_moe_kernel`` with ``use_fp8_w8a8`` and a
   block shape): for each k-block ``kb`` of ``bk`` columns, in order,
   ``acc += (dot(q_a[kb], q_w[n, kb]) * s_a[kb]) * s_w[n // bn, kb]`` in
   float32; the dot of two fp8 vectors is taken exactly (its float64 sum is
   exact) and rounded once to float32.
3. w13: ``h = bf16(block_gemm(q_x, W13))``, gate rows first, then up rows.
4. ``silu_and_mul`` (vLLM's kernel): ``act = bf16(bf16(silu(g)) * u)`` with
   ``silu(g) = g / (1 + exp(-g))`` in float32.
5. act quantised as in 1; w2: ``y = bf16(block_gemm(q_act, W2) * w)`` with
   the routing weight ``w`` (float32).
6. ``moe_sum`` over the top-k in routing order: for K in {2, 3, 4} the
   bfloat16 sum is rounded after every add; for other K the sum is taken in
   float32 and rounded once.  An expert that the map marks absent gives
   ``y = 0``.

Pinning (``tests/test_oracle_fp8.py``): the e4m3fn codec against torch's
``float8_e4m3fn`` conversions (every code, every tie); the group quantiser
by closed forms (the largest element maps to +-448, ``s = absmax / 448``,
power-of-two invariance, zero groups); ``block_gemm`` against the dense
product of independently dequantised operands and a hand-computed case; the
w13 stage bit-exactly on inputs whose sums are exact; the whole MLP against
the unquantised oracle (``oracle.moe.moe_forward``) on the dequantised
weights within the fp8 rounding bound; the ``moe_sum`` rule by known
answers.  The rounding steps of 3-6 follow vLLM's kernels as published; no
reference-held vector pins them (the reference ships no FP8 fixtures).
"""
from __future__ import annotations

import numpy as np
import torch

E4M3_MAX = 448.0
QUANT_EPS = 1e-10
_F32 = np.float32


def _decode_table() -> np.ndarray:
    """Value of every e4m3fn code from the bit layout: sign, 4 exponent bits
    (bias 7), 3 mantissa bits; exponent 0 is subnormal (m * 2^-9); S.1111.111
    is NaN; there is no infinity."""
    out = np.empty(256, dtype=np.float64)
    for b in range(256):
        s, e, m = b >> 7, (b >> 3) & 15, b & 7
        if e == 15 and m == 7:
            v = np.nan
        elif e == 0:
            v = m * 2.0 ** -9
        else:
            v = (1.0 + m / 8.0) * 2.0 ** (e - 7)
        out[b] = -v if s else v
    return out


DECODE = _decode_table()
# the 127 non-negative finite codes 0x00..0x7E ascend with their value
_POS_VALUES = DECODE[:0x7F]


def fp8_decode(codes) -> np.ndarray:
    """e4m3fn codes (uint8) -> float64 values."""
    return DECODE[np.asarray(codes, dtype=np.uint8)]


def fp8_encode(x) -> np.ndarray:
    """float values with |x| <= 448 -> e4m3fn codes, round to nearest, ties
    to the even code (the even mantissa)."""
    x = np.asarray(x, dtype=np.float64)
    if np.any(np.abs(x) > E4M3_MAX) or np.any(np.isnan(x)):
        raise ValueError("fp8_encode takes finite values within +-448")
    a = np.abs(x)
    hi = np.searchsorted(_POS_VALUES, a, side="left").clip(0, 0x7E)
    lo = np.maximum(hi - 1, 0)
    d_hi = _POS_VALUES[hi] - a
    d_lo = a - _POS_VALUES[lo]
    pick_lo = (d_lo < d_hi) | ((d_lo == d_hi) & (lo % 2 == 0))
    code = np.where(pick_lo, lo, hi).astype(np.uint8)
    return np.where(np.signbit(x), code | 0x80, code).astype(np.uint8)


def quant_groups(x, group: int) -> tuple[np.ndarray, np.ndarray]:
    """Per-row, per-group dynamic fp8 quantisation (vLLM
    ``per_token_group_quant_fp8``): ``x [R, C]`` (float32 values) ->
    ``(codes uint8 [R, C], scales float32 [R, ceil(C / group)])``."""
    x = np.asarray(x, dtype=_F32)
    R, Cc = x.shape
    ng = -(-Cc // group)
    codes = np.empty((R, Cc), dtype=np.uint8)
    scales = np.empty((R, ng), dtype=_F32)
    for g in range(ng):
        xs = x[:, g * group:(g + 1) * group]
        amax = np.maximum(np.abs(xs).max(axis=1), _F32(QUANT_EPS)).astype(_F32)
        s = (amax / _F32(E4M3_MAX)).astype(_F32)
        q = np.clip((xs / s[:, None]).astype(_F32), _F32(-E4M3_MAX), _F32(E4M3_MAX))
        codes[:, g * group:(g + 1) * group] = fp8_encode(q)
        scales[:, g] = s
    return codes, scales


def block_gemm(a_codes, a_scales, w_codes, w_scales, bn: int, bk: int) -> np.ndarray:
    """Block-scaled fp8 GEMM: ``a [R, Kd]`` codes with per-row group scales
    ``[R, ceil(Kd / bk)]``, ``w [N, Kd]`` codes with block scales
    ``[ceil(N / bn), ceil(Kd / bk)]`` -> ``[R, N]`` float32."""
    av = fp8_decode(a_codes)
    wv = fp8_decode(w_codes)
    a_scales = np.asarray(a_scales, dtype=_F32)
    w_scales = np.asarray(w_scales, dtype=_F32)
    R, Kd = av.shape
    N = wv.shape[0]
    nkb = -(-Kd // bk)
    rows = np.arange(N) // bn
    acc = np.zeros((R, N), dtype=_F32)
    for kb in range(nkb):
        sl = slice(kb * bk, min((kb + 1) * bk, Kd))
        d = (av[:, sl] @ wv[:, sl].T).astype(_F32)          # exact sum, one rounding
        t = (d * a_scales[:, kb:kb + 1]).astype(_F32)
        t = (t * w_scales[rows, kb][None, :]).astype(_F32)
        acc = (acc + t).astype(_F32)
    return acc


def bf16(a) -> np.ndarray:
    """Round float32 values to bfloat16 (nearest even); float32 result."""
    t = torch.from_numpy(np.ascontiguousarray(np.asarray(a, dtype=_F32)))
    return t.to(torch.bfloat16).to(torch.float32).numpy()


def silu_and_mul(h) -> np.ndarray:
    """``h [R, 2I]`` bf16 values (gate | up) -> act bf16 values ``[R, I]``."""
    h = np.asarray(h, dtype=_F32)
    I = h.shape[1] // 2
    g, u = h[:, :I], h[:, I:]
    with np.errstate(over="ignore"):
        silu = (g / (_F32(1.0) + np.exp(-g).astype(_F32))).astype(_F32)
    return bf16((bf16(silu) * u).astype(_F32))


def moe_sum(y) -> np.ndarray:
    """``y [T, K, H]`` bf16 values -> ``[T, H]``: K in {2, 3, 4} adds in
    bfloat16 in routing order, other K sums in float32 and rounds once."""
    y = np.asarray(y, dtype=_F32)
    K = y.shape[1]
    if K in (2, 3, 4):
        acc = np.zeros((y.shape[0], y.shape[2]), dtype=_F32)
        for k in range(K):
            acc = bf16((acc + y[:, k]).astype(_F32))
        return acc
    return bf16(y.astype(np.float64).sum(axis=1).astype(_F32))


def w13_stage(x, w13_codes, s13, bn: int, bk: int) -> tuple[np.ndarray, np.ndarray]:
    """``x [R, H]`` (bf16 values) through one expert's w13: returns
    ``(h bf16 values [R, 2I], act bf16 values [R, I])``."""
    xq, xs = quant_groups(np.asarray(x, dtype=_F32), bk)
    h = bf16(block_gemm(xq, xs, w13_codes, s13, bn, bk))
    return h, silu_and_mul(h)


def w2_stage(act, w2_codes, s2, weight, bn: int, bk: int) -> np.ndarray:
    """``act [R, I]`` through one expert's w2, times the routing weights
    ``weight [R]``: bf16 values ``[R, H]``."""
    aq, as_ = quant_groups(np.asarray(act, dtype=_F32), bk)
    y = block_gemm(aq, as_, w2_codes, s2, bn, bk)
    return bf16((y * np.asarray(weight, dtype=_F32)[:, None]).astype(_F32))


def _codes(t) -> np.ndarray:
    if isinstance(t, torch.Tensor):
        if t.dtype == torch.float8_e4m3fn:
            t = t.view(torch.uint8)
        return t.cpu().numpy()
    return np.asarray(t, dtype=np.uint8)


def moe_forward_fp8(x, topk_w, topk_ids, w13, w2, s13, s2, block=(128, 128),
                    expert_map=None, return_act: bool = False):
    """Block-FP8 SwiGLU experts with the routing-order ``moe_sum``.

    ``x [T, H]`` (bf16), ``topk_w [T, K]`` (float32), ``topk_ids [T, K]``
    (global ids), ``w13 [E, 2I, H]`` / ``w2 [E, H, I]`` (float8_e4m3fn or
    uint8 codes), ``s13 [E, 2*ceil(I/bn), ceil(H/bk)]`` /
    ``s2 [E, ceil(H/bn), ceil(I/bk)]`` (float32).  Returns the output as
    float32 values of bfloat16 ``[T, H]`` (and ``act [T, K, I]`` when
    ``return_act``)."""
    bn, bk = block
    xv = torch.as_tensor(x).to(torch.float32).numpy()
    tw = np.asarray(torch.as_tensor(topk_w).to(torch.float32).cpu().numpy(), dtype=_F32)
    ids = np.asarray(torch.as_tensor(topk_ids).cpu().numpy(), dtype=np.int64)
    w13c, w2c = _codes(w13), _codes(w2)
    s13 = np.asarray(torch.as_tensor(s13).to(torch.float32).cpu().numpy(), dtype=_F32)
    s2 = np.asarray(torch.as_tensor(s2).to(torch.float32).cpu().numpy(), dtype=_F32)
    T, K = ids.shape
    H = xv.shape[1]
    I = w2c.shape[2]
    y = np.zeros((T, K, H), dtype=_F32)
    act = np.zeros((T, K, I), dtype=_F32)
    for e in np.unique(ids):
        e = int(e)
        if expert_map is not None and int(expert_map[e]) < 0:
            continue
        rows = np.argwhere(ids == e)
        _, a = w13_stage(xv[rows[:, 0]], w13c[e], s13[e], bn, bk)
        act[rows[:, 0], rows[:, 1]] = a
        y[rows[:, 0], rows[:, 1]] = w2_stage(a, w2c[e], s2[e], tw[rows[:, 0], rows[:, 1]], bn, bk)
    out = moe_sum(y)
    return (out, act) if return_act else out


def dequantize(codes, scales, bn: int, bk: int) -> np.ndarray:
    """Dense float64 ``[N, Kd]`` from block-scaled codes (for checks)."""
    v = fp8_decode(_codes(codes))
    s = np.asarray(scales, dtype=np.float64)
    N, Kd = v.shape
    return v * s[np.arange(N)[:, None] // bn, np.arange(Kd)[None, :] // bk]


def quantize_weights(w, bn: int = 128, bk: int = 128) -> tuple[np.ndarray, np.ndarray]:
    """Block-quantise dense weights ``[N, Kd]`` the way FP8 checkpoints are
    made (per-block ``s = absmax / 448``): ``(codes uint8, scales float32)``.
    Test-data helper."""
    w = np.asarray(w, dtype=_F32)
    N, Kd = w.shape
    nb, kb = -(-N // bn), -(-Kd // bk)
    codes = np.empty((N, Kd), dtype=np.uint8)
    scales = np.empty((nb, kb), dtype=_F32)
    for i in range(nb):
        for j in range(kb):
            blk = w[i * bn:(i + 1) * bn, j * bk:(j + 1) * bk]
            s = _F32(max(float(np.abs(blk).max()), 1e-12) / E4M3_MAX)
            scales[i, j] = s
            codes[i * bn:(i + 1) * bn, j * bk:(j + 1) * bk] = fp8_encode(
                np.clip(blk / s, -E4M3_MAX, E4M3_MAX))
    return codes, scales


def _dequant_blocks(codes: torch.Tensor, scales: torch.Tensor, bn: int, bk: int) -> torch.Tensor:
    """Block-FP8 weights ``[N, Kd]`` (e4m3fn) with block scales -> float32."""
    w = codes.view(torch.float8_e4m3fn).to(torch.float32) if codes.dtype != torch.float8_e4m3fn \
        else codes.to(torch.float32)
    s = scales.to(torch.float32).repeat_interleave(bn, 0)[:w.shape[0]]
    return w * s.repeat_interleave(bk, 1)[:, :w.shape[1]]


def _quant_dequant_rows(x: torch.Tensor, bk: int) -> torch.Tensor:
    """Per-row, per-group e4m3fn quantisation of ``x [R, C]`` (float32) and
    back: the values a w8a8 GEMM sees for its activations."""
    R, Cc = x.shape
    g = x.view(R, Cc // bk, bk)
    s = g.abs().amax(dim=2, keepdim=True).clamp_min(QUANT_EPS) / E4M3_MAX
    q = (g / s).clamp(-E4M3_MAX, E4M3_MAX).to(torch.float8_e4m3fn).to(torch.float32)
    return (q * s).view(R, Cc)


def moe_forward_fp8_fast(x, topk_w, topk_ids, w13, w2, s13, s2, block=(128, 128)) -> torch.Tensor:
    """The torch CPU block-FP8 fused-MoE timed as the CPU baseline of the
    block-FP8 decode line (a plain torch implementation, not the oracle):
    per routed expert, the weight blocks dequantised to float32, the
    activations quantised per 128-group and back (w8a8), float32
    ``linear``, SiLU*mul with vLLM's two bf16 roundings, the same for w2,
    and the routing-order combine in float32.  Needs H and I to be multiples of the
    block."""
    bn, bk = block
    x = torch.as_tensor(x).to(torch.float32)
    ids = np.asarray(topk_ids, dtype=np.int64)
    tw = torch.as_tensor(np.asarray(topk_w, dtype=np.float32))
    T, K = ids.shape
    I = w2.shape[2]
    y = torch.zeros((T, K, x.shape[1]), dtype=torch.float32)
    for e in np.unique(ids):
        e = int(e)
        rows = np.argwhere(ids == e)
        xt = _quant_dequant_rows(x[torch.as_tensor(rows[:, 0])], bk)
        h = torch.nn.functional.linear(xt, _dequant_blocks(w13[e], s13[e], bn, bk))
        h = h.to(torch.bfloat16).to(torch.float32)
        silu = torch.nn.functional.silu(h[:, :I]).to(torch.bfloat16).float()
        act = (silu * h[:, I:]).to(torch.bfloat16).float()
        yy = torch.nn.functional.linear(_quant_dequant_rows(act, bk),
                                        _dequant_blocks(w2[e], s2[e], bn, bk))
        y[torch.as_tensor(rows[:, 0]), torch.as_tensor(rows[:, 1])] = yy
    out = torch.zeros((T, x.shape[1]), dtype=torch.float32)
    for k in range(K):
        out += tw[:, k:k + 1] * y[:, k]
    return out.to(torch.bfloat16)
