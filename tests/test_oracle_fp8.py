"""Pins the block-FP8 oracle (oracle/fp8.py): the e4m3fn codec against
torch's float8_e4m3fn conversions, the group quantiser and the block-scaled
GEMM by closed forms and independent dequantisation, the w13 stage bit-exactly
on inputs whose sums are exact, and the whole MLP against the unquantised
oracle on the dequantised weights."""
import numpy as np
import pytest
import torch

from oracle import fp8 as F
from oracle.moe import moe_forward

T8 = torch.float8_e4m3fn


def _torch_decode(codes):
    return torch.from_numpy(np.asarray(codes, dtype=np.uint8)).view(T8).to(torch.float64).numpy()


def _torch_encode(x):
    return torch.from_numpy(np.asarray(x, dtype=np.float32)).to(T8).view(torch.uint8).numpy()


def test_decode_every_code_matches_torch():
    codes = np.arange(256, dtype=np.uint8)
    got, want = F.fp8_decode(codes), _torch_decode(codes)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    assert np.array_equal(got[ok], want[ok])
    assert F.fp8_decode([0x7E])[0] == 448.0 and F.fp8_decode([0x01])[0] == 2.0 ** -9


def test_encode_matches_torch_on_ties_and_sweep():
    rng = np.random.default_rng(0)
    vals = np.unique(F.DECODE[np.isfinite(F.DECODE)])
    mids = (vals[:-1] + vals[1:]) / 2
    x = np.concatenate([vals, mids, np.nextafter(mids, np.inf), np.nextafter(mids, -np.inf),
                        rng.uniform(-448, 448, 20000), rng.uniform(-0.03, 0.03, 20000),
                        [0.0, -0.0, 448.0, -448.0]]).astype(np.float32)
    x = x[np.abs(x) <= 448]
    assert np.array_equal(F.fp8_encode(x), _torch_encode(x))
    with pytest.raises(ValueError):
        F.fp8_encode([449.0])


def test_group_quant_closed_forms():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal((5, 384)) * rng.uniform(0.01, 100, (5, 1))).astype(np.float32)
    x[3, 128:256] = 0.0                      # an all-zero group
    q, s = F.quant_groups(x, 128)
    assert q.shape == x.shape and s.shape == (5, 3) and s.dtype == np.float32
    for r in range(5):
        for g in range(3):
            blk = x[r, g * 128:(g + 1) * 128]
            amax = np.float32(max(np.abs(blk).max(), np.float32(1e-10)))
            assert s[r, g] == np.float32(amax / np.float32(448.0))
            if amax > 1e-10:
                i = int(np.argmax(np.abs(blk)))
                assert q[r, g * 128 + i] == (0xFE if blk[i] < 0 else 0x7E)   # +-448
                deq = F.fp8_decode(q[r, g * 128:(g + 1) * 128]) * s[r, g]
                # e4m3: 3 mantissa bits -> half-ulp 2^-4 relative in the normal
                # range, absolute 2^-10 * s below it
                err = np.abs(deq - blk)
                assert np.all(err <= np.maximum(np.abs(blk) * 2.0 ** -4, 2.0 ** -10 * s[r, g])
                              * (1 + 1e-6))
            else:
                assert not q[r, g * 128:(g + 1) * 128].any()
    # power-of-two scaling leaves the codes and scales the scales exactly
    q2, s2 = F.quant_groups(x * np.float32(8.0), 128)
    keep = s[:, :] > 1e-9
    assert np.array_equal(q2[:, :128][keep[:, 0]], q[:, :128][keep[:, 0]])
    assert np.array_equal(s2[keep], (s * np.float32(8.0))[keep])
    # a partial last group
    q3, s3 = F.quant_groups(x[:, :200], 128)
    assert s3.shape == (5, 2) and np.array_equal(q3[:, :128], q[:, :128])


def test_block_gemm_matches_dense_dequantised_product():
    rng = np.random.default_rng(2)
    finite = np.nonzero(np.isfinite(F.DECODE))[0].astype(np.uint8)
    for (R, N, Kd, bn, bk) in [(3, 384, 256, 128, 128), (2, 96, 200, 32, 64), (4, 40, 130, 16, 128)]:
        a = rng.choice(finite, (R, Kd))
        w = rng.choice(finite, (N, Kd))
        sa = rng.uniform(1e-3, 2, (R, -(-Kd // bk))).astype(np.float32)
        sw = rng.uniform(1e-3, 2, (-(-N // bn), -(-Kd // bk))).astype(np.float32)
        got = F.block_gemm(a, sa, w, sw, bn, bk)
        dense = F.dequantize(a, sa, 1, bk) @ F.dequantize(w, sw, bn, bk).T
        scale = np.abs(F.dequantize(a, sa, 1, bk)) @ np.abs(F.dequantize(w, sw, bn, bk)).T
        assert np.all(np.abs(got - dense) <= 1e-6 * scale + 1e-30)


def test_block_gemm_known_answer():
    # bk = 2, bn = 1: a = [1, 2 | 3, 4] with group scales [0.5, 2];
    # w row 0 = [1, 1 | 1, 1] scale [[1, 1]], row 1 = [2, 0 | 0, 2] scale [[0.25, 4]]
    enc = F.fp8_encode
    a = enc([[1, 2, 3, 4]])
    w = enc([[1, 1, 1, 1], [2, 0, 0, 2]])
    sa = np.array([[0.5, 2.0]], np.float32)
    sw = np.array([[1.0, 1.0], [0.25, 4.0]], np.float32)
    got = F.block_gemm(a, sa, w, sw, 1, 2)
    # row 0: (1+2)*0.5*1 + (3+4)*2*1 = 15.5; row 1: 2*0.5*0.25 + 8*2*4 = 64.25
    assert got.tolist() == [[15.5, 64.25]]


def test_w13_stage_exact_on_exact_inputs():
    # x groups have |max| = 448 * 2^m and fp8 values times 2^m, so the
    # activation quantiser is exact; weights are small fp8 values with
    # power-of-two block scales, so every sum is exact in float32: h must be
    # the bf16 rounding of the exact float64 product
    rng = np.random.default_rng(3)
    H, I, bn, bk = 256, 64, 32, 128
    small = F.fp8_encode(np.array([-2, -1, -0.5, 0, 0.5, 1, 2, 1.5, -1.5]))
    xv = F.fp8_decode(rng.choice(small, (2, H)))
    xv[:, 0] = 448.0
    xv[:, 128] = -448.0
    xv *= np.array([[0.25], [4.0]])
    w = rng.choice(small, (2 * I, H))
    sw = (2.0 ** rng.integers(-3, 3, (2 * I // bn, H // bk))).astype(np.float32)
    h, act = F.w13_stage(xv.astype(np.float32), w, sw, bn, bk)
    exact = xv @ F.dequantize(w, sw, bn, bk).T
    assert np.array_equal(h, F.bf16(exact.astype(np.float32)))
    g, u = h[:, :I].astype(np.float64), h[:, I:].astype(np.float64)
    ref = torch.nn.functional.silu(torch.from_numpy(g)).numpy() * u
    assert np.allclose(act, ref, rtol=2 ** -7, atol=1e-30)


def test_moe_sum_rule_known_answers():
    one, tiny = 1.0, 2.0 ** -8
    y = np.array([[[one], [tiny], [tiny]]], np.float32)       # K = 3: bf16 adds
    # 1 + 2^-8 is a bf16 tie that rounds to 1, twice
    assert F.moe_sum(y).tolist() == [[1.0]]
    y5 = np.array([[[one], [tiny], [tiny], [0.0], [0.0]]], np.float32)   # K = 5: f32 sum
    assert F.moe_sum(y5).tolist() == [[1.0078125]]


def _blocky(rng, N, Kd, bn, bk):
    """Normal weights with a random power-of-two gain per block, so that the
    block scales differ by up to 16x and a misplaced scale shows."""
    gain = 2.0 ** rng.uniform(-2, 2, (-(-N // bn), -(-Kd // bk)))
    return rng.standard_normal((N, Kd)) * 0.05 * np.kron(gain, np.ones((bn, bk)))[:N, :Kd]


def _fp8_experts(rng, E, H, I, bn=128, bk=128):
    w13c, s13, w2c, s2 = [], [], [], []
    for _ in range(E):
        a, b = F.quantize_weights(_blocky(rng, 2 * I, H, bn, bk), bn, bk)
        c, d = F.quantize_weights(_blocky(rng, H, I, bn, bk), bn, bk)
        w13c.append(a), s13.append(b), w2c.append(c), s2.append(d)
    return np.stack(w13c), np.stack(s13), np.stack(w2c), np.stack(s2)


@pytest.mark.parametrize("K", [1, 2, 8])
def test_moe_fp8_close_to_unquantised_oracle(K):
    rng = np.random.default_rng(4 + K)
    E, H, I, T = 10, 256, 256, 3
    w13c, s13, w2c, s2 = _fp8_experts(rng, E, H, I)
    x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to(torch.bfloat16)
    ids = np.stack([rng.permutation(E)[:K] for _ in range(T)])
    tw = rng.uniform(0.1, 1, (T, K)).astype(np.float32)
    got = F.moe_forward_fp8(x, tw, ids, w13c, w2c, s13, s2)
    w13d = torch.from_numpy(np.stack([F.dequantize(w13c[e], s13[e], 128, 128) for e in range(E)]))
    w2d = torch.from_numpy(np.stack([F.dequantize(w2c[e], s2[e], 128, 128) for e in range(E)]))
    ref = moe_forward(x, tw, ids, w13d, w2d).numpy()
    # activation quantisation dominates: e4m3 keeps 3 mantissa bits, a
    # relative rounding error of about 2^-3 / sqrt(12) = 3.6% rms per element
    rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    assert rel < 0.08, rel
    # an absent expert contributes nothing
    emap = np.zeros(E, np.int32)
    emap[ids[0, 0]] = -1
    got2 = F.moe_forward_fp8(x, tw, ids, w13c, w2c, s13, s2, expert_map=emap)
    tw2 = tw.copy()
    tw2[ids == ids[0, 0]] = 0.0
    ref2 = moe_forward(x, tw2, ids, w13d, w2d).numpy()
    assert np.linalg.norm(got2 - ref2) / np.linalg.norm(ref2) < 0.08


def test_moe_fp8_routing_weight_and_linearity_in_w2_scales():
    rng = np.random.default_rng(9)
    E, H, I, T, K = 4, 128, 128, 2, 2
    w13c, s13, w2c, s2 = _fp8_experts(rng, E, H, I)
    x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to(torch.bfloat16)
    ids = np.array([[0, 1], [2, 3]])
    tw = np.array([[0.5, 0.5], [0.25, 0.75]], np.float32)
    base = F.moe_forward_fp8(x, tw, ids, w13c, w2c, s13, s2)
    # doubling every w2 block scale doubles y exactly (bf16 rounding and the
    # bf16 adds commute with a power of two)
    assert np.array_equal(F.moe_forward_fp8(x, tw, ids, w13c, w2c, s13, s2 * 2), base * 2)
    assert np.array_equal(F.moe_forward_fp8(x, tw * 2, ids, w13c, w2c, s13, s2), base * 2)


def test_torch_cpu_baseline_close_to_oracle():
    """The torch CPU block-FP8 fused-MoE that bench.py times as the FP8
    line's CPU baseline computes the same function: within 1e-2 (relative
    L2) of the oracle on a Qwen3-FP8-shaped layer with 16 experts."""
    from oracle.moe import route
    from wisp_amd import workloads as W
    base = W.qwen3_decode(seed=2, steps=3, weights=False)
    base.logits = base.logits[:, :, :16].contiguous()
    wl = W.fp8_layer(base, experts=16)
    w13, w2, s13, s2 = wl.views()
    for t in range(3):
        tw, ids = route(wl.logits[t], 8)
        want = F.moe_forward_fp8(wl.x[t], tw.astype(np.float32), ids, w13, w2, s13, s2)
        got = F.moe_forward_fp8_fast(wl.x[t], tw, ids, w13, w2, s13, s2).float().numpy()
        assert np.linalg.norm(got - want) / np.linalg.norm(want) < 1e-2, t
