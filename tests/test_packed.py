"""Packed bf16 masters (``wisp_pack_bf16``): lossless, host-only packing.

The unpacker below is written from the format description in
``include/wisp_hip.h`` and ``wisp_amd/csrc/packed.h``, independently of the
library's device unpacker; every test checks that it gives back the exact
bits of the masters.  No GPU is used: packing runs on the host.
"""
import ctypes as C

import numpy as np
import pytest

from wisp_amd import _lib


def _a(v, m):
    return (v + m - 1) // m * m


def _unpack_rows(buf, off, rows, L, exc_off):
    nb, nw = L // 64, (L // 64 + 31) // 32
    hdr_bytes = _a(_a(nb, 4) + 4 * nw + 4, 16)
    rb = L + L // 2 + hdr_bytes
    out = np.empty((rows, L), np.uint16)
    for r in range(rows):
        row = buf[off + r * rb: off + (r + 1) * rb]
        lo = row[:L].astype(np.uint16)
        codes = row[L: L + L // 2]
        c = np.empty(L, np.uint16)
        c[0::2], c[1::2] = codes & 15, codes >> 4
        hdr = row[L + L // 2:]
        base = hdr[:nb].astype(np.uint16)
        mask = hdr[_a(nb, 4): _a(nb, 4) + 4 * nw].view("<u4")
        k = int(hdr[_a(nb, 4) + 4 * nw: _a(nb, 4) + 4 * nw + 4].view("<u4")[0])
        e = np.where(c == 15, 0, np.repeat(base, 64) + c).astype(np.uint16)
        for b in range(nb):
            if (int(mask[b >> 5]) >> (b & 31)) & 1:
                e[64 * b: 64 * b + 64] = buf[exc_off + 64 * k: exc_off + 64 * k + 64]
                k += 1
        out[r] = ((lo & 0x80) << 8) | (e << 7) | (lo & 0x7F)
    return out


def _unpack(packed, E, H, I, stride):
    rb13 = H + H // 2 + _a(_a(H // 64, 4) + 4 * ((H // 64 + 31) // 32) + 4, 16)
    rb2 = I + I // 2 + _a(_a(I // 64, 4) + 4 * ((I // 64 + 31) // 32) + 4, 16)
    w2_off = 2 * I * rb13
    exc_off = w2_off + H * rb2
    w13 = np.empty((E, 2 * I, H), np.uint16)
    w2 = np.empty((E, H, I), np.uint16)
    for e in range(E):
        buf = packed[e * stride: (e + 1) * stride]
        w13[e] = _unpack_rows(buf, 0, 2 * I, H, exc_off)
        w2[e] = _unpack_rows(buf, w2_off, H, I, exc_off)
    return w13, w2


def _pack(w13, w2):
    """w13 [E, 2I, H], w2 [E, H, I] as uint16 bf16 bits -> (packed, stride)."""
    E, two_i, H = w13.shape
    I = two_i // 2
    w13 = np.ascontiguousarray(w13)
    w2 = np.ascontiguousarray(w2)
    lib = _lib.lib()
    args = (E, H, I, w13.ctypes.data, two_i * H, w2.ctypes.data, H * I)
    stride = lib.wisp_pack_bf16_stride(*args)
    assert stride > 0 and stride % 256 == 0
    out = np.full(E * stride, 0xAB, np.uint8)
    _lib.check(lib.wisp_pack_bf16(*args, out.ctypes.data, stride), "wisp_pack_bf16")
    return out, stride


def _bf16_bits(x):
    u = np.asarray(x, np.float32).view(np.uint32)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)  # round to nearest even


def _weights(rng, E, H, I, std=0.02):
    return (_bf16_bits(rng.normal(0, std, (E, 2 * I, H))),
            _bf16_bits(rng.normal(0, std, (E, H, I))))


def test_round_trip_typical_weights():
    rng = np.random.default_rng(0)
    w13, w2 = _weights(rng, 3, 128, 64)
    packed, stride = _pack(w13, w2)
    g13, g2 = _unpack(packed, 3, 128, 64, stride)
    assert np.array_equal(g13, w13) and np.array_equal(g2, w2)


def test_round_trip_every_kind_of_block():
    """Zeros of both signs, subnormals, infinities and NaNs, all-zero blocks
    and blocks whose exponents span more than 15 values (the exception
    area), in w13 and w2 rows of several lengths (one and two mask words)."""
    rng = np.random.default_rng(1)
    E, H, I = 2, 2112, 128   # 33 blocks per w13 row: a second mask word
    w13, w2 = _weights(rng, E, H, I)
    w13[0, 0, :64] = 0                                   # all zero
    w13[0, 1, :64] = 0x8000                              # negative zeros
    w13[0, 2, 5] = 0x0001                                # subnormal in a normal block
    w13[0, 3, 64:128] = rng.integers(0, 0x80, 64) | (rng.integers(0, 2, 64) << 15)  # subnormals
    w13[1, 4, 7] = 0x7F80                                # +inf: exponent 255 -> exception
    w13[1, 5, 2047 - 64 * 2] = 0x7FC1                    # NaN
    w13[1, 6, 2100] = _bf16_bits(1e30)                   # wide span in block 32 (mask word 1)
    w13[1, 6, 2101] = _bf16_bits(1e-30)
    w2[0, 7, 10] = _bf16_bits(3e-38)                     # w2 row exception
    w2[1, :, :64] = _bf16_bits(rng.normal(0, 1, (H, 64)) * 10.0 ** rng.integers(-20, 20, (H, 64)))
    packed, stride = _pack(w13, w2)
    g13, g2 = _unpack(packed, E, H, I, stride)
    assert np.array_equal(g13, w13) and np.array_equal(g2, w2)
    # the exceptions made expert 1 larger than the fixed part
    rb13 = H + H // 2 + 48
    rb2 = I + I // 2 + 16
    assert stride > 2 * I * rb13 + H * rb2


def test_typical_weights_pack_to_under_0_78_of_their_bytes():
    rng = np.random.default_rng(2)
    H, I = 2048, 768   # the Qwen3-30B-A3B expert
    w13, w2 = _weights(rng, 1, H, I)
    packed, stride = _pack(w13, w2)
    assert stride / ((3 * H * I) * 2) < 0.78
    g13, g2 = _unpack(packed, 1, H, I, stride)
    assert np.array_equal(g13, w13) and np.array_equal(g2, w2)


@pytest.mark.parametrize("H,I", [(96, 64), (128, 32), (0, 64)])
def test_shapes_that_do_not_pack(H, I):
    w = np.zeros(max(1, 2 * I * max(H, 1) * 2), np.uint16)
    assert _lib.lib().wisp_pack_bf16_stride(1, H, I, w.ctypes.data, 2 * I * H,
                                            w.ctypes.data, H * I) == 0


def test_a_stride_below_the_masters_needs_is_refused():
    rng = np.random.default_rng(3)
    w13, w2 = _weights(rng, 1, 64, 64)
    w13[0, 0, 0], w13[0, 0, 1] = _bf16_bits(1e30), _bf16_bits(1e-30)  # one exception
    packed, stride = _pack(w13, w2)
    out = np.zeros(stride, np.uint8)
    rc = _lib.lib().wisp_pack_bf16(1, 64, 64, w13.ctypes.data, 2 * 64 * 64, w2.ctypes.data,
                                   64 * 64, out.ctypes.data, stride - 256)
    assert rc == _lib.WISP_ERR_INVALID
