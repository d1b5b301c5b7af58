"""Pins of the MXFP4 / W4A16 oracle (oracle/fp4_ref.py) on the CPU.

The element table is checked against the OCP MX v1.0 E2M1 values; the
encoder against every magnitude, every midpoint (ties to the even code),
saturation and the half-spacing error bound; the block quantizer against the
format's invariants; the GEMM against a float64 matmul of integer operands.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import fp4_ref as F4


def test_decode_matches_mx_table():
    # OCP MX v1.0, FP4 E2M1: S.EE.M with bias 1: 0, 0.5 (subnormal), 1, 1.5, 2, 3, 4, 6
    table = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]
    got = F4.decode(np.arange(16))
    np.testing.assert_array_equal(got[:8], np.array(table, np.float32))
    np.testing.assert_array_equal(got[8:], -np.array(table, np.float32))
    # from the bit fields: normal (E > 0): 2^(E-1) (1 + M/2); subnormal: M/2
    for c in range(8):
        e, m = c >> 1, c & 1
        assert got[c] == (2.0 ** (e - 1) * (1 + m / 2) if e else m / 2)


def test_encode_every_magnitude_and_midpoint():
    mags = F4.MAGNITUDES
    np.testing.assert_array_equal(F4.encode(mags), np.arange(8))
    mids = (mags[:-1] + mags[1:]) / 2                    # 0.25 0.75 1.25 1.75 2.5 3.5 5
    want_mid = [0, 2, 2, 4, 4, 6, 6]                     # the even code of each pair
    np.testing.assert_array_equal(F4.encode(mids), want_mid)
    eps = 1e-6
    np.testing.assert_array_equal(F4.encode(mids - eps), np.arange(7))
    np.testing.assert_array_equal(F4.encode(mids + eps), np.arange(1, 8))
    np.testing.assert_array_equal(F4.encode([6.0, 6.5, 7.99, 1e30]), [7, 7, 7, 7])


def test_encode_error_bound_dense_sweep():
    m = np.linspace(0.0, 6.0, 200_001)
    got = F4.decode(F4.encode(m)).astype(np.float64)
    # nearest magnitude: the error is at most half the spacing around m
    idx = np.clip(np.searchsorted(F4.MAGNITUDES, m), 1, 7)
    half = (F4.MAGNITUDES[idx] - F4.MAGNITUDES[idx - 1]) / 2
    assert np.all(np.abs(got - m) <= half + 1e-12)
    assert np.all(np.diff(F4.encode(m).astype(int)) >= 0)  # monotone


def test_block_exponent_rule():
    assert F4.block_exponent(np.array([6.0]))[0] == 0          # floor(log2 6) - 2
    assert F4.block_exponent(np.array([4.0]))[0] == 0
    assert F4.block_exponent(np.array([3.99]))[0] == -1
    assert F4.block_exponent(np.array([0.02]))[0] == -8        # log2 0.02 = -5.64
    assert F4.block_exponent(np.array([0.0]))[0] == -13
    assert F4.block_exponent(np.array([1e-30]))[0] == -13      # clamped up
    assert F4.block_exponent(np.array([1e30]))[0] == 13        # clamped down
    assert F4.block_exponent(np.array([2.0 ** -130]))[0] == -13  # subnormal amax


def test_quantize_invariants():
    rng = np.random.default_rng(7)
    x = (rng.standard_normal((64, 256)) * np.exp2(rng.integers(-12, 12, (64, 1)))).astype(np.float32)
    codes, scales = F4.quantize_mxfp4(x)
    assert codes.shape == (64, 128) and scales.shape == (64, 8)
    e = scales.astype(int) - 127
    assert e.min() >= -13 and e.max() <= 13
    xb = np.abs(x.reshape(64, 8, 32)).max(axis=-1)
    unclamped = (e > -13) & (e < 13)
    r = xb / np.exp2(e)
    assert np.all((r[unclamped] >= 4.0) & (r[unclamped] < 8.0))
    deq = F4.dequantize_mxfp4(codes, scales)
    # every dequantized weight is exactly an fp16 value
    np.testing.assert_array_equal(deq.astype(np.float16).astype(np.float32), deq)
    # error: at most half a code step, or the saturation at 6 * 2^e
    step = np.repeat(np.exp2(e), 32, axis=1).astype(np.float64)
    err = np.abs(deq.astype(np.float64) - x)
    assert np.all((err <= step + 1e-30) | (np.abs(x) > 6 * step))
    # codes of -0 / tiny negatives are +0
    z = np.zeros((1, 32), np.float32)
    z[0, 0] = -0.0
    z[0, 1] = -1e-9
    z[0, 2] = 1.0
    c, s = F4.quantize_mxfp4(z)
    assert F4.unpack(c)[0, 0] == 0 and F4.unpack(c)[0, 1] == 0


def test_quantize_round_trip_of_representable_blocks():
    rng = np.random.default_rng(3)
    mags = F4.MAGNITUDES
    codes = rng.integers(0, 16, (8, 64))
    codes[:, 0] = 7                                       # amax 6 in each block: e = 0 before scaling
    codes[:, 32] = 7
    e = rng.integers(-13, 14, (8, 2))
    vals = F4.decode(codes).astype(np.float64) * np.repeat(np.exp2(e), 32, axis=1)
    q, s = F4.quantize_mxfp4(vals.astype(np.float32))
    np.testing.assert_array_equal(s.astype(int) - 127, e)
    want = np.where(codes % 8 == 0, 0, codes)             # -0 codes become +0
    np.testing.assert_array_equal(F4.unpack(q), want)
    np.testing.assert_array_equal(F4.dequantize_mxfp4(q, s), vals.astype(np.float32))
    assert mags[7] == 6.0


def test_quantize_nonfinite_blocks():
    x = np.ones((2, 64), np.float32)
    x[0, 5] = np.nan
    x[1, 40] = np.inf
    q, s = F4.quantize_mxfp4(x)
    assert s[0, 0] == 0xFF and s[0, 1] != 0xFF and s[1, 1] == 0xFF and s[1, 0] != 0xFF
    assert not F4.unpack(q)[0, :32].any() and not F4.unpack(q)[1, 32:].any()
    d = F4.dequantize_mxfp4(q, s)
    assert np.isnan(d[0, :32]).all() and np.isfinite(d[0, 32:]).all()


@pytest.mark.parametrize("m,n,k", [(5, 7, 32), (33, 17, 96)])
def test_gemm_w4a16_integer_operands(m, n, k):
    rng = np.random.default_rng(m * n)
    a = rng.integers(-8, 9, (m, k)).astype(np.float32)
    codes = rng.integers(0, 16, (n, k))
    codes[:, ::32] = 7
    packed = (codes[:, 0::2] | (codes[:, 1::2] << 4)).astype(np.uint8)
    scales = np.full((n, k // 32), 127, np.uint8)          # 2^0
    got = F4.gemm_w4a16(a, packed, scales)
    np.testing.assert_array_equal(got, a.astype(np.float64) @ F4.decode(codes).astype(np.float64).T)
