"""Pins of the fp8 (OCP E4M3) oracle, CPU only.

`decode` and `encode` are checked against PyTorch's float8_e4m3fn dtype (a
library routine that implements the same OCP format), on every code and on a
dense sweep of |x| <= 448; `encode` further against the closed-form facts of
the format (every code's value encodes to that code; a midpoint between two
neighbouring codes goes to the one with an even mantissa; saturation at 448).
The row quantizer and the GEMM oracle are checked through invariants and a
case that reduces to a plain matmul (inputs already on the E4M3 grid).
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import fp8_ref as F


def _torch():
    return pytest.importorskip("torch")


def test_decode_all_codes_match_torch():
    torch = _torch()
    codes = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    got = F.decode(codes)
    assert np.array_equal(np.isnan(ref), np.isnan(got))
    assert np.array_equal(ref[~np.isnan(ref)], got[~np.isnan(got)])
    # closed form: max 448, smallest subnormal 2^-9, smallest normal 2^-6, 0x7F NaN
    assert got[0x7E] == 448.0 and got[0x01] == 2.0 ** -9 and got[0x08] == 2.0 ** -6
    assert np.isnan(got[0x7F]) and np.isnan(got[0xFF]) and got[0x80] == 0.0 and np.signbit(got[0x80])


def test_encode_matches_torch_on_dense_sweep():
    torch = _torch()
    rng = np.random.default_rng(0)
    x = np.concatenate([
        np.linspace(-448, 448, 400_001, dtype=np.float32),
        (rng.standard_normal(300_000) * np.exp2(rng.integers(-16, 9, 300_000))).astype(np.float32),
    ])
    x = np.clip(x, -448, 448)
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(F.encode(x), ref)


def test_encode_closed_form_grid_midpoints_and_saturation():
    codes = np.array([c for c in range(256) if (c & 0x7F) != 0x7F], np.uint8)
    vals = F.decode(codes)
    # every finite code round-trips (+0 / -0 keep their sign bit)
    assert np.array_equal(F.encode(vals), codes)
    pos = np.sort(np.unique(vals[vals >= 0]))
    lo, hi = pos[:-1], pos[1:]
    mid = ((lo.astype(np.float64) + hi) / 2).astype(np.float32)
    assert np.array_equal(mid.astype(np.float64), (lo.astype(np.float64) + hi) / 2)  # midpoints exact in fp32
    enc = F.encode(mid)
    lo_c, hi_c = F.encode(lo), F.encode(hi)
    even = np.where((lo_c & 1) == 0, lo_c, hi_c)
    assert np.array_equal(enc, even)
    # just off the midpoint: nearest
    assert np.array_equal(F.encode(np.nextafter(mid, np.float32(0))), lo_c)
    assert np.array_equal(F.encode(np.nextafter(mid, np.float32(np.inf))), hi_c)
    # saturation and NaN
    assert list(F.encode(np.array([448.0, 460.0, 1e30, -1e30, np.inf, np.nan], np.float32))) == \
        [0x7E, 0x7E, 0x7E, 0xFE, 0x7E, 0x7F]


def test_quantize_rows_invariants():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal((64, 96)) * np.exp2(rng.integers(-8, 8, (64, 1)))).astype(np.float32)
    x[3] = 0.0
    x[5, 7] = np.inf
    x[6, 0] = np.nan
    q, s = F.quantize_rows(x)
    assert q.shape == x.shape and q.dtype == np.uint8 and s.dtype == np.float32
    assert s[3] == 0.0 and not q[3].any()
    assert np.isnan(s[5]) and np.isnan(s[6]) and (q[5] == 0x7F).all() and (q[6] == 0x7F).all()
    ok = np.array([r not in (3, 5, 6) for r in range(64)])
    amax = np.abs(x[ok]).max(axis=1)
    np.testing.assert_allclose(s[ok] * 448.0, amax, rtol=2 ** -23)
    # the largest element of each row lands on +-448 (code 0x7E / 0xFE)
    arg = np.abs(x[ok]).argmax(axis=1)
    assert np.all((q[ok][np.arange(ok.sum()), arg] & 0x7F) == 0x7E)
    # |x - dequant| <= half a code step: 2^-4 relative for normals, 2^-10 * scale below 2^-6 * scale
    deq = F.dequantize_rows(q[ok], s[ok]).astype(np.float64)
    xs = x[ok].astype(np.float64)
    bound = np.maximum(np.abs(xs) * 2.0 ** -4, s[ok][:, None] * 2.0 ** -10) * (1 + 1e-6)
    assert np.all(np.abs(deq - xs) <= bound)


def test_gemm_fp8_on_grid_inputs_is_plain_matmul():
    rng = np.random.default_rng(2)
    grid = F.decode(np.array([c for c in range(256) if (c & 0x7F) not in (0x7F,)], np.uint8))
    a = rng.choice(grid, (24, 160)).astype(np.float32)
    b = rng.choice(grid, (40, 160)).astype(np.float32)
    a[:, 0], b[:, 0] = 448.0, -448.0          # amax 448 per row: scale 1, inverse scale 1
    qa, sa = F.quantize_rows(a)
    qb, sb = F.quantize_rows(b)
    assert (sa == 1.0).all() and (sb == 1.0).all()
    assert np.array_equal(F.decode(qa), a) and np.array_equal(F.decode(qb), b)
    ref = a.astype(np.float64) @ b.astype(np.float64).T
    assert np.array_equal(F.gemm_fp8(qa, sa, qb, sb), ref)
    # scales enter once per row / column
    got = F.gemm_fp8(qa, sa * 2, qb, sb * np.float32(0.5) * np.arange(1, 41, dtype=np.float32))
    np.testing.assert_allclose(got, ref * np.arange(1, 41)[None, :], rtol=1e-12)


def test_matmul_fp8_policy_close_to_fp32():
    rng = np.random.default_rng(3)
    a = rng.standard_normal((32, 256)).astype(np.float32)
    w = rng.standard_normal((256, 48)).astype(np.float32) * 0.05
    got = F.matmul_fp8_policy(a, w)
    ref = a @ w
    # E4M3 keeps 3 mantissa bits: relative error of a K=256 dot product of
    # random-sign terms is a few percent of its typical magnitude
    assert np.abs(got - ref).max() <= 0.08 * np.abs(ref).max()
    assert np.corrcoef(got.ravel(), ref.ravel())[0, 1] > 0.998
