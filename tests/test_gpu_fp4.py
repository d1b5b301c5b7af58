"""GPU parity of the W4A16 kernels (MXFP4 weights, fp16 activations).

c3h_quantize_mxfp4 must equal oracle.fp4_ref.quantize_mxfp4 bit for bit
(codes and exponents) for fp32 / fp16 / bf16 rows, strided rows, exact
rounding ties, zero, tiny (clamped), huge (saturating) and non-finite blocks.

c3h_gemm_w4a16 widens the weights to fp16 in registers and runs the fp16
MFMA loop of c3h_gemm's register-prefetch kernel, so with that kernel
selected (C3H_DISABLE_DMA) c3h_gemm on the oracle's dequantized fp16 weights
must give the same bits; this pins the decode instruction's nibble order and
scale over all 16 codes and every exponent the quantizer emits.  Against the
float64 oracle the result is within fp32 accumulation error:
|err| <= (k/32 + 8) 2^-24 sum_k |a_k w_k| + one output rounding.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

import switches
from oracle import fp4_ref as F4
from oracle import graph_ref as G

pytestmark = pytest.mark.gpu


def _dev(x, dtype=None):
    from hackathon_amd.device import DeviceArray

    return DeviceArray.from_host(np.ascontiguousarray(x), dtype)


def _input(x32: np.ndarray, kind: str):
    """(device array of x in `kind`, its exact float32 value, dtype code)."""
    from hackathon_amd import _lib
    from hackathon_amd.device import BF16, f32_to_bf16

    if kind == "fp32":
        return _dev(x32), x32, _lib.F32
    if kind == "fp16":
        h = x32.astype(np.float16)
        return _dev(h), h.astype(np.float32), _lib.F16
    return _dev(f32_to_bf16(x32), BF16), G.round_bf16(x32), _lib.BF16


def _quantize_gpu(xd, code, rows, cols, ldx):
    from hackathon_amd import _lib
    from hackathon_amd.device import DeviceArray

    ldc = ((cols // 2 + 15) // 16) * 16
    lds = cols // 32 + 3
    q = DeviceArray.empty((rows, ldc), np.uint8)
    s = DeviceArray.empty((rows, lds), np.uint8)
    a = _lib.Mxfp4QuantArgs()
    a.x, a.codes, a.scales = xd.ptr, q.ptr, s.ptr
    a.rows, a.cols, a.ldx, a.ldc, a.lds, a.x_dtype = rows, cols, ldx, ldc, lds, code
    print(f"quantize_mxfp4 rows={rows} cols={cols} ldx={ldx} dtype={code}", flush=True)
    _lib.launch(a, None)
    return q.get()[:, :cols // 2], s.get()[:, :cols // 32]


def _weights(rng, rows, cols, special=True):
    x = (rng.standard_normal((rows, cols)) * np.exp2(rng.integers(-10, 8, (rows, 1)))).astype(np.float32)
    if special and rows >= 8 and cols >= 64:
        x[0, :32] = 0.0                                    # zero block
        x[1, :32] *= 1e-30                                 # tiny block: exponent clamped to -13
        x[1, 32:64] *= 1e30                                # huge block: clamped to 13, saturating
        x[2, 5] = np.nan                                   # non-finite blocks
        x[3, 40] = -np.inf
        # exact ties: amax 6 * 2^e, then every midpoint between E2M1 magnitudes
        mids = (F4.MAGNITUDES[:-1] + F4.MAGNITUDES[1:]) / 2
        for r, e in ((4, 0), (5, -3), (6, 5)):
            blk = np.resize(np.concatenate([mids, -mids, F4.MAGNITUDES, -F4.MAGNITUDES]), 32)
            blk[0] = 6.0
            x[r, :32] = (blk * 2.0 ** e).astype(np.float32)
        x[7, :32] = -0.0
    return x


@pytest.mark.parametrize("kind", ["fp32", "fp16", "bf16"])
@pytest.mark.parametrize("rows,cols,pad", [(1, 32, 0), (8, 64, 0), (37, 96, 8), (300, 512, 0), (64, 2048, 16),
                                           (130, 4096, 0)])
def test_quantize_mxfp4_bit_exact(gpu, kind, rows, cols, pad):
    rng = np.random.default_rng(rows * 7 + cols + pad)
    x = _weights(rng, rows, cols)                          # (fp16: the huge block becomes Inf)
    xp = np.zeros((rows, cols + pad), np.float32)
    xp[:, :cols] = x
    xd, xv, code = _input(xp, kind)
    q, s = _quantize_gpu(xd, code, rows, cols, cols + pad)
    wq, ws = F4.quantize_mxfp4(xv[:, :cols])
    np.testing.assert_array_equal(s, ws)
    np.testing.assert_array_equal(q, wq)


def _w4_gpu(a16, codes, scales, n, k, out_kind="fp32", bias=None, act=0, residual=None, lda=None):
    from hackathon_amd import _lib
    from hackathon_amd.c35 import engine as E
    from hackathon_amd.device import DeviceArray

    m = a16.shape[0]
    lda = lda or a16.shape[1]
    code, sdt = {"fp32": (_lib.F32, np.float32), "fp16": (_lib.F16, np.float16)}[out_kind]
    out = DeviceArray.empty((m, n), sdt)
    ad, cd, sd = _dev(a16), _dev(codes), _dev(scales)
    bd = _dev(bias) if bias is not None else None
    g = _lib.W4A16GemmArgs()
    g.a, g.b_codes, g.b_scales, g.out = ad.ptr, cd.ptr, sd.ptr, out.ptr
    g.m, g.n, g.k, g.lda, g.ldb, g.ldbs, g.ldo, g.out_dtype = m, n, k, lda, codes.shape[1], scales.shape[1], n, code
    g.epi = E.epilogue(bias=bd, bias_mode=2 if bias is not None else 0, act=act, residual=residual,
                       imm=[math.sqrt(2.0), 1.0, 0.5] if act == 2 else [])
    print(f"gemm_w4a16 m={m} n={n} k={k} out={out_kind} act={act}", flush=True)
    _lib.launch(g, None)
    return out.get()


def _f16_gpu(a16, w16, out_kind="fp32", bias=None, act=0, residual=None, lda=None):
    from hackathon_amd import _lib
    from hackathon_amd.c35 import engine as E
    from hackathon_amd.device import DeviceArray

    m, n, k = a16.shape[0], w16.shape[0], w16.shape[1]
    lda = lda or a16.shape[1]
    code, sdt = {"fp32": (_lib.F32, np.float32), "fp16": (_lib.F16, np.float16)}[out_kind]
    out = DeviceArray.empty((m, n), sdt)
    ad, wd = _dev(a16), _dev(w16)
    bd = _dev(bias) if bias is not None else None
    g = _lib.GemmArgs()
    g.a, g.b, g.out = ad.ptr, wd.ptr, out.ptr
    g.m, g.n, g.k, g.lda, g.ldb, g.ldo, g.batch = m, n, k, lda, k, n, 1
    g.trans_a, g.trans_b, g.in_dtype, g.out_dtype = 0, 1, _lib.F16, code
    g.epi = E.epilogue(bias=bd, bias_mode=2 if bias is not None else 0, act=act, residual=residual,
                       imm=[math.sqrt(2.0), 1.0, 0.5] if act == 2 else [])
    print(f"gemm fp16 m={m} n={n} k={k} out={out_kind} act={act}", flush=True)
    _lib.launch(g, None)
    return out.get()


@pytest.mark.parametrize("m,n,k,out_kind,act", [(64, 64, 32, "fp32", 0), (300, 200, 96, "fp32", 1),
                                                (1000, 64, 320, "fp16", 2), (256, 128, 128, "fp16", 0),
                                                (2048, 2048, 512, "fp16", 2), (4096, 512, 2048, "fp32", 0),
                                                (1024, 8192, 512, "fp32", 0), (130, 600, 544, "fp16", 1)])
def test_gemm_w4a16_equals_fp16_gemm_on_dequantized_weights(gpu, m, n, k, out_kind, act):
    rng = np.random.default_rng(m + 3 * n + k)
    a = rng.standard_normal((m, k)).astype(np.float32)
    w = _weights(rng, n, k, special=False) * 0.05
    codes, scales = F4.quantize_mxfp4(w)
    # every code and every exponent the quantizer emits, in the first rows
    rows = min(n, 27)
    codes[:rows] = rng.integers(0, 256, (rows, k // 2)).astype(np.uint8)
    scales[:rows] = (np.arange(rows)[:, None] % 27 - 13 + 127).astype(np.uint8)
    w16 = F4.dequantize_mxfp4(codes, scales).astype(np.float16)
    np.testing.assert_array_equal(w16.astype(np.float32), F4.dequantize_mxfp4(codes, scales))
    a16 = a.astype(np.float16)
    bias = rng.standard_normal(n).astype(np.float32) if act else None
    res = None
    if out_kind == "fp16":
        res = _dev(rng.standard_normal((m, n)).astype(np.float16))
    got = _w4_gpu(a16, codes, scales, n, k, out_kind, bias, act, res)
    want = switches.with_switch("C3H_DISABLE_DMA", "1", lambda: _f16_gpu(a16, w16, out_kind, bias, act, res))
    np.testing.assert_array_equal(got.view(np.uint8), want.view(np.uint8))
    if out_kind == "fp32" and act == 0:
        ref = F4.gemm_w4a16(a, codes, scales)
        s1 = np.abs(a16.astype(np.float64)) @ np.abs(w16.astype(np.float64)).T
        err = np.abs(got.astype(np.float64) - ref)
        assert np.all(err <= (k / 32 + 8) * 2.0 ** -24 * s1 + 1e-30), float((err / (s1 + 1e-30)).max())


def test_gemm_w4a16_nan_block_poisons_its_column(gpu):
    m, n, k = 128, 128, 64
    rng = np.random.default_rng(11)
    a = rng.standard_normal((m, k)).astype(np.float16)
    w = (rng.standard_normal((n, k)) * 0.1).astype(np.float32)
    w[17, 40] = np.nan
    codes, scales = F4.quantize_mxfp4(w)
    assert scales[17, 1] == 0xFF
    got = _w4_gpu(a, codes, scales, n, k)
    assert np.isnan(got[:, 17]).all()
    assert np.isfinite(np.delete(got, 17, axis=1)).all()


def test_gemm_w4a16_host_checks(gpu):
    from hackathon_amd import _lib
    from hackathon_amd.device import DeviceArray

    a = DeviceArray.empty((32, 64), np.float16)
    c = DeviceArray.empty((32, 32), np.uint8)
    s = DeviceArray.empty((32, 2), np.uint8)
    out = DeviceArray.empty((32, 32), np.float32)
    g = _lib.W4A16GemmArgs()
    g.a, g.b_codes, g.b_scales, g.out = a.ptr, c.ptr, s.ptr, out.ptr
    g.m, g.n, g.k, g.lda, g.ldb, g.ldbs, g.ldo, g.out_dtype = 32, 32, 48, 64, 32, 2, 32, _lib.F32
    with pytest.raises(_lib.C3HError, match="multiple of 32"):
        _lib.launch(g, None)
    g.k, g.ldb = 64, 16
    with pytest.raises(_lib.C3HError, match="ldb"):
        _lib.launch(g, None)
    g.ldb, g.out_dtype = 32, _lib.BF16
    with pytest.raises(_lib.C3HError, match="fp32 or fp16"):
        _lib.launch(g, None)
    q = _lib.Mxfp4QuantArgs()
    q.x, q.codes, q.scales, q.rows, q.cols, q.ldx, q.ldc, q.lds, q.x_dtype = a.ptr, c.ptr, s.ptr, 32, 48, 64, 32, 2, _lib.F16
    with pytest.raises(_lib.C3HError, match="multiple of 32"):
        _lib.launch(q, None)
