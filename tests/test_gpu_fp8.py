"""GPU parity of the fp8 (OCP E4M3) kernels against the fp8 oracle.

c3h_quantize_fp8_rows must equal oracle.fp8_ref.quantize_rows bit for bit
(codes and scales) for fp32 / fp16 / bf16 inputs, ragged widths, strided rows,
zero rows, non-finite rows and exact round-to-nearest-even ties.
c3h_gemm_fp8: integer-valued E4M3 operands make every fp32 partial sum
exact, so the result must be bit-exact whatever order the MFMA sums in (this
pins the lane/K layout of both operands); general operands are compared with
the float64 oracle within |err| <= 2^-10 sum_k |a_k b_k| sa sb -- measured on
gfx950, v_mfma_f32_16x16x128_f8f6f4 adds each aligned group of 8 products
(k = 8j .. 8j+7) at 13 bits below the group's largest product (2^14 + 1 sums
to 2^14, 2^13 + 1 to 2^13 + 1), so a group loses less than 7 * 2^-13 of its
sum |ab| -- plus fp32 accumulation and 1e-6 relative for the scale / bias /
residual roundings; 16-bit outputs within one more rounding of that.  The
typical error is far smaller: the RMS error must stay below 2^-14 of the RMS
sum |ab| scale.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import fp8_ref as F
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


def _quantize_gpu(xd, code, rows, cols, ldx, ldo):
    from hackathon_amd import _lib
    from hackathon_amd.device import DeviceArray

    q = DeviceArray.empty((rows, ldo), np.uint8)
    s = DeviceArray.empty((rows,), np.float32)
    a = _lib.Fp8QuantArgs()
    a.x, a.out, a.scale, a.rows, a.cols, a.ldx, a.ldo, a.x_dtype = xd.ptr, q.ptr, s.ptr, rows, cols, ldx, ldo, code
    _lib.launch(a, None)
    return q.get()[:, :cols], s.get()


def _rows(rng, rows, cols):
    x = (rng.standard_normal((rows, cols)) * np.exp2(rng.integers(-6, 6, (rows, 1)))).astype(np.float32)
    if rows > 4:
        x[1] = 0.0                                   # zero row
        x[2, cols // 2] = np.inf                     # non-finite rows
        x[3, 0] = np.nan
        # exact ties: amax 448 (inverse scale 1), then midpoints between E4M3 neighbours
        grid = np.unique(np.abs(F.decode(np.arange(0x7F, dtype=np.uint8))))
        mids = ((grid[:-1].astype(np.float64) + grid[1:]) / 2).astype(np.float32)
        row = np.resize(np.concatenate([mids, -mids]), cols).astype(np.float32)
        row[0] = 448.0
        x[4] = row
    return x


@pytest.mark.parametrize("kind", ["fp32", "fp16", "bf16"])
@pytest.mark.parametrize("rows,cols,pad", [(1, 8, 0), (37, 96, 8), (300, 512, 0), (64, 2048, 16), (6, 4104, 0),
                                           (130, 4096, 0), (9, 8200, 8)])
def test_quantize_fp8_rows_bit_exact(gpu, kind, rows, cols, pad):
    rng = np.random.default_rng(rows * 7 + cols)
    x32 = _rows(rng, rows, cols)
    if kind == "fp16":
        x32 = np.where(np.isfinite(x32), np.clip(x32, -60000, 60000), x32)
    full = np.zeros((rows, cols + pad), np.float32)
    full[:, :cols] = x32
    xd, xval, code = _input(full, kind)
    print(f"quantize_fp8_rows {kind} rows={rows} cols={cols} ldx={cols + pad}", flush=True)
    q, s = _quantize_gpu(xd, code, rows, cols, cols + pad, cols + 8)
    rq, rs = F.quantize_rows(xval[:, :cols])
    np.testing.assert_array_equal(np.isnan(s), np.isnan(rs))
    np.testing.assert_array_equal(s[~np.isnan(s)], rs[~np.isnan(rs)])
    np.testing.assert_array_equal(q, rq)


def _gemm_gpu(qa, sa, qb, sb, out_kind, bias=None, act=0, residual=None, ldo=None):
    from hackathon_amd import _lib
    from hackathon_amd.c35 import engine as E
    from hackathon_amd.device import BF16, DeviceArray

    m, k = qa.shape
    n = qb.shape[0]
    ldo = ldo or n
    code, sdt = {"fp32": (_lib.F32, np.float32), "bf16": (_lib.BF16, BF16), "fp16": (_lib.F16, np.float16)}[out_kind]
    out = DeviceArray.empty((m, ldo), sdt)
    keep = [_dev(qa), _dev(qb), _dev(sa), _dev(sb)]
    g = _lib.Fp8GemmArgs()
    g.a, g.b, g.a_scale, g.b_scale, g.out = keep[0].ptr, keep[1].ptr, keep[2].ptr, keep[3].ptr, out.ptr
    g.m, g.n, g.k, g.lda, g.ldb, g.ldo, g.out_dtype = m, n, k, k, k, ldo, code
    bd = _dev(bias) if bias is not None else None
    g.epi = E.epilogue(bias=bd, bias_mode=2 if bias is not None else 0, act=act, residual=residual,
                       imm=[math.sqrt(2.0), 1.0, 0.5] if act == 2 else [])
    print(f"gemm_fp8 m={m} n={n} k={k} out={out_kind} act={act}", flush=True)
    _lib.launch(g, None)
    got = out.get()[:, :n]
    return got.astype(np.float32) if out_kind == "fp16" else (got if out_kind == "fp32" else _bf(got))


def _bf(a):
    from hackathon_amd.device import bf16_to_f32

    return bf16_to_f32(a)


@pytest.mark.parametrize("m,n,k", [(16, 16, 16), (64, 64, 128), (300, 200, 96), (1000, 64, 576), (130, 600, 528),
                                   (77, 90, 144), (520, 1030, 1024), (256, 64, 4096)])
def test_gemm_fp8_integer_operands_bit_exact(gpu, m, n, k):
    rng = np.random.default_rng(m + n + k)
    vals = np.arange(-8, 9, dtype=np.float32)          # exact in E4M3
    a = rng.choice(vals, (m, k)).astype(np.float32)
    b = rng.choice(vals, (n, k)).astype(np.float32)
    qa, qb = F.encode(a), F.encode(b)
    ones_m, ones_n = np.ones(m, np.float32), np.ones(n, np.float32)
    got = _gemm_gpu(qa, ones_m, qb, ones_n, "fp32")
    ref = F.gemm_fp8(qa, ones_m, qb, ones_n)          # |partial sums| <= 64 k < 2^24: exact in fp32
    np.testing.assert_array_equal(got, ref.astype(np.float32))


@pytest.mark.parametrize("m,n,k,out_kind,act", [(300, 200, 96, "fp32", 1), (1000, 64, 576, "fp16", 2),
                                                (130, 600, 528, "bf16", 0), (2048, 512, 2048, "fp16", 0),
                                                (512, 2048, 512, "fp16", 2), (77, 1000, 512, "fp32", 0)])
def test_gemm_fp8_epilogue_matches_oracle(gpu, m, n, k, out_kind, act):
    rng = np.random.default_rng(m * 3 + n + k)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = (rng.standard_normal((n, k)) * 0.05).astype(np.float32)
    qa, sa = F.quantize_rows(a)
    qb, sb = F.quantize_rows(b)
    bias = rng.standard_normal(n).astype(np.float32)
    res = None
    res_val = np.zeros((m, n), np.float32)
    if out_kind != "fp32":
        from hackathon_amd.device import BF16, f32_to_bf16

        r32 = rng.standard_normal((m, n)).astype(np.float32)
        if out_kind == "fp16":
            res, res_val = _dev(r32.astype(np.float16)), r32.astype(np.float16).astype(np.float32)
        else:
            res, res_val = _dev(f32_to_bf16(r32), BF16), G.round_bf16(r32)
    got = _gemm_gpu(qa, sa, qb, sb, out_kind, bias=bias, act=act, residual=res)
    da, db = F.decode(qa).astype(np.float64), F.decode(qb).astype(np.float64)
    v = F.gemm_fp8(qa, sa, qb, sb) + bias[None, :] + res_val
    # the instruction sums aligned groups of 8 products, truncating each to
    # 13 bits below the group's largest (< 7 * 2^-13 of the group's sum|ab|),
    # then accumulates in fp32
    bound = (np.abs(da) @ np.abs(db).T) * sa[:, None] * sb[None, :] * (2.0 ** -10 + (k / 128 + 8) * 2.0 ** -24)
    if act == 1:
        v = np.maximum(v, 0)
    elif act == 2:
        from scipy.special import erf

        v = v * (erf(v / math.sqrt(2.0)) + 1.0) * 0.5
        bound = bound * 1.2 + 1e-6
    err = np.abs(got.astype(np.float64) - v)
    s1 = (np.abs(da) @ np.abs(db).T) * sa[:, None] * sb[None, :]
    if out_kind == "fp32":
        assert np.sqrt(np.mean(err ** 2)) <= 2.0 ** -14 * np.sqrt(np.mean(s1 ** 2))
        assert np.all(err <= bound + 1e-6 * np.abs(v)), float((err - bound).max())
    else:
        ulp = 2.0 ** -10 if out_kind == "fp16" else 2.0 ** -7
        assert np.all(err <= bound + ulp * np.abs(v) + 1e-6), float((err - bound - ulp * np.abs(v)).max())


def test_gemm_fp8_host_checks(gpu):
    from hackathon_amd import _lib
    from hackathon_amd.device import DeviceArray

    a = DeviceArray.empty((32, 40), np.uint8)
    s = DeviceArray.empty((64,), np.float32)
    out = DeviceArray.empty((32, 32), np.float32)
    g = _lib.Fp8GemmArgs()
    g.a, g.b, g.a_scale, g.b_scale, g.out = a.ptr, a.ptr, s.ptr, s.ptr, out.ptr
    g.m, g.n, g.k, g.lda, g.ldb, g.ldo, g.out_dtype = 32, 32, 40, 40, 40, 32, _lib.F32
    with pytest.raises(_lib.C3HError, match="multiples of 16"):
        _lib.launch(g, None)
    g.k, g.lda, g.ldb = 32, 32, 32
    g.b_scale = s.ptr + 4
    with pytest.raises(_lib.C3HError, match="aligned"):
        _lib.launch(g, None)
    q = _lib.Fp8QuantArgs()
    q.x, q.out, q.scale, q.rows, q.cols, q.ldx, q.ldo, q.x_dtype = a.ptr, a.ptr, s.ptr, 4, 12, 16, 16, _lib.F16
    with pytest.raises(_lib.C3HError, match="multiples of 8"):
        _lib.launch(q, None)
