"""GPU checks of the GEMM epilogue's row_max side output + c3h_argmax_finish.

A GEMM with row_max writes, for every output row and 64-column block, the
largest stored value (NaN ignored) and whether the block may hold a NaN;
c3h_argmax_finish completes each row's ArgMax from those and the few blocks
that can hold the answer.  The result must equal c3h_argmax over the stored output
(and NumPy's argmax of it, the same first-index / NaN-is-maximum rule) bit for
bit, for the 16-bit and int8 (modes 2 / 3) GEMMs on their kernel variants, on
ragged edge tiles, on planted ties across blocks and lanes, on NaN and all
-inf rows; the stored output must not change.  The E4M3 and W4A16 GEMMs run
the same register epilogue; the full-size programs (test_gpu_fullsize)
check every ArgMax output against their own logits.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

import switches

pytestmark = pytest.mark.gpu


def _dev(x, dtype=None):
    from hackathon_amd.device import DeviceArray

    return DeviceArray.from_host(np.ascontiguousarray(x), dtype)


def _out16(x, kind):
    from hackathon_amd.device import BF16, f32_to_bf16

    if kind == "bf16":
        return f32_to_bf16(x), BF16
    return np.asarray(x, np.float32).astype(np.float16), np.float16


def _as_f32(host, kind):
    from hackathon_amd.device import bf16_to_f32

    if kind == "fp32":
        return host
    if kind == "bf16":
        return bf16_to_f32(host.view(np.uint16))
    return host.astype(np.float32)


def _residual(rng, m, n, kind):
    """A residual that plants exact ties, NaN and all -inf rows in the output
    (the GEMM values are small, the planted ones dominate)."""
    r = rng.standard_normal((m, n)).astype(np.float32) * 0.01
    # large enough that the GEMM's own value vanishes in the rounding: exact ties
    big = 2.0 ** 15 if kind == "fp16" else 2.0 ** 30
    r[1, [0, 70, 200 % n]] = big                      # tie across blocks: first column wins
    r[2, [5, 6, 7, 4]] = big                          # tie inside a lane's 4 columns / across lanes
    r[3, n - 1] = big                                 # last column
    r[4, [n // 2, 3]] = np.nan                        # NaN beats everything, first NaN
    r[5, :] = -np.inf                                 # all -inf: column 0
    r[6, [n - 2, 17]] = [np.inf, np.inf]              # +inf tie (blocks flagged, no NaN)
    r[7, [20, 130 % n]] = [np.inf, np.nan]            # an infinity before a NaN: the NaN
    r[8, [0, n - 3]] = [big, np.nan]                  # a NaN in the last block wins over an earlier max
    r[m - 1, 9] = big                                 # last row (edge tile)
    if kind == "fp32":
        return r, r
    h, _ = _out16(r, kind)
    return h, None


def _argmax_finish(parts, outd, m, n, code):
    from hackathon_amd import _lib
    from hackathon_amd.device import DeviceArray

    out = DeviceArray.empty((m,), np.int64)
    a = _lib.ArgmaxFinishArgs()
    a.parts, a.in_, a.out = parts.ptr, outd.ptr, out.ptr
    a.rows, a.cols, a.n_parts, a.ld, a.in_ld, a.in_dtype = m, n, -(-n // 64), parts.shape[1], n, code
    _lib.launch(a, None)
    return out.get()


def _argmax_dev(outd, m, n, code):
    from hackathon_amd import _lib
    from hackathon_amd.device import DeviceArray

    got = DeviceArray.empty((m,), np.int64)
    a = _lib.ArgmaxArgs()
    a.in_, a.out, a.rows, a.cols, a.in_dtype = outd.ptr, got.ptr, m, n, code
    _lib.launch(a, None)
    return got.get()


def _check(run, m, n, out_kind):
    """run(row_max_ptr, ld) launches the GEMM (None: without the side output)
    and returns the output device array."""
    from hackathon_amd import _lib
    from hackathon_amd.device import DeviceArray

    code = {"fp32": _lib.F32, "bf16": _lib.BF16, "fp16": _lib.F16}[out_kind]
    plain = run(None, 0).get().copy()
    ld = -(-n // 64) + 3
    parts = DeviceArray.empty((m, ld), np.int64)
    parts.copy_from_host(np.full((m, ld), -1, np.int64))
    outd = run(parts.ptr, ld)
    stored = outd.get()
    np.testing.assert_array_equal(stored.view(np.uint8), plain.view(np.uint8))   # the output is unchanged
    got = _argmax_finish(parts, outd, m, n, code)
    want = _argmax_dev(outd, m, n, code)
    np.testing.assert_array_equal(got, want)
    vals = _as_f32(stored, out_kind).reshape(m, n)
    np.testing.assert_array_equal(got, np.argmax(vals, axis=-1))
    return got, vals


@pytest.mark.parametrize("kind,m,n,k,out_kind,act,bigtile", [
    ("bf16", 4096, 4096, 192, "fp32", 0, True),
    ("bf16", 4096, 4096, 192, "bf16", 1, False),
    ("fp16", 1000, 1000, 320, "fp32", 0, False),     # ragged M and N (N % 64 != 0)
    ("fp16", 300, 260, 64, "fp16", 0, False),
    ("fp16", 8192, 8192, 512, "fp32", 0, True),      # the decoder fp16 LM head shape class
    # the fp16 decoder's QKV shape: the 256 x 192 tile (tile192_wins), whose
    # wave tiles keep three 64-column block maxima per lane (TN = 12)
    ("fp16", 16384, 1536, 512, "fp16", 0, True),
    # wide rows: 192, 625 and 1094 block maxima per row (the finish kernel
    # keeps up to 4, 16 block maxima per lane in registers, else re-reads)
    ("fp16", 64, 12288, 64, "fp32", 0, True),
    ("bf16", 64, 40000, 64, "bf16", 0, True),
    ("fp16", 32, 70000, 64, "fp32", 0, True),
])
def test_gemm16_row_max(gpu, kind, m, n, k, out_kind, act, bigtile):
    from hackathon_amd import _lib
    from hackathon_amd.c35 import engine as E
    from hackathon_amd.device import BF16, DeviceArray, f32_to_bf16

    rng = np.random.default_rng(m + n + k)
    in_code = _lib.BF16 if kind == "bf16" else _lib.F16
    a32 = rng.standard_normal((m, k)).astype(np.float32)
    b32 = (rng.standard_normal((n, k)) * 0.1).astype(np.float32)
    conv = (lambda x: f32_to_bf16(x)) if kind == "bf16" else (lambda x: x.astype(np.float16))
    ad, bd = _dev(conv(a32), BF16 if kind == "bf16" else None), _dev(conv(b32), BF16 if kind == "bf16" else None)
    bias = _dev(rng.standard_normal(n).astype(np.float32) * 0.01)
    res_host, _ = _residual(rng, m, n, out_kind)
    rd = _dev(res_host, BF16 if out_kind == "bf16" else None)
    sdt = {"fp32": np.float32, "bf16": BF16, "fp16": np.float16}[out_kind]
    out = DeviceArray.empty((m, n), sdt)

    def run(rb, ld):
        g = _lib.GemmArgs()
        g.a, g.b, g.out = ad.ptr, bd.ptr, out.ptr
        g.m, g.n, g.k, g.lda, g.ldb, g.ldo, g.batch = m, n, k, k, k, n, 1
        g.trans_a, g.trans_b, g.in_dtype = 0, 1, in_code
        g.out_dtype = {"fp32": _lib.F32, "bf16": _lib.BF16, "fp16": _lib.F16}[out_kind]
        g.epi = E.epilogue(bias=bias, bias_mode=2, act=act, residual=rd)
        g.epi.row_max, g.epi.row_max_ld = rb, ld
        print(f"gemm16 row_max m={m} n={n} k={k} {kind}->{out_kind} act={act} big={bigtile} rb={bool(rb)}",
              flush=True)
        _lib.launch(g, None)
        return out

    fn = (lambda: _check(run, m, n, out_kind)) if bigtile else \
        (lambda: switches.with_switch("C3H_DISABLE_BIGTILE", "1", lambda: _check(run, m, n, out_kind)))
    got, vals = fn()
    if act == 0:  # (ReLU turns the NaN row into zeros)
        assert got[5] == 0 and got[1] == 0 and got[2] == 4 and got[3] == n - 1 and got[4] == 3 and got[6] == 17
        assert got[7] == 130 % n and got[8] == n - 3 and got[m - 1] == 9


@pytest.mark.parametrize("m,n,k,mode,out_kind,switch", [
    (4096, 32000, 768, 3, "fp32", None),             # the W8A8 LM head (a quarter of its rows)
    (16384, 768, 3072, 3, "bf16", None),             # W8A8 FFN2 shape: the 256 x 192 tile (TN = 12)
    (300, 1000, 256, 3, "fp32", "C3H_DISABLE_BIGTILE"),
    (1000, 264, 128, 2, "bf16", "C3H_DISABLE_DMA"),  # register-prefetch kernel, ragged
])
def test_qgemm_row_max(gpu, m, n, k, mode, out_kind, switch):
    from hackathon_amd import _lib
    from hackathon_amd.c35 import engine as E
    from hackathon_amd.device import BF16, DeviceArray

    rng = np.random.default_rng(m + n + k + mode)
    ad = _dev(rng.integers(-128, 128, size=(m, k), dtype=np.int8))
    bd = _dev(rng.integers(-127, 128, size=(n, k), dtype=np.int8))
    sbd = _dev((rng.random(n) * 0.001 + 0.0001).astype(np.float32))
    res_host, _ = _residual(rng, m, n, out_kind)
    rd = _dev(res_host, BF16 if out_kind == "bf16" else None)
    sdt = {"fp32": np.float32, "bf16": BF16}[out_kind]
    out = DeviceArray.empty((m, n), sdt)

    def run(rb, ld):
        g = _lib.QGemmArgs()
        g.a, g.b, g.out, g.m, g.n, g.k, g.lda, g.ldb, g.ldo = ad.ptr, bd.ptr, out.ptr, m, n, k, k, k, n
        g.a_scale, g.y_scale, g.b_scale, g.mode = 0.02, 0.05, sbd.ptr, mode
        g.out_dtype = {"fp32": _lib.F32, "bf16": _lib.BF16}[out_kind]
        g.epi = E.epilogue(residual=rd)
        g.epi.row_max, g.epi.row_max_ld = rb, ld
        print(f"qgemm row_max m={m} n={n} k={k} mode={mode} {out_kind} switch={switch} rb={bool(rb)}", flush=True)
        _lib.launch(g, None)
        return out

    fn = lambda: _check(run, m, n, out_kind)  # noqa: E731
    got, vals = switches.with_switch(switch, "1", fn) if switch else fn()
    assert got[5] == 0 and got[1] == 0 and got[2] == 4 and got[3] == n - 1 and got[4] == 3 and got[6] == 17
    assert got[7] == 130 % n and got[8] == n - 3


def test_row_max_host_checks(gpu):
    from hackathon_amd import _lib
    from hackathon_amd.c35 import engine as E
    from hackathon_amd.device import DeviceArray

    a = DeviceArray.empty((64, 64), np.float16)
    out = DeviceArray.empty((64, 64), np.float32)
    parts = DeviceArray.empty((64, 1), np.int64)
    g = _lib.GemmArgs()
    g.a, g.b, g.out = a.ptr, a.ptr, out.ptr
    g.m, g.n, g.k, g.lda, g.ldb, g.ldo, g.batch = 64, 64, 64, 64, 64, 64, 1
    g.trans_a, g.trans_b, g.in_dtype, g.out_dtype = 0, 1, _lib.F16, _lib.F32
    g.epi = E.epilogue(act=2, imm=[math.sqrt(2.0), 1.0, 0.5])
    g.epi.row_max, g.epi.row_max_ld = parts.ptr, 1
    with pytest.raises(_lib.C3HError, match="act <= 1"):
        _lib.launch(g, None)
    g.epi = E.epilogue()
    g.epi.row_max, g.epi.row_max_ld = parts.ptr, 0
    with pytest.raises(_lib.C3HError, match="row_max_ld"):
        _lib.launch(g, None)
    g.epi.row_max_ld, g.batch = 1, 2
    with pytest.raises(_lib.C3HError, match="batch 1"):
        _lib.launch(g, None)
    g.batch, g.in_dtype = 1, _lib.F32
    with pytest.raises(_lib.C3HError, match="row_max is taken only"):
        _lib.launch(g, None)
