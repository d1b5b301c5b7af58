"""c3h_gemm_splitk_noalloc: the split-K GEMM over the library's static device
scratch instead of a workspace, checked through the C-ABI against
c3h_gemm_splitk (the same kernels over a caller workspace).  Two calls in a
row, the second smaller (the array keeps the first call's partials, which
must not leak into the second), and a request above the 32 MiB scratch is
refused before any launch."""

from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 32 << 20


def _case(rng, kind, m, n, k):
    from hackathon_amd import _lib
    from hackathon_amd.c35 import engine as E
    from hackathon_amd.device import BF16, DeviceArray, f32_to_bf16

    def st(x):
        if kind == "fp32":
            return x
        return f32_to_bf16(x) if kind == "bf16" else x.astype(np.float16)

    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((n, k)).astype(np.float32)
    res = rng.standard_normal((m, n)).astype(np.float32)
    keep = [DeviceArray.from_host(np.ascontiguousarray(st(a))), DeviceArray.from_host(np.ascontiguousarray(st(b))),
            DeviceArray.from_host(rng.standard_normal(n).astype(np.float32)),
            DeviceArray.from_host(np.ascontiguousarray(st(res)))]
    code = {"fp32": _lib.F32, "bf16": _lib.BF16, "fp16": _lib.F16}[kind]
    odt = {"fp32": np.float32, "bf16": BF16, "fp16": np.float16}[kind]
    g = _lib.GemmArgs()
    g.a, g.b, g.m, g.n, g.k, g.lda, g.ldb, g.ldo, g.batch = keep[0].ptr, keep[1].ptr, m, n, k, k, k, n, 1
    g.trans_a, g.trans_b, g.in_dtype, g.out_dtype = 0, 1, code, code
    g.epi = E.epilogue(bias=keep[2], bias_mode=2, act=1, residual=keep[3], alpha=0.5)
    return g, keep, odt


def _noalloc(g, splits, out):
    from hackathon_amd import _lib

    g.out = out.ptr
    _lib.check(_lib.lib().c3h_gemm_splitk_noalloc(C.byref(g), splits, None), "c3h_gemm_splitk_noalloc")
    return out.get()


def _workspace(g, splits, out):
    from hackathon_amd import _lib
    from hackathon_amd.device import DeviceArray

    ws = DeviceArray.empty((splits * g.m * g.n,), np.float32)
    g.out = out.ptr
    _lib.check(_lib.lib().c3h_gemm_splitk(C.byref(g), splits, ws.ptr, ws.nbytes, None), "c3h_gemm_splitk")
    return out.get()


@pytest.mark.parametrize("kind", ["fp32", "bf16", "fp16"])
def test_gemm_splitk_noalloc_matches_workspace_entry(gpu, kind):
    from hackathon_amd.device import DeviceArray

    rng = np.random.default_rng({"fp32": 1, "bf16": 2, "fp16": 3}[kind])
    # first call: the ResNet-18 224 classifier shape (8.2 MB of partials); second: smaller
    for m, n, k, splits in ((256, 1000, 512, 8), (64, 72, 256, 4)):
        g, keep, odt = _case(rng, kind, m, n, k)
        out_a, out_b = DeviceArray.empty((m, n), odt), DeviceArray.empty((m, n), odt)
        out_a.copy_from_host(np.zeros(out_a.nbytes, np.uint8))
        print(f"noalloc split-K {kind} {m}x{n}x{k} splits={splits}", flush=True)
        got = _noalloc(g, splits, out_a)
        want = _workspace(g, splits, out_b)
        np.testing.assert_array_equal(got.view(np.uint8), want.view(np.uint8))
        assert np.any(got.view(np.uint8) != 0)


def test_gemm_splitk_noalloc_rejects_oversize(gpu):
    from hackathon_amd import _lib
    from hackathon_amd.device import DeviceArray

    rng = np.random.default_rng(4)
    g, keep, odt = _case(rng, "fp32", 1024, 1025, 64)  # 8 splits: 33.6 MB of partials > 32 MiB
    out = DeviceArray.empty((1024, 1025), odt)
    g.out = out.ptr
    assert 8 * 1024 * 1025 * 4 > SCRATCH_BYTES
    rc = _lib.lib().c3h_gemm_splitk_noalloc(C.byref(g), 8, None)
    assert rc != 0 and "static scratch" in _lib.last_error()
    # exactly at the limit is accepted
    g2, keep2, _ = _case(rng, "fp32", 1024, 1024, 64)
    out2 = DeviceArray.empty((1024, 1024), np.float32)
    assert 8 * 1024 * 1024 * 4 == SCRATCH_BYTES
    got = _noalloc(g2, 8, out2)
    want = _workspace(g2, 8, DeviceArray.empty((1024, 1024), np.float32))
    np.testing.assert_array_equal(got, want)
